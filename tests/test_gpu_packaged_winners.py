"""Every configuration in the packaged MI355X winner cache, at its own shape.

``kernelforge/tuned/mi355x_gfx950.json`` is what an entry point runs when it
is called without a configuration on a shape that ships a winner. Each entry
is run here with its configuration at its shape, on seeded inputs, and gated
against a torch fp32 reference on the same device at the reference's
per-dtype thresholds (fp32 1e-5, fp16 5e-3, bf16 2e-2;
kernelforge/testing.py:31-35); vector_add must match exactly. GEMM references
run with TF32 off. ``+bt`` shapes pass B as an ``nn.Linear`` weight,
``weight.t()``.
"""

from __future__ import annotations

import json
from pathlib import Path

import pytest
import torch

from kernelforge.testing import exact_fp32_matmul, verify
from kernelforge.tuning.config import KernelConfig

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda")
CACHE = Path(__file__).resolve().parents[1] / "kernelforge" / "tuned" / "mi355x_gfx950.json"
DTYPES = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}


def _entries():
    entries = json.loads(CACHE.read_text())["entries"]["AMD_Instinct_MI355X_gfx950"]
    return [(op, dt, shape, entry["config"])
            for op, by_dtype in sorted(entries.items())
            for dt, by_shape in sorted(by_dtype.items())
            for shape, entry in sorted(by_shape.items())]


def _randn(*shape, seed, scale=1.0):
    g = torch.Generator(device=DEV).manual_seed(seed)
    return torch.randn(*shape, generator=g, device=DEV).mul_(scale)


@pytest.mark.parametrize("op,dt,shape,cfg", _entries(),
                         ids=[f"{op}-{dt}-{shape}" for op, dt, shape, _ in _entries()])
def test_packaged_winner_passes_the_gate_at_its_shape(op, dt, shape, cfg):
    print(f"{op} {dt} {shape} {cfg}", flush=True)
    dtype = DTYPES[dt]
    config = KernelConfig(op, **cfg)
    key, _, layout = shape.partition("+")
    dims = [int(v) for v in key.split("x")]
    if op in ("matmul", "fused_linear"):
        from kernelforge.kernels.fused_linear import fused_linear_gelu
        from kernelforge.kernels.matmul import matmul

        m, n, k = dims
        a = _randn(m, k, seed=m + 1).to(dtype)
        if layout == "bt":  # an nn.Linear weight (N, K), passed as weight.t()
            b = _randn(n, k, seed=n + 2, scale=k**-0.5).to(dtype).t()
        else:
            b = _randn(k, n, seed=n + 2, scale=k**-0.5).to(dtype)
        with exact_fp32_matmul():
            ref = a.float() @ b.float()
        if op == "matmul":
            out = matmul(a, b, config=config)
        else:
            bias = _randn(n, seed=7).to(dtype)
            ref = torch.nn.functional.gelu(ref + bias.float(), approximate="tanh")
            out = fused_linear_gelu(a, b, bias, config=config)
    elif op == "softmax":
        from kernelforge.kernels.softmax import softmax

        x = _randn(*dims, seed=3, scale=3.0).to(dtype)
        ref = torch.softmax(x.float(), dim=-1)
        out = softmax(x, config=config)
    elif op == "rmsnorm":
        from kernelforge.kernels.rmsnorm import rmsnorm

        x = _randn(*dims, seed=4).to(dtype)
        gamma = (1.0 + _randn(dims[1], seed=5, scale=0.1)).to(dtype)
        xf = x.float()
        ref = xf * torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + 1e-6) * gamma.float()
        out = rmsnorm(x, gamma, eps=1e-6, config=config)
    elif op == "vector_add":
        from kernelforge.kernels.vector_add import vector_add

        x, y = _randn(dims[0], seed=6).to(dtype), _randn(dims[0], seed=8).to(dtype)
        assert torch.equal(vector_add(x, y, config=config), x + y)
        return
    else:
        pytest.fail(f"no reference for {op}")
    res = verify(ref, out, dtype=dtype)
    print(f"  max normalised error {res.error:.3g} (threshold {res.threshold:g})", flush=True)
    assert res.passed, res.reason


# --- the CPU oracle, once per tile family ---------------------------------------------


def _families():
    """One entry per (operation, dtype, B layout, configuration): the shipped
    tile families, each with the first shape that ships it."""
    seen = {}
    for op, dt, shape, cfg in _entries():
        layout = shape.partition("+")[2]
        seen.setdefault((op, dt, layout, json.dumps(cfg, sort_keys=True)), (op, dt, shape, cfg))
    return list(seen.values())


def _small(op, shape, cfg):
    """A small shape on which ``cfg`` still runs its own kernel: ragged against
    the tile where the pipeline allows, 16-byte multiples of N and K kept for
    the direct pipeline, the row width kept for the row kernels."""
    key, _, layout = shape.partition("+")
    dims = [int(v) for v in key.split("x")]
    if op in ("matmul", "fused_linear"):
        m, n, k = dims
        if cfg.get("GEMV"):
            return (m, min(n, 1032), min(k, 520)), layout
        bm, bn = cfg["BLOCK_M"], cfg["BLOCK_N"]
        return (min(m, 2 * bm + 17), min(n, 2 * bn + 24), min(k, 264)), layout
    if op in ("softmax", "rmsnorm"):
        return (min(dims[0], 64), dims[1]), layout
    return (min(dims[0], 100003),), layout


@pytest.mark.parametrize("op,dt,shape,cfg", _families(),
                         ids=[f"{op}-{dt}-{shape}-{i}" for i, (op, dt, shape, _) in enumerate(_families())])
def test_packaged_tile_family_matches_the_cpu_oracle(op, dt, shape, cfg):
    """Every shipped configuration, on a small shape of its operation, against
    oracle/ops.py on the CPU (the restatement of the reference's PyTorch
    references) at the reference's per-dtype thresholds."""
    from oracle import ops

    dtype = DTYPES[dt]
    config = KernelConfig(op, **cfg)
    dims, layout = _small(op, shape, cfg)
    print(f"{op} {dt} {dims}{'+' + layout if layout else ''} {cfg}", flush=True)
    g = torch.Generator().manual_seed(sum(dims) + 11)
    if op in ("matmul", "fused_linear"):
        from kernelforge.kernels.fused_linear import fused_linear_gelu
        from kernelforge.kernels.matmul import matmul

        m, n, k = dims
        a = (torch.rand(m, k, generator=g) * 2 - 1).to(dtype)
        b = ((torch.rand(k, n, generator=g) * 2 - 1) * k**-0.5).to(dtype)
        db = b.t().contiguous().to(DEV).t() if layout == "bt" else b.to(DEV)
        if op == "matmul":
            ref, out = ops.matmul_ref(a, b), matmul(a.to(DEV), db, config=config)
        else:
            bias = ((torch.rand(n, generator=g) * 2 - 1) * 0.5).to(dtype)
            ref = ops.linear_gelu_ref(a, b, bias)
            out = fused_linear_gelu(a.to(DEV), db, bias.to(DEV), config=config)
    elif op == "softmax":
        from kernelforge.kernels.softmax import softmax

        x = (3.0 * torch.randn(*dims, generator=g)).to(dtype)
        ref, out = ops.softmax_ref(x), softmax(x.to(DEV), config=config)
    elif op == "rmsnorm":
        from kernelforge.kernels.rmsnorm import rmsnorm

        x = torch.randn(*dims, generator=g).to(dtype)
        gamma = (1.0 + 0.1 * torch.randn(dims[1], generator=g)).to(dtype)
        ref = ops.rmsnorm_ref(x, gamma, 1e-6)
        out = rmsnorm(x.to(DEV), gamma.to(DEV), eps=1e-6, config=config)
    elif op == "vector_add":
        from kernelforge.kernels.vector_add import vector_add

        x, y = torch.randn(dims[0], generator=g).to(dtype), torch.randn(dims[0], generator=g).to(dtype)
        got = vector_add(x.to(DEV), y.to(DEV), config=config).cpu()
        assert torch.equal(got, ops.vector_add_ref(x, y))  # correctly rounded: bit for bit
        return
    else:
        pytest.fail(f"no oracle for {op}")
    res = verify(ref.float(), out.cpu().float(), dtype=dtype)
    print(f"  max normalised error {res.error:.3g} (threshold {res.threshold:g})", flush=True)
    assert res.passed, res.reason
