"""GPU parity for the rows beyond the kernel set: vector_add, the two-pass
RMSNorm, the TransformerBlock dispatch consumer and the benchmark / compare /
report commands end to end.

vector_add is integer-exact work in disguise: the fp32 sum rounded once is
the correctly rounded 16-bit sum, so it is compared bit for bit with the
oracle (itself pinned against exact rational arithmetic). The two-pass RMSNorm
is gated against the same oracle as the single-pass kernel at the
reference's thresholds (fp32 1e-5, fp16 5e-3, bf16 2e-2). The block compares
its two backends on one set of weights (kernelforge/tests/
test_transformer.py:37-83).
"""

from __future__ import annotations

import ctypes
import subprocess
import sys

import pytest
import torch

from kernelforge.benchmark.workloads import VECTOR_SHAPES
from kernelforge.dtypes import abi_code
from kernelforge.runtime import hip
from kernelforge.testing import verify
from kernelforge.tuning.config import KernelConfig, Problem
from kernelforge.tuning.search import TWO_PASS_MAX_STAGED_BYTES, two_pass_block
from oracle import ops

pytestmark = pytest.mark.gpu

DTYPES = (torch.float32, torch.float16, torch.bfloat16)
DEV = "cuda"


def _randn(*shape, dtype, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g, dtype=torch.float32) * scale).to(dtype)


def _bits(t: torch.Tensor) -> torch.Tensor:
    t = t.detach().cpu().contiguous()
    return t.view(torch.int32 if t.element_size() == 4 else torch.int16)


def _gate(ref: torch.Tensor, out: torch.Tensor, dtype: torch.dtype, what: str) -> None:
    res = verify(ref, out.cpu(), dtype=dtype)
    assert res.passed, f"{what}: {res.reason}"


# --- vector_add -------------------------------------------------------------------


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("n", VECTOR_SHAPES["correctness"])
def test_vector_add_is_bit_exact_across_sizes(n, dtype):
    from kernelforge.kernels.vector_add import DEFAULT_CONFIG, vector_add

    a = _randn(n, dtype=dtype, seed=n)
    b = _randn(n, dtype=dtype, seed=n + 1)
    for cfg in (DEFAULT_CONFIG, None):
        out = vector_add(a.to(DEV), b.to(DEV), config=cfg)
        assert torch.equal(_bits(out), _bits(ops.vector_add_ref(a, b))), f"n={n} {cfg}"


def test_vector_add_every_candidate_agrees():
    from kernelforge.kernels.vector_add import vector_add
    from kernelforge.runtime.env import MI355X_CAPS
    from kernelforge.tuning.search import VectorAddSearchSpace

    n = 1_000_003
    a = _randn(n, dtype=torch.float16, seed=5)
    b = _randn(n, dtype=torch.float16, seed=6)
    expected = _bits(ops.vector_add_ref(a, b))
    da, db = a.to(DEV), b.to(DEV)
    problem = Problem.create("vector_add", "fp16", n=n)
    cands = VectorAddSearchSpace().candidates(problem, MI355X_CAPS, max_candidates=100)
    assert len(cands) >= 20
    for cfg in cands:
        assert torch.equal(_bits(vector_add(da, db, config=cfg)), expected), str(cfg)


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
def test_vector_add_unaligned_and_strided_operands(dtype):
    """Views that start off a 16-byte boundary take the element path; a
    strided view is made contiguous by the wrapper, as in the reference."""
    from kernelforge.kernels.vector_add import vector_add

    n = 70_001
    big_a = _randn(n + 3, dtype=dtype, seed=7)
    big_b = _randn(2 * n, dtype=dtype, seed=8)
    a, b = big_a[3:], big_b[::2]
    da, db = big_a.to(DEV)[3:], big_b.to(DEV)[::2]
    out = vector_add(da, db, config=KernelConfig("vector_add", BLOCK_SIZE=4096, num_warps=4))
    assert torch.equal(_bits(out), _bits(ops.vector_add_ref(a, b)))


def test_vector_add_writes_nothing_past_n():
    """The C-ABI with the output inside a NaN-filled guard buffer."""
    lib = hip.load()
    n, pad = 12_345, 4096
    a = _randn(n, dtype=torch.float32, seed=9).to(DEV)
    b = _randn(n, dtype=torch.float32, seed=10).to(DEV)
    guard = torch.full((n + 2 * pad,), float("nan"), device=DEV)
    out = guard[pad:pad + n]
    rc = lib.kf_vector_add(abi_code(torch.float32), a.data_ptr(), b.data_ptr(), out.data_ptr(), n,
                           8192, 2, hip.stream_of(a))
    hip.check(rc, "vector_add")
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), ops.vector_add_ref(a.cpu(), b.cpu()))
    assert guard[:pad].isnan().all() and guard[pad + n:].isnan().all()


def test_vector_add_validates_device_inputs():
    from kernelforge.kernels.vector_add import vector_add

    a = torch.zeros(8, device=DEV, dtype=torch.float16)
    with pytest.raises(ValueError, match="shape mismatch"):
        vector_add(a, torch.zeros(9, device=DEV, dtype=torch.float16))
    with pytest.raises(ValueError, match="dtype mismatch"):
        vector_add(a, torch.zeros(8, device=DEV, dtype=torch.float32))
    assert vector_add(a[:0], a[:0]).numel() == 0


# --- two-pass RMSNorm ----------------------------------------------------------------

WIDE_SHAPES = [(3, 16385), (5, 40000), (2, 65536), (4, 100003), (7, 1), (3, 127), (64, 4096)]


@pytest.mark.parametrize("dtype", DTYPES, ids=lambda d: str(d).split(".")[-1])
@pytest.mark.parametrize("rows,cols", WIDE_SHAPES)
def test_two_pass_rmsnorm_default_and_both_stagings(rows, cols, dtype):
    from kernelforge.kernels.rmsnorm import rmsnorm

    x = _randn(rows, cols, dtype=dtype, seed=rows * 13 + cols, scale=2.0)
    g = (_randn(cols, dtype=torch.float32, seed=cols) * 0.1 + 1.0).to(dtype)
    ref = ops.rmsnorm_ref(x, g, 1e-6)
    dx, dg = x.to(DEV), g.to(DEV)
    if cols > 16384:
        _gate(ref, rmsnorm(dx, dg, eps=1e-6), dtype, f"default {rows}x{cols}")
    elem = x.element_size()
    for stage in (0, 1):
        if stage and cols * elem > TWO_PASS_MAX_STAGED_BYTES:
            continue
        cfg = KernelConfig("rmsnorm", TWO_PASS=1, BLOCK_SIZE=two_pass_block(8, 2, elem),
                           ROWS_PER_PROGRAM=2, STAGE_ROW=stage, num_warps=8)
        _gate(ref, rmsnorm(dx, dg, eps=1e-6, config=cfg), dtype, f"{rows}x{cols} {cfg}")


@pytest.mark.parametrize("warps,unroll", [(4, 1), (4, 8), (8, 4), (16, 1), (16, 4), (8, 8)])
@pytest.mark.parametrize("rpp", (1, 3))
@pytest.mark.parametrize("stage", (0, 1))
def test_two_pass_rmsnorm_trip_shapes(warps, unroll, rpp, stage):
    """Every unroll and wave count, rows-per-program tails, staged or not."""
    from kernelforge.kernels.rmsnorm import rmsnorm

    rows, cols = 37, 20000
    x = _randn(rows, cols, dtype=torch.float16, seed=21)
    g = (_randn(cols, dtype=torch.float32, seed=22) * 0.1 + 1.0).to(torch.float16)
    cfg = KernelConfig("rmsnorm", TWO_PASS=1, BLOCK_SIZE=two_pass_block(warps, unroll, 2),
                       ROWS_PER_PROGRAM=rpp, STAGE_ROW=stage, num_warps=warps)
    out = rmsnorm(x.to(DEV), g.to(DEV), config=cfg)
    _gate(ops.rmsnorm_ref(x, g), out, torch.float16, str(cfg))


def test_two_pass_rmsnorm_every_candidate_agrees():
    from kernelforge.kernels.rmsnorm import rmsnorm
    from kernelforge.runtime.env import MI355X_CAPS
    from kernelforge.tuning.search import RMSNormSearchSpace

    rows, cols = 64, 24000
    x = _randn(rows, cols, dtype=torch.bfloat16, seed=23)
    g = (_randn(cols, dtype=torch.float32, seed=24) * 0.1 + 1.0).to(torch.bfloat16)
    ref = ops.rmsnorm_ref(x, g)
    dx, dg = x.to(DEV), g.to(DEV)
    problem = Problem.create("rmsnorm", "bf16", rows=rows, cols=cols)
    cands = RMSNormSearchSpace().candidates(problem, MI355X_CAPS, max_candidates=200)
    assert cands and all(c["TWO_PASS"] for c in cands)
    for cfg in cands:
        _gate(ref, rmsnorm(dx, dg, config=cfg), torch.bfloat16, str(cfg))


@pytest.mark.parametrize("stage", (0, 1))
def test_two_pass_rmsnorm_unaligned_strided_rows_and_guard_band(stage):
    """Rows that start off a 16-byte boundary (element path) inside a wider
    buffer, written into a NaN guard buffer through the C-ABI."""
    lib = hip.load()
    rows, cols, pitch = 6, 17003, 17011
    base = _randn(rows, pitch, dtype=torch.float32, seed=25)
    x = base[:, 1:1 + cols]  # row stride 17011, base 4 bytes past alignment
    g = (_randn(cols, dtype=torch.float32, seed=26) * 0.1 + 1.0)
    dbase, dg = base.to(DEV), g.to(DEV)
    dx = dbase[:, 1:1 + cols]
    guard = torch.full((rows + 2, pitch), float("nan"), device=DEV)
    y = guard[1:1 + rows, 3:3 + cols]
    rc = lib.kf_rmsnorm_two_pass(
        abi_code(torch.float32), dx.data_ptr(), dg.data_ptr(), y.data_ptr(), rows, cols,
        dx.stride(0), y.stride(0), ctypes.c_float(1e-5), two_pass_block(8, 4, 4), 1, 8, stage,
        hip.stream_of(dx),
    )
    hip.check(rc, "rmsnorm_two_pass")
    torch.cuda.synchronize()
    _gate(ops.rmsnorm_ref(x, g, 1e-5), y, torch.float32, f"unaligned stage={stage}")
    host = guard.cpu()
    assert host[0].isnan().all() and host[-1].isnan().all()
    assert host[1:-1, :3].isnan().all() and host[1:-1, 3 + cols:].isnan().all()


def test_two_pass_rmsnorm_matches_single_pass_where_both_fit():
    from kernelforge.kernels.rmsnorm import default_config, rmsnorm

    x = _randn(256, 8192, dtype=torch.float32, seed=27).to(DEV)
    g = (_randn(8192, dtype=torch.float32, seed=28) * 0.1 + 1.0).to(DEV)
    single = rmsnorm(x, g, config=default_config(8192))
    cfg = KernelConfig("rmsnorm", TWO_PASS=1, BLOCK_SIZE=8192, ROWS_PER_PROGRAM=1, STAGE_ROW=1,
                       num_warps=8)
    double = rmsnorm(x, g, config=cfg)
    assert verify(single.cpu().double(), double.cpu(), dtype=torch.float32).passed


def test_two_pass_rmsnorm_zero_row_and_zero_size():
    from kernelforge.kernels.rmsnorm import rmsnorm

    x = torch.zeros(3, 30000, dtype=torch.float16, device=DEV)
    g = torch.ones(30000, dtype=torch.float16, device=DEV)
    out = rmsnorm(x, g)
    assert torch.isfinite(out).all() and (out == 0).all()
    assert rmsnorm(x[:0], g).shape == (0, 30000)


def test_wide_row_full_size_is_deterministic_and_normalised():
    """A 4096 x 32768 fp16 row set (the bench shape), too big for a quick CPU
    oracle run over every row: two runs are bitwise equal, every row's
    mean square after dividing out gamma is 1, and a sample of rows passes
    the gate against the oracle."""
    from kernelforge.kernels.rmsnorm import rmsnorm

    rows, cols = 4096, 32768
    x = _randn(rows, cols, dtype=torch.float16, seed=29).to(DEV)
    g = (_randn(cols, dtype=torch.float32, seed=30) * 0.1 + 1.0).to(torch.float16).to(DEV)
    a = rmsnorm(x, g, eps=1e-6)
    b = rmsnorm(x, g, eps=1e-6)
    assert torch.equal(a, b)
    ms = (a.float() / g.float()).pow(2).mean(dim=1)
    assert torch.allclose(ms, torch.ones_like(ms), atol=2e-2)
    sample = torch.arange(0, rows, 97)
    _gate(ops.rmsnorm_ref(x[sample].cpu(), g.cpu(), 1e-6), a[sample], torch.float16, "sample")


# --- TransformerBlock -----------------------------------------------------------------


def _block(seed=0):
    from kernelforge.integration.transformer import BlockConfig, TransformerBlock

    torch.manual_seed(seed)
    block = TransformerBlock(BlockConfig(hidden=256, heads=8, intermediate=512), device=DEV,
                             dtype=torch.float16)
    with torch.no_grad():
        for p in block.parameters():
            p.copy_((torch.randn(p.shape, generator=torch.Generator().manual_seed(seed)) * 0.02)
                    .to(p.dtype))
            seed += 1
    return block


@pytest.mark.parametrize("batch,seq", [(2, 128), (1, 1), (1, 7), (3, 5)])
def test_block_backends_agree_on_one_set_of_weights(batch, seq):
    from kernelforge.integration.transformer import BACKEND_KERNELFORGE, BACKEND_TORCH

    block = _block()
    x = _randn(batch, seq, 256, dtype=torch.float16, seed=31).to(DEV)
    with torch.inference_mode():
        block.backend = BACKEND_TORCH
        expected = block(x)
        block.backend = BACKEND_KERNELFORGE
        actual = block(x)
    res = verify(expected.float().cpu(), actual.cpu(), dtype=torch.float16)
    assert res.passed, f"batch={batch} seq={seq}: {res.reason}"


def test_block_resolves_configurations_once_per_shape():
    from kernelforge.integration.transformer import BACKEND_KERNELFORGE

    block = _block()
    block.backend = BACKEND_KERNELFORGE
    x = _randn(1, 64, 256, dtype=torch.float16, seed=32).to(DEV)
    with torch.inference_mode():
        block(x)
        chosen = block._paths["kernelforge"].chosen
        resolved = dict(chosen)
        block(x)
    assert chosen == resolved
    assert {op for op, _, _ in resolved} == {"rmsnorm", "fused_linear"}


def test_block_validates_its_input():
    block = _block()
    with pytest.raises(ValueError, match=r"\(batch, seq, hidden\)"):
        block(torch.zeros(4, 256, device=DEV, dtype=torch.float16))
    with pytest.raises(ValueError, match="expected hidden"):
        block(torch.zeros(1, 4, 512, device=DEV, dtype=torch.float16))


def test_benchmark_block_times_both_backends():
    from kernelforge.integration.transformer import BACKENDS, BlockConfig, benchmark_block

    results = benchmark_block(BlockConfig(hidden=256, heads=8, intermediate=512), batch=1, seq=128,
                              device=DEV, warmup=2, iterations=5)
    assert set(results) == set(BACKENDS)
    for timing in results.values():
        assert timing.median_ms > 0 and timing.timer == "hip_event"


# --- CLI end to end ---------------------------------------------------------------------


def _cli(*argv, timeout=240):
    return subprocess.run([sys.executable, "-m", "kernelforge", *argv], capture_output=True,
                          text=True, timeout=timeout)


def test_cli_benchmark_then_report(tmp_path):
    db, out = tmp_path / "r.db", tmp_path / "report"
    for op in ("vector_add", "rmsnorm"):
        run = _cli("benchmark", op, "--suite", "smoke", "--dtype", "fp16", "--db", str(db),
                   "--no-cache", "--warmup", "3", "--iterations", "10")
        assert run.returncode == 0, run.stdout + run.stderr
        assert "kernelforge" in run.stdout and "GB/s" in run.stdout
    rep = _cli("report", "--db", str(db), "--out", str(out))
    assert rep.returncode == 0, rep.stderr
    text = (out / "summary.md").read_text()
    assert "## vector_add" in text and "## rmsnorm" in text and "of MI355X peak" in text
    assert {"vector_add.csv", "rmsnorm.csv"} <= {p.name for p in out.iterdir()}


def test_cli_compare_one_shape_and_a_block(tmp_path):
    run = _cli("compare", "rmsnorm", "--rows", "64", "--cols", "20000", "--dtype", "fp32",
               "--no-cache", "--warmup", "2", "--iterations", "5")
    assert run.returncode == 0, run.stdout + run.stderr
    assert "kernelforge" in run.stdout and "torch_eager" in run.stdout
    run = _cli("compare", "transformer", "--hidden", "256", "--heads", "8", "--intermediate", "512",
               "--seq", "64", "--no-cache", "--warmup", "2", "--iterations", "5")
    assert run.returncode == 0, run.stdout + run.stderr
    assert "Block latency" in run.stdout and "kernelforge" in run.stdout
