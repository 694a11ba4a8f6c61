"""kf_gemv_no_alloc against kf_gemv through the C-ABI, on the GPU.

The no-allocation entry point runs the same kernels as kf_gemv with its
split-K workspace in a static device array, so its output must equal
kf_gemv's bit for bit (the cross-slice reduction has a fixed order). Two calls
in a row share that array; the second is smaller, so it runs on counters and
partials the first one left behind. Each result is also gated against the CPU
oracle at the bf16/fp16 thresholds (2e-2 / 5e-3, kernelforge/testing.py:31-35).
"""

from __future__ import annotations

import pytest
import torch

from kernelforge.dtypes import abi_code
from kernelforge.runtime import hip
from kernelforge.testing import verify
from oracle import ops

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _operands(m, n, k, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    x = (torch.rand(m, k, generator=g) * 2 - 1).to(dtype)
    w = (torch.rand(k, n, generator=g) * 2 - 1).to(dtype)
    bias = (torch.rand(n, generator=g) * 2 - 1).to(dtype)
    return x, w, bias


def _call(entry, x, w, bias, y, split_k, waves, lanes, epilogue, workspace=None):
    lib = hip.load()
    m, k = x.shape
    n = w.shape[1]
    args = [abi_code(x.dtype), x.data_ptr(), w.data_ptr(), bias.data_ptr() if epilogue else None,
            y.data_ptr(), m, n, k, x.stride(0), x.stride(1), w.stride(0), w.stride(1),
            y.stride(0), y.stride(1), epilogue, split_k, waves, lanes]
    if entry == "kf_gemv":
        args += [workspace.data_ptr(), workspace.numel()]
    rc = getattr(lib, entry)(*args, hip.stream_of(x))
    hip.check(rc, entry)


# (m, n, k, dtype, split_k, waves, lanes_per_row, epilogue, W layout); the second
# call of each pair is the smaller one.
PAIRS = [
    ((4, 11008, 4096, torch.bfloat16, 8, 8, 32, 0, "n"),
     (1, 4097, 127, torch.bfloat16, 4, 4, 16, 0, "n")),
    ((1, 11008, 4096, torch.bfloat16, 4, 8, 32, 1, "n"),
     (3, 1000, 301, torch.bfloat16, 3, 4, 16, 1, "n")),
    ((2, 4096, 4096, torch.float16, 6, 8, 16, 0, "k"),
     (1, 7, 8, torch.float16, 2, 1, 8, 0, "k")),
]


@pytest.mark.parametrize("first,second", PAIRS, ids=("bf16-decode", "bf16-gelu", "fp16-kcontig"))
def test_no_alloc_matches_kf_gemv_on_two_calls(first, second):
    for i, (m, n, k, dtype, split, waves, lanes, epi, layout) in enumerate((first, second)):
        print(f"no_alloc call {i}: m={m} n={n} k={k} {dtype} split={split} waves={waves} "
              f"lanes={lanes} epilogue={epi} W={layout}-contiguous", flush=True)
        assert hip.load().kf_gemv_workspace_bytes(m, n, split) <= hip.KF_GEMV_NO_ALLOC_SCRATCH_BYTES
        x, w, bias = _operands(m, n, k, dtype, seed=m * 31 + n + k)
        dx, dbias = x.to(DEV), bias.to(DEV)
        dw = w.to(DEV) if layout == "n" else w.t().contiguous().to(DEV).t()
        want = torch.full((m, n), float("nan"), dtype=dtype, device=DEV)
        got = torch.full((m, n), float("nan"), dtype=dtype, device=DEV)
        ws = torch.zeros(max(hip.load().kf_gemv_workspace_bytes(m, n, split), 16),
                         dtype=torch.uint8, device=DEV)
        _call("kf_gemv", dx, dw, dbias, want, split, waves, lanes, epi, workspace=ws)
        _call("kf_gemv_no_alloc", dx, dw, dbias, got, split, waves, lanes, epi)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), \
            f"call {i}: kf_gemv_no_alloc differs from kf_gemv"
        ref = ops.linear_gelu_ref(x, w, bias) if epi else ops.matmul_ref(x, w)
        res = verify(ref, got.cpu(), dtype=dtype)
        assert res.passed, f"call {i}: {res.reason}"


def test_no_alloc_repeats_bitwise_and_refuses_oversized_splits():
    """Ten calls in a row give one result (counters return to zero each time);
    a split beyond the static scratch is refused without launching."""
    m, n, k = 1, 11008, 4096
    x, w, _ = _operands(m, n, k, torch.bfloat16, seed=5)
    dx, dw = x.to(DEV), w.to(DEV)
    outs = []
    for _ in range(10):
        y = torch.empty(m, n, dtype=torch.bfloat16, device=DEV)
        _call("kf_gemv_no_alloc", dx, dw, dx, y, 4, 8, 32, 0)
        outs.append(y)
    torch.cuda.synchronize()
    assert all(torch.equal(o, outs[0]) for o in outs[1:])
    lib = hip.load()
    too_many = (hip.KF_GEMV_NO_ALLOC_SCRATCH_BYTES // (8 * n * 4)) + 1
    y = torch.empty(8, n, dtype=torch.bfloat16, device=DEV)
    x8 = torch.zeros(8, k, dtype=torch.bfloat16, device=DEV)
    rc = lib.kf_gemv_no_alloc(abi_code(torch.bfloat16), x8.data_ptr(), dw.data_ptr(), None,
                              y.data_ptr(), 8, n, k, k, 1, n, 1, n, 1, 0, too_many, 8, 32,
                              hip.stream_of(x8))
    assert rc == hip.KF_ERR_WORKSPACE and "static scratch" in hip.last_error()
    # More column blocks than a workspace has counters: the scratch would be
    # large enough, so both entry points refuse it the same way, without
    # launching (the pointers are never dereferenced).
    wide = hip.KF_WORKSPACE_COUNTERS + 1
    codes = []
    for entry in ("kf_gemv", "kf_gemv_no_alloc"):
        args = [abi_code(torch.bfloat16), dx.data_ptr(), dw.data_ptr(), None, y.data_ptr(),
                1, wide, k, k, 1, wide, 1, wide, 1, 0, 2, 8, 32]
        if entry == "kf_gemv":
            args += [None, 0]
        codes.append(getattr(lib, entry)(*args, hip.stream_of(dx)))
        assert "counters" in hip.last_error(), (entry, hip.last_error())
    assert codes == [hip.KF_ERR_INVALID_ARGUMENT] * 2
