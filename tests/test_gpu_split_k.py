"""GPU parity of the split-K GEMM (kf_gemm_split_k) and of shared split-K workspaces.

Each output is written into a NaN-filled buffer with a NaN guard band around
it, so a tile that no program finished (a lost ticket) shows as NaN instead of
passing on memory left over from an earlier call, and a write outside C shows
in the guard. Results are gated against the CPU oracle with the reference's
per-dtype thresholds (kernelforge/testing.py:31-35). The workspace comes from
the same per-stream pool the kernels use, so consecutive cases share it, as
calls in a program do.
"""

from __future__ import annotations

import pytest
import torch

from kernelforge.dtypes import abi_code
from kernelforge.runtime import hip
from kernelforge.testing import verify
from kernelforge.tuning.config import KernelConfig
from oracle import ops

pytestmark = pytest.mark.gpu

DEV = "cuda"
PAD = 4


def _randn(*shape, dtype, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g, dtype=torch.float32) * scale).to(dtype)


def _gate(ref, out, dtype, what):
    res = verify(ref, out.cpu(), dtype=dtype)
    assert res.passed, f"{what}: {res.reason}"


def _split_call(da, db, bias, bm, bn, waves, split, *, stages=3, out_dtype=None):
    """kf_gemm_split_k into a NaN buffer with a guard band; returns (C, guard intact)."""
    m, k = da.shape
    n = db.shape[1]
    dtype = out_dtype or da.dtype
    pitch = n + 2 * PAD + 8  # 16-byte multiple for every 16-bit n % 8 == 0
    buf = torch.full(((m + 2 * PAD) * pitch,), float("nan"), dtype=dtype, device=DEV)
    cptr = buf.data_ptr() + (PAD * pitch + PAD) * buf.element_size()
    lib = hip.load()
    stream = hip.stream_of(da)
    need = lib.kf_gemm_workspace_bytes(m, n, bm, bn, split)
    ws = hip.workspaces.get(da.device, stream, need) if need else None
    epi = hip.KF_EPILOGUE_BIAS_GELU if bias is not None else hip.KF_EPILOGUE_NONE
    rc = lib.kf_gemm_split_k(
        abi_code(dtype), da.data_ptr(), db.data_ptr(), bias.data_ptr() if bias is not None else None,
        cptr, m, n, k, da.stride(0), da.stride(1), db.stride(0), db.stride(1), pitch, 1, epi,
        bm, bn, 64, waves, stages, 8, split, ws.data_ptr() if ws is not None else None,
        ws.numel() if ws is not None else 0, stream,
    )
    hip.check(rc, "split-K gemm")
    torch.cuda.synchronize()
    host = buf.cpu().view(m + 2 * PAD, pitch).float()
    inside = host[PAD : PAD + m, PAD : PAD + n]
    guard = torch.ones_like(host, dtype=torch.bool)
    guard[PAD : PAD + m, PAD : PAD + n] = False
    return inside, bool(torch.isnan(host[guard]).all())


# (BLOCK_M, BLOCK_N, waves[, stages]); the 256x256 tile (32x32x16 fragments,
# four 16-byte parts per fragment in a partial tile) has two stages only.
_TILES = [(32, 64, 4), (64, 64, 4), (32, 128, 4), (64, 128, 8), (128, 128, 8), (256, 128, 8),
          (256, 256, 8, 2)]


@pytest.mark.parametrize("tile", _TILES, ids=lambda t: "x".join(map(str, t)))
@pytest.mark.parametrize("split", (2, 3, 4, 8, 16))
@pytest.mark.parametrize(
    "m,n,k",
    [(32, 4096, 4096), (33, 1000, 1032), (64, 520, 4104), (100, 264, 200), (7, 64, 128)],
)
def test_split_k_matches_the_oracle(tile, split, m, n, k):
    """Shapes with M/N edges, K tails (K % 64 != 0), programs whose k-range is
    short or empty (K=128 at split 3..16 leaves programs with no slice), and
    split counts that do not divide the slice count."""
    bm, bn, w = tile[:3]
    stages = tile[3] if len(tile) > 3 else 3
    a = _randn(m, k, dtype=torch.float16, seed=m + k)
    b = _randn(k, n, dtype=torch.float16, seed=n + split, scale=k**-0.5)
    out, guard = _split_call(a.to(DEV), b.to(DEV), None, bm, bn, w, split, stages=stages)
    assert guard, "split-K wrote outside C"
    assert torch.isfinite(out).all(), "a tile was never finished"
    _gate(ops.matmul_ref(a, b), out, torch.float16, f"{tile} split {split} {m}x{n}x{k}")


@pytest.mark.parametrize("layout", ("nn", "nt"))
@pytest.mark.parametrize("dtype", (torch.float16, torch.bfloat16), ids=("fp16", "bf16"))
@pytest.mark.parametrize("stages", (2, 3))
def test_split_k_layouts_dtypes_and_stages(layout, dtype, stages):
    m, n, k = 48, 1032, 2056
    a = _randn(m, k, dtype=dtype, seed=1)
    b = _randn(k, n, dtype=dtype, seed=2, scale=k**-0.5)
    db = b.to(DEV) if layout == "nn" else b.t().contiguous().to(DEV).t()
    out, guard = _split_call(a.to(DEV), db, None, 64, 64, 4, 4, stages=stages)
    assert guard and torch.isfinite(out).all()
    _gate(ops.matmul_ref(a, b), out, dtype, f"{layout} {dtype} S{stages}")


@pytest.mark.parametrize("split", (2, 4, 8))
def test_split_k_fused_epilogue_runs_once_on_the_sum(split):
    """bias + GELU apply to the reduced tile, not to each partial."""
    m, n, k = 32, 1024, 4096
    x = _randn(m, k, dtype=torch.float16, seed=3)
    w = _randn(k, n, dtype=torch.float16, seed=4, scale=k**-0.5)
    bias = _randn(n, dtype=torch.float16, seed=5)
    out, guard = _split_call(x.to(DEV), w.to(DEV), bias.to(DEV), 32, 64, 4, split)
    assert guard and torch.isfinite(out).all()
    _gate(ops.linear_gelu_ref(x, w, bias), out, torch.float16, f"fused split {split}")


def test_split_k_is_deterministic():
    """The last program adds the partials in ascending order whoever it is."""
    a = _randn(32, 4096, dtype=torch.float16, seed=6).to(DEV)
    b = _randn(4096, 4096, dtype=torch.float16, seed=7, scale=1 / 64).to(DEV)
    first, _ = _split_call(a, b, None, 32, 64, 4, 8)
    for _ in range(4):
        again, _ = _split_call(a, b, None, 32, 64, 4, 8)
        assert torch.equal(first, again)


def test_shared_workspace_serves_any_sequence_of_calls():
    """Split-K GEMMs and GEMVs of different block counts through one workspace.

    Every entry point keeps its arrival counters in the same fixed region, so
    partial sums written by one call never sit where a later call, with more
    blocks, expects a zero counter. The sequence grows the counter count after
    a call with large partials, the order that exposes an overlap."""
    from kernelforge.kernels.matmul import launch_gemm

    cases = [
        # (m, n, k, config)
        (64, 4096, 4096, KernelConfig("matmul", BLOCK_M=32, BLOCK_N=64, BLOCK_K=64, GROUP_M=8,
                                      DIRECT=1, SPLIT_K=16, num_warps=4, num_stages=3)),
        (1, 11008, 4096, KernelConfig("matmul", GEMV=1, SPLIT_K=4, LANES_PER_ROW=16, num_warps=4)),
        (32, 11008, 4096, KernelConfig("matmul", BLOCK_M=32, BLOCK_N=64, BLOCK_K=64, GROUP_M=8,
                                       DIRECT=1, SPLIT_K=4, num_warps=4, num_stages=3)),
        (4, 4096, 11008, KernelConfig("matmul", GEMV=1, SPLIT_K=8, LANES_PER_ROW=32, num_warps=8)),
        (128, 4096, 4096, KernelConfig("matmul", BLOCK_M=64, BLOCK_N=128, BLOCK_K=64, GROUP_M=8,
                                       DIRECT=1, SPLIT_K=4, num_warps=8, num_stages=3)),
        (32, 4096, 4096, KernelConfig("matmul", BLOCK_M=32, BLOCK_N=64, BLOCK_K=64, GROUP_M=8,
                                      DIRECT=1, SPLIT_K=2, num_warps=4, num_stages=3)),
    ]
    for rnd in range(2):
        for i, (m, n, k, cfg) in enumerate(cases):
            a = _randn(m, k, dtype=torch.float16, seed=10 * i + rnd)
            b = _randn(k, n, dtype=torch.float16, seed=10 * i + 5, scale=k**-0.5)
            out = torch.full((m, n), float("nan"), dtype=torch.float16, device=DEV)
            launch_gemm(a.to(DEV), b.to(DEV), None, out, cfg)
            torch.cuda.synchronize()
            assert torch.isfinite(out).all(), f"case {i} round {rnd}: unfinished output"
            _gate(ops.matmul_ref(a, b), out, torch.float16, f"case {i} round {rnd} {cfg}")


@pytest.mark.parametrize("split", (2, 3, 4))
@pytest.mark.parametrize("fused", (False, True))
def test_split_k_of_the_last_partial_round(split, fused):
    """260 tiles of 256x128 (one workgroup per CU): 256 run unsplit, the 4 of
    the last round split; every tile is finished exactly once."""
    m, n, k = 1024, 8320, 1032
    x = _randn(m, k, dtype=torch.float16, seed=20 + split)
    w = _randn(k, n, dtype=torch.float16, seed=21, scale=k**-0.5)
    bias = _randn(n, dtype=torch.float16, seed=22) if fused else None
    out, guard = _split_call(x.to(DEV), w.to(DEV), bias.to(DEV) if fused else None, 256, 128, 8,
                             split)
    assert guard and torch.isfinite(out).all()
    ref = ops.linear_gelu_ref(x, w, bias) if fused else ops.matmul_ref(x, w)
    _gate(ref, out, torch.float16, f"tail split {split} fused={fused}")


@pytest.mark.parametrize("split", (3, 4, 8))
def test_last_round_shared_out_in_ranges_that_cross_tiles(split):
    """344 tiles of 256x128: 256 unsplit, the last 88 shared out over one
    round of 256 programs, 88*16/256 = 5.5 k-slices each, so most ranges end
    inside one tile and go on in the next."""
    m, n, k = 1024, 11008, 1024
    x = _randn(m, k, dtype=torch.float16, seed=40 + split)
    w = _randn(k, n, dtype=torch.float16, seed=41, scale=k**-0.5)
    bias = _randn(n, dtype=torch.float16, seed=42)
    out, guard = _split_call(x.to(DEV), w.to(DEV), bias.to(DEV), 256, 128, 8, split)
    assert guard and torch.isfinite(out).all()
    _gate(ops.linear_gelu_ref(x, w, bias), out, torch.float16, f"stream-K tail split {split}")
    again, _ = _split_call(x.to(DEV), w.to(DEV), bias.to(DEV), 256, 128, 8, split)
    assert torch.equal(out, again)


def test_concurrent_tiles_on_mi355x():
    """One 256x128 DMA workgroup per CU (147 KiB of LDS); 32x64 tiles up to
    four per CU (36 KiB of LDS each; registers may allow fewer)."""
    lib = hip.load()
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    assert lib.kf_gemm_concurrent_tiles(1, 256, 128, 64, 8, 3, 1) == cus
    small = lib.kf_gemm_concurrent_tiles(1, 32, 64, 64, 4, 3, 1)
    assert small % cus == 0 and 1 <= small // cus <= 4


def test_split_k_with_only_full_rounds_runs_unsplit():
    """256 tiles of 256x128 fill exactly one round: nothing is split, so the
    result is bitwise the unsplit kernel's."""
    from kernelforge.kernels.matmul import matmul

    a = _randn(2048, 1024, dtype=torch.float16, seed=30).to(DEV)
    b = _randn(1024, 4096, dtype=torch.float16, seed=31, scale=1 / 32).to(DEV)
    split, _ = _split_call(a, b, None, 256, 128, 8, 4)
    plain = matmul(a, b, config=KernelConfig("matmul", BLOCK_M=256, BLOCK_N=128, BLOCK_K=64,
                                             GROUP_M=8, DIRECT=1, num_warps=8, num_stages=3))
    assert torch.equal(split.to(torch.float16), plain.cpu())


def test_split_k_on_a_layout_the_dma_cannot_take_runs_unsplit():
    """Strided A sends the tile to the register-staged fallback, which ignores
    split_k; the result is still whole and correct."""
    m, n, k = 32, 512, 1024
    a = _randn(m, k, dtype=torch.float16, seed=8)
    b = _randn(k, n, dtype=torch.float16, seed=9, scale=k**-0.5)
    da = a.t().contiguous().to(DEV).t()  # lda_k != 1
    out, guard = _split_call(da, b.to(DEV), None, 64, 64, 4, 4)
    assert guard and torch.isfinite(out).all()
    _gate(ops.matmul_ref(a, b), out, torch.float16, "strided A")


def test_split_k_through_the_operator_and_a_graph():
    """matmul() with a SPLIT_K config, eager and as HIP graph replays (the
    kernel returns its counters to zero, so replays need no memset node)."""
    from kernelforge.kernels.fused_linear import fused_linear_gelu
    from kernelforge.kernels.matmul import matmul

    cfg = KernelConfig("matmul", BLOCK_M=32, BLOCK_N=64, BLOCK_K=64, GROUP_M=8, DIRECT=1,
                       SPLIT_K=4, num_warps=4, num_stages=3)
    fcfg = KernelConfig("fused_linear", BLOCK_M=64, BLOCK_N=128, BLOCK_K=64, GROUP_M=8, DIRECT=1,
                        SPLIT_K=8, num_warps=8, num_stages=3)
    a = _randn(32, 4096, dtype=torch.float16, seed=11).to(DEV)
    b = _randn(4096, 2048, dtype=torch.float16, seed=12, scale=1 / 64).to(DEV)
    bias = _randn(2048, dtype=torch.float16, seed=13).to(DEV)

    def run():
        return [matmul(a, b, config=cfg), fused_linear_gelu(a, b, bias, config=fcfg)]

    eager = run()
    torch.cuda.synchronize()
    _gate(ops.matmul_ref(a.cpu(), b.cpu()), eager[0], torch.float16, "matmul split")
    _gate(ops.linear_gelu_ref(a.cpu(), b.cpu(), bias.cpu()), eager[1], torch.float16, "fused split")
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = run()
    for _ in range(3):
        for t in captured:
            t.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        for got, want in zip(captured, eager):
            assert torch.equal(got, want)
        _ = run()
        torch.cuda.synchronize()


def test_split_k_workspaces_of_captured_graphs_stay_private():
    """Graphs keep the split-K workspace they were captured with.

    Graph A captures a small split-K GEMV; graph B, captured later, a split-K
    GEMM that needs a larger workspace. Eager calls that need a larger eager
    workspace still run in between. Every replay of A and of B must equal the
    eager result bit for bit: a graph replaying on a workspace that was freed
    and handed to someone else, or whose counters another graph left non-zero,
    would not."""
    from kernelforge.kernels.matmul import launch_gemm

    gemv_cfg = KernelConfig("matmul", GEMV=1, SPLIT_K=4, LANES_PER_ROW=16, num_warps=4)
    gemm_cfg = KernelConfig("matmul", BLOCK_M=32, BLOCK_N=64, BLOCK_K=64, GROUP_M=8, DIRECT=1,
                            SPLIT_K=8, num_warps=4, num_stages=3)
    xa = _randn(1, 4096, dtype=torch.float16, seed=41).to(DEV)
    wa = _randn(4096, 4096, dtype=torch.float16, seed=42, scale=1 / 64).to(DEV)
    xb = _randn(64, 4096, dtype=torch.float16, seed=43).to(DEV)
    wb = _randn(4096, 11008, dtype=torch.float16, seed=44, scale=1 / 64).to(DEV)

    def run_a():
        out = torch.empty(1, 4096, dtype=torch.float16, device=DEV)
        launch_gemm(xa, wa, None, out, gemv_cfg)
        return out

    def run_b():
        out = torch.empty(64, 11008, dtype=torch.float16, device=DEV)
        launch_gemm(xb, wb, None, out, gemm_cfg)
        return out

    want_a, want_b = run_a(), run_b()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm up outside the capture, as torch.cuda.graph asks
        run_a()
        run_b()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph_a, graph_b = torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph_a):
        out_a = run_a()
    with torch.cuda.graph(graph_b):
        out_b = run_b()
    torch.cuda.synchronize()
    for rnd in range(3):
        graph_a.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_a, want_a), f"replay {rnd} of graph A"
        # An eager call that needs more workspace than any before it.
        big = torch.empty(128, 11008, dtype=torch.float16, device=DEV)
        launch_gemm(_randn(128, 4096, dtype=torch.float16, seed=45).to(DEV), wb, None, big,
                    KernelConfig("matmul", BLOCK_M=32, BLOCK_N=64, BLOCK_K=64, GROUP_M=8,
                                 DIRECT=1, SPLIT_K=16, num_warps=4, num_stages=3))
        graph_b.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_b, want_b), f"replay {rnd} of graph B"
        assert torch.equal(run_a(), want_a) and torch.equal(run_b(), want_b)
