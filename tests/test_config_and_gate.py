"""Descriptors (KernelConfig, Problem, dtypes) and the correctness gate.

Mirrors the reference's tests/test_config.py and tests/test_verification.py:
config identity, JSON and digest; problem keys; and closed-form gate cases
(zero error, fp16 rounding passes fp16 but fails fp32, an unwritten column is
caught, NaN/inf, shape mismatch, zero reference, empty, scale invariance).
"""

from __future__ import annotations

import hashlib

import pytest
import torch

from kernelforge.dtypes import abi_code, dtype_name, itemsize, parse_dtype
from kernelforge.testing import (
    ERROR_THRESHOLDS,
    assert_verified,
    exact_fp32_matmul,
    threshold_for,
    verify,
)
from kernelforge.tuning.config import LAUNCH_KEYS, KernelConfig, Problem

# --- KernelConfig ----------------------------------------------------------------


def test_config_is_an_immutable_sorted_mapping():
    cfg = KernelConfig("matmul", num_warps=8, BLOCK_N=128, BLOCK_M=256)
    assert list(cfg) == ["BLOCK_M", "BLOCK_N", "num_warps"]
    assert cfg["BLOCK_M"] == 256 and len(cfg) == 3
    with pytest.raises(TypeError):
        cfg["BLOCK_M"] = 1  # type: ignore[index]


def test_config_rejects_non_int_values():
    with pytest.raises(TypeError):
        KernelConfig("matmul", BLOCK_M=1.5)  # type: ignore[arg-type]
    with pytest.raises(TypeError):
        KernelConfig("matmul", DIRECT=True)  # bool is not an int here


def test_config_equality_hash_and_operation():
    a = KernelConfig("matmul", BLOCK_M=64, BLOCK_N=64)
    b = KernelConfig("matmul", BLOCK_N=64, BLOCK_M=64)
    c = KernelConfig("fused_linear", BLOCK_M=64, BLOCK_N=64)
    assert a == b and hash(a) == hash(b)
    assert a != c


def test_meta_and_launch_split():
    cfg = KernelConfig("matmul", BLOCK_M=64, num_warps=4, num_stages=2)
    assert cfg.meta == {"BLOCK_M": 64}
    assert cfg.launch == {"num_stages": 2, "num_warps": 4}
    assert LAUNCH_KEYS == {"num_warps", "num_stages"}


def test_json_round_trip_and_digest():
    cfg = KernelConfig("softmax", BLOCK_SIZE=4096, ROWS_PER_PROGRAM=1, num_warps=4)
    assert cfg.to_json() == '{"BLOCK_SIZE":4096,"ROWS_PER_PROGRAM":1,"num_warps":4}'
    assert KernelConfig.from_json("softmax", cfg.to_json()) == cfg
    expected = hashlib.sha1(f"softmax|{cfg.to_json()}".encode()).hexdigest()[:16]
    assert cfg.digest == expected and len(cfg.digest) == 16


def test_render_respects_order():
    cfg = KernelConfig("matmul", BLOCK_M=64, BLOCK_N=32, num_warps=4)
    lines = cfg.render(("num_warps", "BLOCK_M")).splitlines()
    assert lines[0].startswith("num_warps:") and lines[1].startswith("BLOCK_M:")


# --- Problem and dtypes -------------------------------------------------------------


def test_problem_keys():
    p = Problem.create("matmul", "fp16", M=2048, N=4096, K=4096)
    assert p.shape_key == "2048x4096x4096"
    assert p.cache_key == "matmul/fp16/2048x4096x4096"
    assert p.dims_dict == {"M": 2048, "N": 4096, "K": 4096}
    assert p["N"] == 4096 and p.itemsize == 2
    assert p.describe() == "matmul M/N/K=2048 x 4096 x 4096 fp16"
    assert p.as_dict()["dtype"] == "fp16"


@pytest.mark.parametrize("bad", [0, -1, 1.0, True])
def test_problem_rejects_bad_dims(bad):
    with pytest.raises(ValueError):
        Problem.create("matmul", "fp16", M=bad, N=1, K=1)


def test_dtype_names_round_trip():
    for name in ("fp16", "bf16", "fp32"):
        assert dtype_name(parse_dtype(name)) == name
    assert parse_dtype("FP16") is torch.float16
    assert itemsize(torch.bfloat16) == 2
    assert [abi_code(d) for d in (torch.float32, torch.float16, torch.bfloat16)] == [0, 1, 2]
    with pytest.raises(ValueError):
        parse_dtype("fp64")
    with pytest.raises(ValueError):
        parse_dtype(torch.float64)
    with pytest.raises(ValueError):
        abi_code(torch.float64)


# --- the gate -------------------------------------------------------------------------


def test_thresholds_are_the_references():
    assert ERROR_THRESHOLDS == {torch.float32: 1e-5, torch.float16: 5e-3, torch.bfloat16: 2e-2}
    assert threshold_for(torch.float16) == 5e-3
    with pytest.raises(ValueError):
        threshold_for(torch.float64)


def test_identical_tensors_pass_with_zero_error():
    x = torch.randn(16, 16)
    res = verify(x, x.clone())
    assert res.passed and res.error == 0.0 and res.mismatched == 0
    assert "ok" in str(res)


def test_fp16_rounding_passes_fp16_but_fails_fp32():
    ref = torch.randn(256, 256, generator=torch.Generator().manual_seed(0))
    rounded = ref.to(torch.float16).to(torch.float32)
    assert verify(ref, rounded, dtype=torch.float16).passed
    assert not verify(ref, rounded, dtype=torch.float32).passed


def test_an_unwritten_column_is_caught():
    ref = torch.randn(64, 64) + 3.0
    out = ref.clone()
    out[:, 17] = 0.0
    res = verify(ref, out, dtype=torch.float16)
    assert not res.passed and res.mismatched == 64
    assert "exceeds" in res.reason


@pytest.mark.parametrize("bad", [float("nan"), float("inf"), float("-inf")])
def test_non_finite_output_fails(bad):
    ref = torch.ones(8)
    out = ref.clone()
    out[3] = bad
    res = verify(ref, out)
    assert not res.passed and res.error == float("inf") and "non-finite" in res.reason


def test_shape_mismatch_fails():
    res = verify(torch.ones(4, 4), torch.ones(4, 5))
    assert not res.passed and "shape mismatch" in res.reason


def test_zero_reference_falls_back_to_absolute_error():
    assert verify(torch.zeros(8), torch.full((8,), 1e-6)).passed
    assert not verify(torch.zeros(8), torch.full((8,), 1.0)).passed


def test_empty_tensors_pass():
    res = verify(torch.empty(0, 4), torch.empty(0, 4))
    assert res.passed and res.total == 0


def test_gate_is_scale_invariant():
    ref = torch.randn(128, generator=torch.Generator().manual_seed(1))
    noise = 1e-3 * torch.randn(128, generator=torch.Generator().manual_seed(2))
    small = verify(ref, ref + noise, dtype=torch.float16)
    big = verify(ref * 1024.0, (ref + noise) * 1024.0, dtype=torch.float16)  # exact rescale
    assert small.error == pytest.approx(big.error, rel=1e-5)


def test_assert_verified_raises_with_context():
    with pytest.raises(AssertionError, match="ctx: normalised error"):
        assert_verified(torch.ones(4), torch.zeros(4), context="ctx")


def test_exact_fp32_matmul_restores_flags():
    before = (torch.backends.cuda.matmul.allow_tf32, torch.get_float32_matmul_precision())
    with exact_fp32_matmul():
        assert torch.backends.cuda.matmul.allow_tf32 is False
        assert torch.get_float32_matmul_precision() == "highest"
    assert (torch.backends.cuda.matmul.allow_tf32, torch.get_float32_matmul_precision()) == before


def test_problem_layout_is_part_of_the_key_only_when_set():
    import pickle

    plain = Problem.create("matmul", "bf16", M=1, N=11008, K=4096)
    bt = Problem.create("matmul", "bf16", layout="bt", M=1, N=11008, K=4096)
    assert plain.cache_key == "matmul/bf16/1x11008x4096"  # the reference's key, unchanged
    assert bt.cache_key == "matmul/bf16/1x11008x4096+bt"
    assert bt != plain and hash(bt) != hash(plain)
    assert pickle.loads(pickle.dumps(bt)) == bt
    assert bt.with_layout("") == plain
    assert "k-contiguous" in bt.describe() and bt.as_dict()["layout"] == "bt"
    with pytest.raises(ValueError, match="layout"):
        Problem.create("matmul", "fp16", layout="tt", M=1, N=2, K=3)
    with pytest.raises(ValueError, match="no operand layouts"):
        Problem.create("rmsnorm", "fp16", layout="bt", rows=1, cols=2)


def test_decode_over_k_contiguous_weights_ranks_the_dot_kernel_shape_first():
    """gemv_dot measured fastest with whole 64-lane columns and no split."""
    from kernelforge.runtime.env import MI355X_CAPS
    from kernelforge.tuning.search import search_space

    bt = Problem.create("matmul", "bf16", layout="bt", M=1, N=11008, K=4096)
    first = search_space("matmul").candidates(bt, MI355X_CAPS, max_candidates=1)[0]
    assert (first["GEMV"], first["LANES_PER_ROW"], first["SPLIT_K"]) == (1, 64, 1)
    plain = bt.with_layout("")
    assert search_space("matmul").candidates(plain, MI355X_CAPS, max_candidates=1)[0] != first


def test_select_config_borrows_row_major_winners_for_tiles_but_not_for_decode(tmp_path):
    from kernelforge.kernels import get_operator
    from kernelforge.runtime.dispatch import SOURCE_CACHE, SOURCE_DEFAULT, select_config
    from kernelforge.tuning.cache import ConfigCache

    cache = ConfigCache(tmp_path / "c.json")
    op = get_operator("fused_linear")
    tile = KernelConfig("fused_linear", BLOCK_M=128, BLOCK_N=128, BLOCK_K=64, GROUP_M=8, DIRECT=1,
                        num_stages=3, num_warps=8)
    gemv = KernelConfig("fused_linear", GEMV=1, LANES_PER_ROW=32, SPLIT_K=4, num_warps=8)
    cache.put(Problem.create("fused_linear", "fp16", M=512, N=11008, K=4096), "cpu", tile)
    cache.put(Problem.create("fused_linear", "fp16", M=1, N=11008, K=4096), "cpu", gemv)
    big = select_config(op, Problem.create("fused_linear", "fp16", layout="bt", M=512, N=11008, K=4096),
                        cache=cache, device="cpu", use_packaged=False)
    assert (big.source, big.config) == (SOURCE_CACHE, tile)
    decode = select_config(op, Problem.create("fused_linear", "fp16", layout="bt", M=1, N=11008, K=4096),
                           cache=cache, device="cpu", use_packaged=False)
    assert decode.source == SOURCE_DEFAULT and decode.config["LANES_PER_ROW"] == 64
