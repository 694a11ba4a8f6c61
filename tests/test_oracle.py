"""Pin the CPU oracle before trusting it as the GPU kernels' checker.

Every oracle function is checked three independent ways:

1. against the committed fp64 golden vectors (tests/golden/make_golden.py,
   textbook formulas evaluated with numpy, not torch);
2. against the oracle module's own fp64 brute-force forms on random small
   shapes, and against closed forms the reference's tests use (constant-row
   softmax = 1/n, all-zero RMSNorm row = 0, zero weight => gelu(bias),
   identity weight => gelu(x));
3. with planted mistakes -- a dropped bias, a dropped GELU cubic term, a
   wrong GELU scale, a transposed operand, softmax without the max shift,
   RMSNorm with a sum instead of a mean or eps outside the root -- each of
   which must fail the same checks, so the checks are known to be sensitive.
"""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import pytest
import torch

from kernelforge.testing import verify
from oracle import ops

GOLDEN = Path(__file__).resolve().parent / "golden" / "kernels_fp64.npz"
_DT = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}


@pytest.fixture(scope="module")
def golden():
    data = np.load(GOLDEN)  # allow_pickle defaults to False
    cases: dict[str, dict[str, np.ndarray]] = {}
    for key in data.files:
        case, field = key.split("/")
        cases.setdefault(case, {})[field] = data[key]
    return cases


def _t(a: np.ndarray, dtype: str) -> torch.Tensor:
    return torch.from_numpy(np.asarray(a, dtype=np.float32)).to(_DT[dtype])


def _check(expected: np.ndarray, out: torch.Tensor, dtype: str):
    return verify(torch.from_numpy(expected), out.double(), dtype=_DT[dtype])


# --- 1. golden vectors ------------------------------------------------------------


def _run_case(name: str, c: dict[str, np.ndarray], impl=ops):
    dtype = str(c["dtype"])
    if name.startswith("matmul"):
        return impl.matmul_ref(_t(c["a"], dtype), _t(c["b"], dtype)), dtype
    if name.startswith(("linear_gelu", "gelu_identity")):
        return impl.linear_gelu_ref(_t(c["x"], dtype), _t(c["w"], dtype), _t(c["bias"], dtype)), dtype
    if name.startswith("softmax"):
        return impl.softmax_ref(_t(c["x"], dtype)), dtype
    if name.startswith("rmsnorm"):
        return impl.rmsnorm_ref(_t(c["x"], dtype), _t(c["gamma"], dtype), float(c["eps"])), dtype
    raise KeyError(name)


def test_golden_file_covers_every_oracle_function(golden):
    prefixes = {name.split("_")[0] for name in golden}
    assert {"matmul", "linear", "gelu", "softmax", "rmsnorm"} <= prefixes


@pytest.mark.parametrize(
    "name",
    [
        "matmul_1x7x3_bf16",
        "matmul_5x9x17_fp16",
        "matmul_4x3x33_fp32",
        "linear_gelu_4x6x5_fp32",
        "linear_gelu_4x6x5_fp16",
        "linear_gelu_4x6x5_bf16",
        "gelu_identity_fp32",
        "softmax_3x127_fp16",
        "softmax_const_2x8_fp32",
        "rmsnorm_3x127_fp32",
        "rmsnorm_2x64_bf16",
    ],
)
def test_oracle_matches_fp64_golden_vectors(golden, name):
    out, dtype = _run_case(name, golden[name])
    res = _check(golden[name]["expected"], out, dtype)
    assert res.passed, f"{name}: {res.reason}"


# --- 2. fp64 brute force and closed forms -------------------------------------------


@pytest.mark.parametrize("m,n,k", [(1, 1, 1), (1, 7, 3), (3, 5, 7), (17, 9, 33)])
@pytest.mark.parametrize("dtype", list(_DT.values()), ids=list(_DT))
def test_matmul_ref_matches_triple_loop(m, n, k, dtype):
    g = torch.Generator().manual_seed(m * 100 + n * 10 + k)
    a = torch.randn(m, k, generator=g).to(dtype)
    b = torch.randn(k, n, generator=g).to(dtype)
    res = verify(torch.from_numpy(ops.matmul_fp64(a, b)), ops.matmul_ref(a, b).double(), dtype=dtype)
    assert res.passed, res.reason


def test_linear_gelu_ref_matches_fp64_definition():
    g = torch.Generator().manual_seed(1)
    x, w, b = torch.randn(6, 9, generator=g), torch.randn(9, 4, generator=g), torch.randn(4, generator=g)
    res = verify(torch.from_numpy(ops.linear_gelu_fp64(x, w, b)), ops.linear_gelu_ref(x, w, b).double(),
                 dtype=torch.float32)
    assert res.passed, res.reason


def test_softmax_and_rmsnorm_refs_match_fp64_definitions():
    g = torch.Generator().manual_seed(2)
    x = 3 * torch.randn(5, 33, generator=g)
    res = verify(torch.from_numpy(ops.softmax_fp64(x)), ops.softmax_ref(x).double(), dtype=torch.float32)
    assert res.passed, res.reason
    gamma = 1 + 0.1 * torch.randn(33, generator=g)
    res = verify(torch.from_numpy(ops.rmsnorm_fp64(x, gamma, 1e-6)),
                 ops.rmsnorm_ref(x, gamma, 1e-6).double(), dtype=torch.float32)
    assert res.passed, res.reason


def test_softmax_constant_row_is_exactly_one_over_n():
    out = ops.softmax_ref(torch.full((2, 4096), 7.25, dtype=torch.float16))
    assert (out == torch.tensor(1.0 / 4096, dtype=torch.float16)).all()


def test_softmax_overflow_rows_stay_finite_and_sum_to_one():
    x = torch.tensor([[60.0, 80.0, 0.0], [80.0, 80.0, 80.0]], dtype=torch.float16)
    out = ops.softmax_ref(x).float()
    assert torch.isfinite(out).all()
    assert torch.allclose(out.sum(-1), torch.ones(2), atol=1e-3)


def test_rmsnorm_zero_row_is_zero_and_finite():
    out = ops.rmsnorm_ref(torch.zeros(2, 64), torch.ones(64), 1e-5)
    assert torch.isfinite(out).all() and (out == 0).all()


def test_zero_weight_gives_gelu_of_bias():
    bias = torch.tensor([-3.0, -0.5, 0.0, 0.5, 3.0])
    out = ops.linear_gelu_ref(torch.randn(4, 8), torch.zeros(8, 5), bias)
    expect = torch.from_numpy(ops.gelu_tanh_fp64(bias.double().numpy())).float()
    assert torch.allclose(out, expect.expand(4, 5), atol=1e-6)


def test_gelu_constant_is_two_sqrt_two_over_pi():
    assert ops.GELU_COEFF == pytest.approx(1.5957691216057308, rel=1e-15)
    assert ops.GELU_COEFF == pytest.approx(2 * math.sqrt(2 / math.pi))


# --- 3. planted mistakes must fail the same checks ---------------------------------


class _Planted:
    """The oracle with one mistake; every other function delegates."""

    def __init__(self, **overrides):
        self.__dict__.update(overrides)

    def __getattr__(self, name):
        return getattr(ops, name)


def _gelu_no_cubic(x, w, bias):
    acc = torch.matmul(x.float(), w.float()) + bias.float()
    return (0.5 * acc * (1 + torch.tanh(math.sqrt(2 / math.pi) * acc))).to(x.dtype)


def _gelu_half_scale(x, w, bias):
    acc = torch.matmul(x.float(), w.float()) + bias.float()
    inner = math.sqrt(2 / math.pi) * (acc + 0.044715 * acc**3)  # missing the 2x of the sigmoid form
    return (acc / (1 + torch.exp(-inner))).to(x.dtype)


def _softmax_no_shift(x):
    e = torch.exp(x)  # in the input dtype, as a naive kernel would
    return (e / e.sum(-1, keepdim=True)).to(x.dtype)


def _rmsnorm_sum(x, gamma, eps=1e-5):
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).sum(-1, keepdim=True) + eps) * gamma.float()).to(x.dtype)


def _rmsnorm_eps_outside(x, gamma, eps=1e-5):
    xf = x.float()
    rms = xf.pow(2).mean(-1, keepdim=True).sqrt()
    return (xf / (rms + eps) * gamma.float()).to(x.dtype)


@pytest.mark.parametrize(
    "name,planted",
    [
        ("linear_gelu_4x6x5_fp32", _Planted(linear_gelu_ref=lambda x, w, b: ops.matmul_ref(x, w))),
        ("linear_gelu_4x6x5_fp32", _Planted(linear_gelu_ref=lambda x, w, b: torch.nn.functional.gelu(
            torch.matmul(x.float(), w.float())).to(x.dtype))),  # bias dropped
        ("linear_gelu_4x6x5_fp32", _Planted(linear_gelu_ref=_gelu_no_cubic)),
        ("linear_gelu_4x6x5_fp32", _Planted(linear_gelu_ref=_gelu_half_scale)),
        ("matmul_5x9x17_fp16", _Planted(matmul_ref=lambda a, b: -ops.matmul_ref(a, b))),
        ("matmul_4x3x33_fp32", _Planted(matmul_ref=lambda a, b: ops.matmul_ref(a[:, :-1], b[:-1]))),
        ("softmax_3x127_fp16", _Planted(softmax_ref=_softmax_no_shift)),
        ("softmax_3x127_fp16", _Planted(softmax_ref=lambda x: torch.softmax(x.float(), 0).to(x.dtype))),
        ("rmsnorm_3x127_fp32", _Planted(rmsnorm_ref=_rmsnorm_sum)),
        ("rmsnorm_2x64_bf16", _Planted(rmsnorm_ref=lambda x, g, eps: ops.rmsnorm_ref(x, torch.ones_like(g), eps))),
    ],
)
def test_planted_mistakes_fail_the_golden_checks(golden, name, planted):
    out, dtype = _run_case(name, golden[name], impl=planted)
    assert not _check(golden[name]["expected"], out, dtype).passed


def test_transposed_operand_fails_a_square_golden_check():
    g = torch.Generator().manual_seed(3)
    a, b = torch.randn(8, 8, generator=g), torch.randn(8, 8, generator=g)
    expected = ops.matmul_fp64(a, b)
    assert verify(torch.from_numpy(expected), ops.matmul_ref(a, b).double(), dtype=torch.float32).passed
    assert not verify(torch.from_numpy(expected), ops.matmul_ref(a, b.t()).double(), dtype=torch.float32).passed


def test_eps_outside_the_root_is_caught_on_a_small_row():
    x = torch.full((1, 16), 1e-3)
    expect = torch.from_numpy(ops.rmsnorm_fp64(x, torch.ones(16), 1e-5))
    assert verify(expect, ops.rmsnorm_ref(x, torch.ones(16), 1e-5).double(), dtype=torch.float32).passed
    assert not verify(expect, _rmsnorm_eps_outside(x, torch.ones(16), 1e-5).double(), dtype=torch.float32).passed


# --- vector_add: bit-exact against the IEEE definition -----------------------------

_HALF = (torch.float16, torch.bfloat16)


def _bits(t: torch.Tensor) -> torch.Tensor:
    return t.contiguous().view(torch.int16)


def _adversarial_pairs(dtype):
    """Ties at every binade, sums that cancel, overflow to inf, subnormals."""
    frac = {torch.float16: 10, torch.bfloat16: 7}[dtype]
    half_ulp_of_one = 2.0 ** -(frac + 1)
    a = [1.0, 1.0 + 2.0 ** -frac, 3.0, -1.0, 2.0 ** -14, 6.0e4, 1e-7, 0.0, -0.0]
    b = [half_ulp_of_one, half_ulp_of_one, 3 * half_ulp_of_one * 2, -half_ulp_of_one,
         2.0 ** -24, 6.0e4, -1e-7, -0.0, -0.0]
    return torch.tensor(a).to(dtype), torch.tensor(b).to(dtype)


@pytest.mark.parametrize("dtype", _HALF, ids=["fp16", "bf16"])
def test_vector_add_ref_is_the_correctly_rounded_sum(dtype):
    g = torch.Generator().manual_seed(11)
    scale = torch.exp(4 * torch.randn(4000, generator=g))
    a = (torch.randn(4000, generator=g) * scale).to(dtype)
    b = (torch.randn(4000, generator=g) * scale.flip(0)).to(dtype)
    assert torch.equal(_bits(ops.vector_add_ref(a, b)), _bits(ops.vector_add_exact(a, b)))
    a, b = _adversarial_pairs(dtype)
    assert torch.equal(_bits(ops.vector_add_ref(a, b)), _bits(ops.vector_add_exact(a, b)))


def test_exact_rounding_breaks_ties_to_even():
    one = torch.tensor([1.0, 1.0 + 2.0 ** -10], dtype=torch.float16)
    half_ulp = torch.full((2,), 2.0 ** -11, dtype=torch.float16)
    out = ops.vector_add_exact(one, half_ulp).tolist()
    assert out == [1.0, 1.0 + 2.0 ** -9]  # even neighbour each time
    assert ops.vector_add_exact(torch.tensor([6.0e4], dtype=torch.float16),
                                torch.tensor([6.0e4], dtype=torch.float16)).isinf().all()


@pytest.mark.parametrize("dtype", [torch.float32, *_HALF], ids=["fp32", "fp16", "bf16"])
def test_vector_add_closed_forms(dtype):
    g = torch.Generator().manual_seed(12)
    a = torch.randn(1000, generator=g).to(dtype)
    b = torch.randn(1000, generator=g).to(dtype)
    assert torch.equal(ops.vector_add_ref(a, torch.zeros_like(a)), a)
    neg = ops.vector_add_ref(a, -a)
    assert (neg == 0).all() and not torch.signbit(neg).any()  # x + (-x) = +0 in round-to-nearest
    assert torch.equal(ops.vector_add_ref(a, b), ops.vector_add_ref(b, a))


def _truncating_add(a, b):
    """Round toward zero instead of to nearest even: where rounding went up in
    magnitude, step one unit of the 16-bit format back toward zero."""
    s = a.double() + b.double()
    q = s.to(a.dtype)
    over = (q.double().abs() > s.abs()) & torch.isfinite(q)
    toward_zero = (_bits(q) - 1).view(a.dtype)
    return torch.where(over, toward_zero, q)


def _double_rounded_add(a, b):
    """fp16 sum rounded through bf16 first: too few bits in the intermediate."""
    return (a.float() + b.float()).to(torch.bfloat16).to(a.dtype)


@pytest.mark.parametrize("planted", [_truncating_add, _double_rounded_add,
                                     lambda a, b: ops.vector_add_ref(a, -b)])
def test_planted_vector_add_mistakes_fail_the_exact_check(planted):
    g = torch.Generator().manual_seed(13)
    a = torch.randn(2000, generator=g).to(torch.float16)
    b = torch.randn(2000, generator=g).to(torch.float16)
    assert not torch.equal(_bits(planted(a, b)), _bits(ops.vector_add_exact(a, b)))


# --- the two-pass RMSNorm shares rmsnorm_ref: pin it at widths past 16384 ---------


@pytest.mark.parametrize("cols", [16385, 40000])
def test_rmsnorm_ref_matches_fp64_on_rows_past_the_single_pass_limit(cols):
    g = torch.Generator().manual_seed(cols)
    x = torch.randn(2, cols, generator=g)
    gamma = 1 + 0.1 * torch.randn(cols, generator=g)
    res = verify(torch.from_numpy(ops.rmsnorm_fp64(x, gamma, 1e-6)),
                 ops.rmsnorm_ref(x, gamma, 1e-6).double(), dtype=torch.float32)
    assert res.passed, res.reason
    # Dividing by the single-pass block (16384) instead of the width must fail.
    wrong = (x * torch.rsqrt(x.pow(2).sum(-1, keepdim=True) / 16384 + 1e-6) * gamma)
    assert not verify(torch.from_numpy(ops.rmsnorm_fp64(x, gamma, 1e-6)), wrong.double(),
                      dtype=torch.float32).passed
