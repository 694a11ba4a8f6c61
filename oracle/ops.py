"""CPU oracle for the kernelforge hot path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module, and only as the checker (or the timed CPU baseline),
never as a path that product code routes through.

Each function restates the reference's own PyTorch oracle for one kernel on
the host CPU, in fp32 (the precision the reference's gate assumes), plus
fp64 brute-force forms for tiny shapes that pin the restatements to the
mathematics rather than to torch:

=====================  ===========================================================
function               reference it restates
=====================  ===========================================================
matmul_ref             MatmulOperator.reference: torch.matmul under TF32-off
                       (kernelforge/kernels/matmul.py:228-233, testing.py:157-175)
linear_gelu_ref        linear_gelu_reference: gelu(x@w + bias, approximate="tanh")
                       (kernelforge/kernels/fused_linear.py:160-162)
softmax_ref            SoftmaxOperator.reference: torch.softmax(x, dim=-1)
                       (kernelforge/kernels/softmax.py:124-126)
rmsnorm_ref            rmsnorm_reference (kernelforge/kernels/rmsnorm.py:130-143);
                       also the oracle of the two-pass kernel for rows of any
                       width (the same function, README.md:656-660)
vector_add_ref         VectorAddOperator.reference: a + b
                       (kernelforge/kernels/vector_add.py:85-87)
*_fp64                 textbook definitions evaluated in float64 with numpy
vector_add_exact       the correctly rounded sum from exact rational arithmetic
=====================  ===========================================================

How each is pinned (tests/test_oracle.py): against the fp64 definitions on
small shapes, against closed forms the reference's tests use (constant-row
softmax = 1/n, identity/zero-weight GELU, all-zero RMSNorm row), against the
committed golden vectors in tests/golden/, and with planted mistakes (a
dropped bias, a wrong GELU constant, a transposed operand) that must fail.
vector_add_ref is pinned bit for bit against vector_add_exact (Fractions,
round half to even) on random and adversarial 16-bit pairs, and against the
closed forms a + 0 = a, a + (-a) = +0 and a + b = b + a.

The oracle computes in fp32 with one final rounding to the output dtype,
which is the contract the HIP kernels implement (fp32 accumulate, single
rounding). The reference's GPU oracle rounds intermediates to the input
dtype (e.g. ``matmul`` then ``+ bias`` in fp16); the difference is inside
the per-dtype gate tolerance by design (kernelforge/testing.py:26-35).
"""

from __future__ import annotations

import math

import numpy as np
import torch

#: 2*sqrt(2/pi): tanh(z) = 2*sigmoid(2z) - 1 folds the factor of two in.
GELU_COEFF = 2.0 * math.sqrt(2.0 / math.pi)
GELU_CUBIC = 0.044715


def _f32(t: torch.Tensor) -> torch.Tensor:
    return t.detach().to(device="cpu", dtype=torch.float32)


def matmul_ref(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """``a @ b`` with fp32 accumulation, rounded once to the input dtype."""
    prev = torch.get_float32_matmul_precision()
    torch.set_float32_matmul_precision("highest")
    try:
        return torch.matmul(_f32(a), _f32(b)).to(a.dtype)
    finally:
        torch.set_float32_matmul_precision(prev)


def linear_gelu_ref(x: torch.Tensor, w: torch.Tensor, bias: torch.Tensor) -> torch.Tensor:
    """``gelu_tanh(x @ w + bias)`` in fp32, rounded once."""
    acc = torch.matmul(_f32(x), _f32(w)) + _f32(bias)
    return torch.nn.functional.gelu(acc, approximate="tanh").to(x.dtype)


def softmax_ref(x: torch.Tensor) -> torch.Tensor:
    """Row softmax over the last dimension in fp32, rounded once."""
    return torch.softmax(_f32(x), dim=-1).to(x.dtype)


def rmsnorm_ref(x: torch.Tensor, gamma: torch.Tensor, eps: float = 1e-5) -> torch.Tensor:
    """``x * rsqrt(mean(x^2) + eps) * gamma`` in fp32, rounded once."""
    xf = _f32(x)
    inv_rms = torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + eps)
    return (xf * inv_rms * _f32(gamma)).to(x.dtype)


def vector_add_ref(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """``a + b`` formed in fp32 and rounded once to the input dtype."""
    return (_f32(a) + _f32(b)).to(a.dtype)


# --- fp64 textbook definitions (small shapes only) ----------------------------


def _np64(t: torch.Tensor) -> np.ndarray:
    return t.detach().to(device="cpu", dtype=torch.float64).numpy()


def matmul_fp64(a: torch.Tensor, b: torch.Tensor) -> np.ndarray:
    """Triple loop: c[i, j] = sum_k a[i, k] * b[k, j]."""
    A, B = _np64(a), _np64(b)
    m, k = A.shape
    n = B.shape[1]
    C = np.zeros((m, n))
    for i in range(m):
        for j in range(n):
            s = 0.0
            for q in range(k):
                s += A[i, q] * B[q, j]
            C[i, j] = s
    return C


def gelu_tanh_fp64(v: np.ndarray) -> np.ndarray:
    """0.5 v (1 + tanh(sqrt(2/pi) (v + 0.044715 v^3)))."""
    return 0.5 * v * (1.0 + np.tanh(math.sqrt(2.0 / math.pi) * (v + GELU_CUBIC * v**3)))


def linear_gelu_fp64(x: torch.Tensor, w: torch.Tensor, bias: torch.Tensor) -> np.ndarray:
    return gelu_tanh_fp64(matmul_fp64(x, w) + _np64(bias)[None, :])


def softmax_fp64(x: torch.Tensor) -> np.ndarray:
    X = _np64(x)
    out = np.empty_like(X)
    for r in range(X.shape[0]):
        row = X[r]
        e = np.exp(row - row.max())
        out[r] = e / e.sum()
    return out


def rmsnorm_fp64(x: torch.Tensor, gamma: torch.Tensor, eps: float = 1e-5) -> np.ndarray:
    X, G = _np64(x), _np64(gamma)
    out = np.empty_like(X)
    for r in range(X.shape[0]):
        ms = sum(v * v for v in X[r]) / X.shape[1]
        out[r] = X[r] / math.sqrt(ms + eps) * G
    return out


def _round_to_format(q, mantissa_bits: int, min_exp: int, max_exp: int) -> float:
    """Nearest value of a binary format to the rational ``q``, ties to even.

    The format has ``mantissa_bits`` fraction bits, normal exponents
    ``min_exp..max_exp`` and subnormals below; overflow gives +-inf.
    """
    from fractions import Fraction

    if q == 0:
        return 0.0
    sign = -1.0 if q < 0 else 1.0
    q = abs(Fraction(q))
    exp = q.numerator.bit_length() - q.denominator.bit_length()
    if Fraction(2) ** exp > q:
        exp -= 1
    exp = max(exp, min_exp)  # subnormals share the smallest exponent's spacing
    ulp = Fraction(2) ** (exp - mantissa_bits)
    units = q / ulp
    n = units.numerator // units.denominator
    rem = units - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    value = n * ulp
    largest = (2 - Fraction(2) ** -mantissa_bits) * Fraction(2) ** max_exp
    if value > largest:
        return sign * math.inf
    return sign * float(value)


#: (fraction bits, smallest normal exponent, largest exponent) per dtype.
_FORMATS = {torch.float16: (10, -14, 15), torch.bfloat16: (7, -126, 127)}


def vector_add_exact(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """The exact sum of each pair, rounded to nearest-even in the 16-bit
    input format: the IEEE definition of the correctly rounded addition,
    computed with Python Fractions (small inputs only)."""
    from fractions import Fraction

    fmt = _FORMATS[a.dtype]
    av = a.detach().to("cpu", torch.float64).reshape(-1).tolist()
    bv = b.detach().to("cpu", torch.float64).reshape(-1).tolist()
    out = []
    for x, y in zip(av, bv):
        if math.isinf(x) or math.isinf(y) or math.isnan(x) or math.isnan(y):
            out.append(x + y)
            continue
        exact = Fraction(x) + Fraction(y)
        if exact == 0:
            # An exact zero sum is +0 under round-to-nearest, except -0 + -0.
            both_negative = math.copysign(1.0, x) < 0 and math.copysign(1.0, y) < 0
            out.append(-0.0 if both_negative else 0.0)
            continue
        out.append(_round_to_format(exact, *fmt))
    return torch.tensor(out, dtype=torch.float64).reshape(a.shape).to(a.dtype)
