"""Write tests/golden/kernels_fp64.npz: small known-answer vectors.

The reference commits no golden vectors (every test draws seeded inputs and
compares to torch at run time), so these are computed here, in float64, from
the textbook definitions with numpy loops -- not with torch and not with the
reference:

    matmul          c[i,j] = sum_k a[i,k] b[k,j]
    linear_gelu     gelu_tanh(x @ w + bias), gelu_tanh(v) = 0.5 v (1 + tanh(sqrt(2/pi)(v + 0.044715 v^3)))
    softmax         exp(x - max) / sum(exp(x - max)) per row
    rmsnorm         x / sqrt(mean(x^2) + eps) * gamma per row

Inputs are rounded to their dtype first (stored as float32, exact for fp16 /
bf16 / fp32), so the expected outputs are the exact-arithmetic answers for the
very values a kernel sees. Run from the repository root:

    python tests/golden/make_golden.py
"""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import torch

OUT = Path(__file__).resolve().parent / "kernels_fp64.npz"

_DT = {"fp16": torch.float16, "bf16": torch.bfloat16, "fp32": torch.float32}


def _round(a: np.ndarray, dtype: str) -> np.ndarray:
    return torch.from_numpy(a.astype(np.float32)).to(_DT[dtype]).to(torch.float32).numpy()


def _matmul(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    m, k = a.shape
    n = b.shape[1]
    c = np.zeros((m, n))
    for i in range(m):
        for j in range(n):
            c[i, j] = math.fsum(float(a[i, q]) * float(b[q, j]) for q in range(k))
    return c


def _gelu(v: np.ndarray) -> np.ndarray:
    return 0.5 * v * (1.0 + np.tanh(math.sqrt(2.0 / math.pi) * (v + 0.044715 * v**3)))


def _softmax(x: np.ndarray) -> np.ndarray:
    out = np.empty_like(x, dtype=np.float64)
    for r in range(x.shape[0]):
        e = np.exp(x[r].astype(np.float64) - x[r].max())
        out[r] = e / math.fsum(e)
    return out


def _rmsnorm(x: np.ndarray, g: np.ndarray, eps: float) -> np.ndarray:
    out = np.empty_like(x, dtype=np.float64)
    for r in range(x.shape[0]):
        ms = math.fsum(float(v) * float(v) for v in x[r]) / x.shape[1]
        out[r] = x[r].astype(np.float64) / math.sqrt(ms + eps) * g.astype(np.float64)
    return out


def build() -> dict[str, np.ndarray]:
    rng = np.random.default_rng(20261201)
    arrays: dict[str, np.ndarray] = {}

    def put(name: str, **items: np.ndarray) -> None:
        for key, value in items.items():
            arrays[f"{name}/{key}"] = value

    # GEMMs: the BASELINE edge shape 1x7x3, an awkward fp16 shape, fp32.
    for name, (m, n, k), dtype in (
        ("matmul_1x7x3_bf16", (1, 7, 3), "bf16"),
        ("matmul_5x9x17_fp16", (5, 9, 17), "fp16"),
        ("matmul_4x3x33_fp32", (4, 3, 33), "fp32"),
    ):
        a = _round(rng.uniform(-1, 1, (m, k)), dtype)
        b = _round(rng.uniform(-1, 1, (k, n)), dtype)
        put(name, a=a, b=b, expected=_matmul(a, b), dtype=np.array(dtype))

    # Fused linear with bias, in every dtype.
    for dtype in ("fp32", "fp16", "bf16"):
        x = _round(rng.normal(0, 1, (4, 5)), dtype)
        w = _round(rng.normal(0, 1 / math.sqrt(5), (5, 6)), dtype)
        bias = _round(rng.normal(0, 1, 6), dtype)
        put(f"linear_gelu_4x6x5_{dtype}", x=x, w=w, bias=bias,
            expected=_gelu(_matmul(x, w) + bias[None, :]), dtype=np.array(dtype))

    # GELU tail: identity weight over [-60, 60] and +-1e4 (test_fused_linear.py:96-122).
    vals = np.concatenate([np.linspace(-60, 60, 14), [-1e4, 1e4]]).astype(np.float32)
    put("gelu_identity_fp32", x=np.diag(vals), w=np.eye(16, dtype=np.float32),
        bias=np.zeros(16, np.float32), expected=_gelu(np.diag(vals.astype(np.float64))),
        dtype=np.array("fp32"))

    # Softmax: a +60 overflow row in fp16, a constant row, a non-power-of-two width.
    x = rng.normal(0, 3, (3, 127))
    x[1] += 60.0
    x = _round(x, "fp16")
    put("softmax_3x127_fp16", x=x, expected=_softmax(x), dtype=np.array("fp16"))
    c = np.full((2, 8), 7.25, np.float32)
    put("softmax_const_2x8_fp32", x=c, expected=_softmax(c), dtype=np.array("fp32"))

    # RMSNorm: eps=1e-6 fp32 and an all-zero row.
    x = _round(rng.normal(0, 1, (3, 127)), "fp32")
    g = _round(1.0 + 0.1 * rng.normal(0, 1, 127), "fp32")
    x[2] = 0.0
    put("rmsnorm_3x127_fp32", x=x, gamma=g, eps=np.array(1e-6),
        expected=_rmsnorm(x, g, 1e-6), dtype=np.array("fp32"))
    x16 = _round(rng.normal(0, 1, (2, 64)), "bf16")
    g16 = _round(1.0 + 0.1 * rng.normal(0, 1, 64), "bf16")
    put("rmsnorm_2x64_bf16", x=x16, gamma=g16, eps=np.array(1e-5),
        expected=_rmsnorm(x16, g16, 1e-5), dtype=np.array("bf16"))
    return arrays


def main() -> None:
    np.savez_compressed(OUT, **build())
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
