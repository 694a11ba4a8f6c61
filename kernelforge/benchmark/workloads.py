"""Named problem suites.

The shape lists are the reference's (kernelforge/benchmark/workloads.py:
26-136; the vector_add counts at :108-113): a Llama-7B-sized transformer
(hidden 4096, MLP 11008), decode and prefill token counts, and a
``correctness`` suite of awkward shapes -- 1s, primes and off-by-one tile
boundaries -- that exercises every masked tail.
"""

from __future__ import annotations

import torch

from kernelforge.tuning.config import Problem

HIDDEN = 4096
INTERMEDIATE = 11008

#: A single decode step, a small decode batch, and two prefill lengths.
TOKEN_COUNTS = (1, 32, 512, 2048)

MATMUL_SHAPES: dict[str, tuple[tuple[int, int, int], ...]] = {
    "smoke": ((512, 512, 512), (1024, 1024, 1024)),
    "sweep": (
        (512, 512, 512),
        (1024, 1024, 1024),
        (2048, 2048, 2048),
        (4096, 4096, 4096),
        (512, 4096, 4096),
        (4096, 512, 4096),
        (4096, 4096, 512),
        (2048, 4096, 4096),
        (1024, 4096, 1024),
        (4096, 1024, 4096),
    ),
    "transformer": tuple(
        shape
        for tokens in TOKEN_COUNTS
        for shape in (
            (tokens, HIDDEN, HIDDEN),
            (tokens, INTERMEDIATE, HIDDEN),
            (tokens, HIDDEN, INTERMEDIATE),
        )
    ),
    "correctness": (
        (1, 1, 1),
        (1, 128, 128),
        (128, 1, 128),
        (128, 128, 1),
        (127, 127, 127),
        (128, 128, 128),
        (129, 129, 129),
        (257, 129, 65),
        (511, 769, 1025),
        (1023, 1023, 1023),
        (1024, 1024, 1024),
        (2057, 127, 513),
        (768, 2048, 4096),
    ),
}

ROW_SHAPES: dict[str, tuple[tuple[int, int], ...]] = {
    "smoke": ((2048, 1024), (4096, 4096)),
    "sweep": tuple(
        (rows, cols) for rows in (512, 2048, 8192) for cols in (128, 256, 512, 1024, 2048, 4096, 8192)
    ),
    "transformer": tuple((tokens, HIDDEN) for tokens in TOKEN_COUNTS)
    + tuple((tokens, 768) for tokens in TOKEN_COUNTS),
    "correctness": (
        (1, 1),
        (1, 4096),
        (3, 127),
        (17, 257),
        (128, 511),
        (333, 769),
        (1024, 1023),
        (2048, 1024),
        (4096, 4096),
        (129, 8192),
    ),
}

#: vector_add element counts: a prime just over a million and a 32 MiB fp16
#: stream for smoke; powers of four for the sweep; one prefill activation;
#: and counts around every tile boundary for correctness.
VECTOR_SHAPES: dict[str, tuple[int, ...]] = {
    "smoke": (1_000_003, 16_777_216),
    "sweep": (1 << 16, 1 << 20, 1 << 24, 1 << 26),
    "transformer": (TOKEN_COUNTS[-1] * HIDDEN,),
    "correctness": (1, 2, 13, 127, 128, 129, 1024, 12_345, 1_000_003, 1 << 20),
}

SUITES: tuple[str, ...] = ("smoke", "sweep", "transformer", "correctness")


def problems(operation: str, suite: str = "sweep", dtype: str | torch.dtype = "fp16") -> list[Problem]:
    """Every problem in ``suite`` for ``operation``."""
    if suite not in SUITES:
        raise ValueError(f"unknown suite {suite!r}; available: {', '.join(SUITES)}")
    if operation in ("matmul", "fused_linear"):
        return [Problem.create(operation, dtype, M=m, N=n, K=k) for m, n, k in MATMUL_SHAPES[suite]]
    if operation in ("rmsnorm", "softmax"):
        return [
            Problem.create(operation, dtype, rows=rows, cols=cols) for rows, cols in ROW_SHAPES[suite]
        ]
    if operation == "vector_add":
        return [Problem.create(operation, dtype, n=n) for n in VECTOR_SHAPES[suite]]
    raise ValueError(f"no workload suite defined for {operation!r}")
