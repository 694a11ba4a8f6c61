"""Entry points called without a configuration run the shipped MI355X winner.

The reference runs a fixed ``DEFAULT_CONFIG`` when no configuration is given
(kernels/matmul.py:118-120); here the packaged winner for the call's shape is
used when one ships, and the search space's heuristic otherwise. Checked by
result identity: configurations differ in split-K and reduction layout, so
the shipped and the heuristic configuration give bitwise different outputs
on these shapes.
"""

from __future__ import annotations

import pytest
import torch

from kernelforge.kernels import get_operator
from kernelforge.kernels.fused_linear import fused_linear_gelu
from kernelforge.kernels.matmul import _heuristic_config, matmul
from kernelforge.kernels.rmsnorm import rmsnorm
from kernelforge.kernels.softmax import softmax
from kernelforge.runtime.dispatch import SOURCE_PACKAGED, select_config, shipped_config
from kernelforge.tuning.cache import ConfigCache
from kernelforge.tuning.config import Problem

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda")


def _packaged(operation, dtype, tmp_path, **dims):
    sel = select_config(get_operator(operation), Problem.create(operation, dtype, **dims),
                        cache=ConfigCache(tmp_path / "empty.json"), device=DEV)
    assert sel.source == SOURCE_PACKAGED
    return sel.config


def test_gemv_without_config_runs_the_shipped_winner(tmp_path):
    g = torch.Generator().manual_seed(3)
    x = (torch.rand(1, 4096, generator=g) * 2 - 1).bfloat16().to(DEV)
    w = (torch.rand(4096, 11008, generator=g) * 2 - 1).bfloat16().to(DEV)
    cfg = _packaged("matmul", torch.bfloat16, tmp_path, M=1, N=11008, K=4096)
    assert shipped_config("matmul", torch.bfloat16, DEV, M=1, N=11008, K=4096) == cfg
    assert torch.equal(matmul(x, w), matmul(x, w, config=cfg))


def test_gemm_without_config_runs_the_shipped_winner(tmp_path):
    g = torch.Generator().manual_seed(4)
    a = torch.randn(2048, 4096, generator=g).half().to(DEV)
    b = torch.randn(4096, 4096, generator=g).half().to(DEV)
    cfg = _packaged("matmul", torch.float16, tmp_path, M=2048, N=4096, K=4096)
    assert torch.equal(matmul(a, b), matmul(a, b, config=cfg))


def test_fused_linear_without_config_runs_the_shipped_winner(tmp_path):
    g = torch.Generator().manual_seed(5)
    x = torch.randn(128, 4096, generator=g).half().to(DEV)
    w = (torch.randn(4096, 11008, generator=g) / 64).half().to(DEV)
    bias = torch.randn(11008, generator=g).half().to(DEV)
    cfg = _packaged("fused_linear", torch.float16, tmp_path, M=128, N=11008, K=4096)
    assert torch.equal(fused_linear_gelu(x, w, bias), fused_linear_gelu(x, w, bias, config=cfg))


def test_row_kernels_without_config_run_the_shipped_winner(tmp_path):
    g = torch.Generator().manual_seed(6)
    x = torch.randn(4096, 4096, generator=g).to(DEV)
    gamma = torch.randn(4096, generator=g).to(DEV)
    cfg = _packaged("rmsnorm", torch.float32, tmp_path, rows=4096, cols=4096)
    assert torch.equal(rmsnorm(x, gamma), rmsnorm(x, gamma, config=cfg))
    s = torch.randn(8192, 11008, generator=g).half().to(DEV)
    cfg = _packaged("softmax", torch.float16, tmp_path, rows=8192, cols=11008)
    assert torch.equal(softmax(s), softmax(s, config=cfg))


def test_unshipped_shape_falls_back_to_the_heuristic():
    g = torch.Generator().manual_seed(7)
    a = torch.randn(1000, 999, generator=g).half().to(DEV)
    b = torch.randn(999, 1001, generator=g).half().to(DEV)
    assert shipped_config("matmul", torch.float16, DEV, M=1000, N=1001, K=999) is None
    heuristic = _heuristic_config("matmul", 1000, 1001, 999, torch.float16)
    assert torch.equal(matmul(a, b), matmul(a, b, config=heuristic))
    empty = torch.empty(0, 64, dtype=torch.float16, device=DEV)
    assert matmul(empty, torch.randn(64, 32, dtype=torch.float16, device=DEV)).shape == (0, 32)


def test_decode_over_nn_linear_weights_runs_its_own_winner(tmp_path):
    """``x @ weight.t()`` is the dot-kernel layout: its shipped winner is keyed
    ``+bt`` and differs from the row-major winner of the same shape."""
    g = torch.Generator().manual_seed(8)
    x = (torch.rand(1, 4096, generator=g) * 2 - 1).bfloat16().to(DEV)
    weight = (torch.rand(11008, 4096, generator=g) * 2 - 1).bfloat16().to(DEV)
    bt = _packaged_bt("matmul", torch.bfloat16, tmp_path, M=1, N=11008, K=4096)
    row_major = _packaged("matmul", torch.bfloat16, tmp_path, M=1, N=11008, K=4096)
    assert bt["LANES_PER_ROW"] == 64 and bt != row_major
    assert torch.equal(matmul(x, weight.t()), matmul(x, weight.t(), config=bt))
    bias = torch.randn(11008, generator=g).bfloat16().to(DEV)
    fbt = _packaged_bt("fused_linear", torch.bfloat16, tmp_path, M=1, N=11008, K=4096)
    assert torch.equal(fused_linear_gelu(x, weight.t(), bias), fused_linear_gelu(x, weight.t(), bias, config=fbt))


def _packaged_bt(operation, dtype, tmp_path, **dims):
    sel = select_config(get_operator(operation), Problem.create(operation, dtype, layout="bt", **dims),
                        cache=ConfigCache(tmp_path / "empty_bt.json"), device=DEV)
    assert sel.source == SOURCE_PACKAGED
    return sel.config
