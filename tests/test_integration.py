"""TransformerBlock without a GPU: geometry checks, backend selection, a
closed form of the torch backend, and that the kernelforge backend refuses
host tensors instead of falling back (kernelforge/tests/test_transformer.py:
25-34). The backend-parity tests run on the GPU (test_gpu_widening.py).
"""

from __future__ import annotations

import pytest
import torch

from kernelforge.integration.transformer import (
    BACKEND_KERNELO,
    BACKEND_TORCH,
    BACKENDS,
    BlockConfig,
    TransformerBlock,
)

SMALL = BlockConfig(hidden=64, heads=4, intermediate=96)


def test_indivisible_head_count_is_rejected():
    with pytest.raises(ValueError, match="not divisible"):
        BlockConfig(hidden=100, heads=8, intermediate=256)


def test_head_dim_and_defaults_are_llama_7b():
    cfg = BlockConfig()
    assert (cfg.hidden, cfg.heads, cfg.intermediate, cfg.head_dim) == (4096, 32, 11008, 128)


def test_unknown_backend_is_rejected():
    with pytest.raises(ValueError, match="backend must be one of"):
        TransformerBlock(SMALL, device="cpu", dtype=torch.float32, backend="cutlass")
    assert BACKENDS == (BACKEND_TORCH, BACKEND_KERNELO)


def test_zero_weights_make_the_block_the_identity():
    """Attention and MLP outputs are multiplied by zero projections, so the
    two residual adds return x unchanged whatever the norms and GELU do."""
    block = TransformerBlock(SMALL, device="cpu", dtype=torch.float32)
    with torch.no_grad():
        for name, p in block.named_parameters():
            if "proj" in name or "mlp" in name:
                p.zero_()
        block.mlp_up.bias.fill_(0.5)
    x = torch.randn(2, 5, 64, generator=torch.Generator().manual_seed(0))
    with torch.inference_mode():
        assert torch.equal(block(x), x)


def test_torch_backend_runs_on_the_cpu_and_is_causal():
    """Changing a later token must not change an earlier token's output."""
    block = TransformerBlock(SMALL, device="cpu", dtype=torch.float32)
    g = torch.Generator().manual_seed(1)
    with torch.no_grad():
        for p in block.parameters():
            p.copy_(torch.randn(p.shape, generator=g) * 0.05)
    x = torch.randn(1, 6, 64, generator=g)
    y = x.clone()
    y[:, 4:] += 1.0
    with torch.inference_mode():
        a, b = block(x), block(y)
    assert a.shape == x.shape
    assert torch.allclose(a[:, :4], b[:, :4], atol=1e-6)
    assert not torch.allclose(a[:, 4:], b[:, 4:])


def test_input_shape_is_validated():
    block = TransformerBlock(SMALL, device="cpu", dtype=torch.float32)
    with pytest.raises(ValueError, match=r"\(batch, seq, hidden\)"):
        block(torch.zeros(4, 64))
    with pytest.raises(ValueError, match="expected hidden"):
        block(torch.zeros(1, 4, 128))


def test_kernel_backend_refuses_host_tensors():
    block = TransformerBlock(SMALL, device="cpu", dtype=torch.float32, backend=BACKEND_KERNELO)
    with pytest.raises(ValueError, match="ROCm device tensor"), torch.inference_mode():
        block(torch.zeros(1, 4, 64))
