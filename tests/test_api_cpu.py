"""Host-side behaviour of the drop-in module that needs no GPU: argument
errors raised before any launch, AttentionConfig, and that CPU tensors are
refused (there is no CPU fallback)."""
import pytest
import torch

import npu_flash_attention as nfa


def cpu(*shape, dtype=torch.float16):
    return torch.randn(*shape, dtype=dtype)


def test_public_names():
    for name in ("npu_flash_attention_forward", "npu_flash_attention_backward", "NPUFlexAttention",
                 "npu_flex_attention", "AttentionConfig", "flex_attention"):
        assert hasattr(nfa, name)


def test_head_dim_mismatch_rejected():  # R04, npu_flash_attention.py:620
    with pytest.raises((AssertionError, RuntimeError)):
        nfa.npu_flash_attention_forward(cpu(1, 1, 128, 64), cpu(1, 1, 128, 128), cpu(1, 1, 128, 64), causal=True)


def test_value_dim_mismatch_rejected():  # npu_flash_attention.py:621
    with pytest.raises(AssertionError):
        nfa.npu_flash_attention_forward(cpu(1, 1, 16, 64), cpu(1, 1, 16, 64), cpu(1, 1, 16, 32))


def test_heads_not_divisible_rejected():  # R05, npu_flash_attention.py:622
    with pytest.raises((AssertionError, RuntimeError)):
        nfa.npu_flash_attention_forward(cpu(1, 3, 128, 64), cpu(1, 2, 128, 64), cpu(1, 2, 128, 64), causal=True)


def test_backward_requires_out():  # npu_flash_attention.py:684
    q = cpu(1, 1, 16, 64)
    with pytest.raises(AssertionError):
        nfa.npu_flash_attention_backward(q, q, q, None, torch.zeros(1, 1, 16), q)


def test_cpu_tensors_have_no_fallback():
    q = cpu(1, 1, 16, 64)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        nfa.npu_flash_attention_forward(q, q, q)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        nfa.npu_flash_attention_backward(q, q, q, q, torch.zeros(1, 1, 16), q)


def test_attention_config_validation():  # npu_flash_attention.py:840-844
    with pytest.raises(ValueError):
        nfa.AttentionConfig(sliding_window=-1)
    with pytest.raises(ValueError):
        nfa.AttentionConfig(soft_cap=-0.5)
    c = nfa.AttentionConfig()
    assert (c.causal, c.sliding_window, c.alibi_slope, c.scale, c.soft_cap, c.block_m, c.block_n) == \
        (False, 0, None, None, 0.0, 16, 64)


def test_flex_attention_kwargs_validated():
    q = cpu(1, 1, 16, 64)
    with pytest.raises(ValueError):
        nfa.flex_attention(q, q, q, sliding_window=-2)
    with pytest.raises(TypeError):
        nfa.flex_attention(q, q, q, not_a_field=1)


def test_kernel_ready_layout_rules():
    t = torch.randn(2, 3, 8, 64, dtype=torch.bfloat16)
    assert nfa._kernel_ready(t)
    assert not nfa._kernel_ready(t.transpose(2, 3))           # innermost stride != 1
    assert nfa._kernel_ready(t[:, :1].expand(2, 3, 8, 64))     # stride-0 heads are fine
    assert not nfa._kernel_ready(torch.randn(1, 1, 8, 65)[..., :64])  # rows not 16-byte aligned


# ------------------------------------------------------------ document masks --
def test_document_bounds_match_oracle_mask():
    """The host-side bounds ([lo, hi) per position) describe exactly the
    oracle's document mask (runs of equal ids)."""
    from oracle import attention_oracle as orc

    ids = torch.tensor([[0, 0, 0, 1, 1, 2, 2, 2, 2, 3, 0, 0, 0], [5] * 7 + [6] * 6, [9] * 13])
    bounds = nfa._doc_bounds(ids, 3, 13, 13, "cpu")
    assert bounds.dtype == torch.int32 and bounds.shape == (3, 13, 2) and bounds.is_contiguous()
    j = torch.arange(13)
    mask = (j.view(1, 1, 13) >= bounds[..., :1]) & (j.view(1, 1, 13) < bounds[..., 1:])
    assert torch.equal(mask.unsqueeze(1), orc.document_mask(ids))


def test_document_ids_rejected_when_malformed():
    ids = torch.zeros(1, 16, dtype=torch.int64)
    with pytest.raises(RuntimeError):
        nfa._doc_bounds(ids, 1, 8, 16, "cpu")           # Sq != Skv
    with pytest.raises(RuntimeError):
        nfa._doc_bounds(ids, 2, 16, 16, "cpu")          # batch mismatch
    with pytest.raises(RuntimeError):
        nfa._doc_bounds(ids.float(), 1, 16, 16, "cpu")  # not integers


def test_attention_config_carries_document_ids():
    cfg = nfa.AttentionConfig(causal=True, document_ids=torch.zeros(1, 4, dtype=torch.int32))
    assert cfg.document_ids is not None and cfg.causal
