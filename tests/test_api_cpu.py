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


# ------------------------------------------------- PrefixLM and block masks --
def _interval_dense(bounds, n):
    j = torch.arange(n)
    return (j.view(1, 1, n) >= bounds[..., :1]) & (j.view(1, 1, n) < bounds[..., 1:])


@pytest.mark.parametrize("sq,skv,prefix,with_doc", [
    (13, 13, [0, 4, 13], False), (13, 13, [2, 7, 30], True), (9, 14, [5, 0, 14], False), (16, 7, 3, False)])
def test_prefix_bounds_match_oracle_mask(sq, skv, prefix, with_doc):
    """Row bounds (keys per query row) and column bounds (query rows per key)
    both describe the oracle's causal PrefixLM mask, intersected with the
    document mask when ids are given, and are non-decreasing."""
    from oracle import attention_oracle as orc

    B = 3
    ids = torch.tensor([[0] * 5 + [1] * 8, [2] * 13, [0, 0, 1, 1, 1, 1, 1, 1, 1, 2, 2, 3, 3]]) if with_doc else None
    doc = nfa._doc_bounds(ids, B, sq, skv, "cpu") if with_doc else None
    rows, cols = nfa._prefix_bounds(prefix, doc, B, sq, skv, "cpu")
    assert rows.dtype == cols.dtype == torch.int32 and rows.shape == (B, sq, 2) and cols.shape == (B, skv, 2)
    for x in (rows, cols):
        assert (x[:, 1:] >= x[:, :-1]).all()
    pl = torch.as_tensor(prefix).expand(B) if isinstance(prefix, int) else torch.tensor(prefix)
    want = torch.stack([orc._mask(sq, skv, True, 0, None if ids is None else ids[b:b + 1], pl[b:b + 1])
                        .reshape(sq, skv) for b in range(B)])
    assert torch.equal(_interval_dense(rows, skv), want)
    assert torch.equal(_interval_dense(cols, sq), want.transpose(1, 2))


def test_masks_encode_prefix_without_causal_flag():
    m = nfa._masks(True, None, 4, None, 1, 2, 8, 8, "cpu")
    assert m.causal is False and m.rows is not None and m.cols is not None and m.blocks is None
    assert nfa._masks(True, None, None, None, 1, 2, 8, 8, "cpu") is None
    assert nfa._masks(False, None, 4, None, 1, 2, 8, 8, "cpu") is None  # prefix only relaxes causal
    with pytest.raises(RuntimeError):
        nfa._prefix_bounds(torch.tensor([1.5]), None, 1, 8, 8, "cpu")
    with pytest.raises(RuntimeError):
        nfa._prefix_bounds([1, 2, 3], None, 2, 8, 8, "cpu")
    with pytest.raises(ValueError):
        nfa.AttentionConfig(prefix_len=3)


def test_block_map_forms_agree():
    """Dense map, (kv_num_blocks, kv_indices), BlockMask.from_kv_blocks and a
    block-aligned create_block_mask give the same uint8 map."""
    from torch.nn.attention.flex_attention import BlockMask, create_block_mask

    B, H, S = 2, 4, 300  # 3 x 3 blocks of 128, the last ones partial
    gen = torch.Generator().manual_seed(1)
    dense = torch.rand(B, H, 3, 3, generator=gen) > 0.5
    want = dense.to(torch.uint8)
    num = dense.sum(-1).to(torch.int32)
    idx = torch.sort(torch.where(dense, torch.arange(3), 3 + torch.arange(3)), dim=-1).values.to(torch.int32)
    idx = torch.where(idx >= 3, torch.zeros_like(idx), idx)  # unlisted slots hold junk the count excludes
    for form in (dense, dense.to(torch.int64), (num, idx), BlockMask.from_kv_blocks(num, idx, BLOCK_SIZE=128)):
        got = nfa._block_map(form, B, H, S, S, "cpu")
        assert got.dtype == torch.uint8 and got.is_contiguous() and torch.equal(got, want)
    # full blocks of a mask_mod that is constant over each 128 x 128 block
    bm = create_block_mask(lambda b, h, q, kv: (q // 128) >= (kv // 128), 1, 1, 384, 384, device="cpu")
    assert torch.equal(nfa._block_map(bm, 2, 4, 384, 384, "cpu"),
                       torch.tril(torch.ones(3, 3, dtype=torch.uint8)).expand(2, 1, 3, 3))
    # batch 1 broadcasts, heads 1 stay one map
    one = nfa._block_map(dense[:1, :1], B, H, S, S, "cpu")
    assert one.shape == (B, 1, 3, 3) and torch.equal(one[1], want[0, :1])


def test_block_map_rejections():
    from torch.nn.attention.flex_attention import BlockMask, create_block_mask

    m = torch.ones(1, 1, 3, 3, dtype=torch.uint8)
    with pytest.raises(RuntimeError):
        nfa._block_map(m[..., :2], 1, 2, 300, 300, "cpu")             # wrong block count
    with pytest.raises(RuntimeError):
        nfa._block_map(m.float(), 1, 2, 300, 300, "cpu")              # not bool / integer
    with pytest.raises(RuntimeError):
        nfa._block_map(m.expand(1, 3, 3, 3), 1, 2, 300, 300, "cpu")   # 3 heads for Hq = 2
    num = torch.tensor([[[1, 1, 1]]], dtype=torch.int32)
    with pytest.raises(RuntimeError):
        nfa._block_map((num, torch.tensor([[[[0], [3], [1]]]], dtype=torch.int32)), 1, 1, 300, 300, "cpu")
    with pytest.raises(RuntimeError):                                 # 64-wide blocks
        nfa._block_map(BlockMask.from_kv_blocks(num, torch.zeros(1, 1, 3, 1, dtype=torch.int32), BLOCK_SIZE=64),
                       1, 1, 192, 192, "cpu")
    with pytest.raises(RuntimeError):                                 # partial blocks need the mask_mod
        nfa._block_map(create_block_mask(lambda b, h, q, kv: q >= kv, 1, 1, 256, 256, device="cpu"),
                       1, 1, 256, 256, "cpu")
    with pytest.raises(RuntimeError):
        nfa._block_map("not a mask", 1, 1, 256, 256, "cpu")


def test_bench_metric_names():
    """bench.py labels the north-star workload with BASELINE.json's metric and
    every other workload with its own dtype and primitives."""
    import json
    import os

    import bench

    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    want = json.load(open(os.path.join(root, "BASELINE.json")))["metric"]
    B, Hq, Hkv, Sq, Skv, D, dts, causal, window, cap, alibi, scale, _ = bench.CONFIGS["gqa_llama3_8b"]
    assert bench.metric_name(dts, Hq, Hkv, Sq, Skv, D, causal, window, cap, alibi, scale) == want
    names = {bench.metric_name(*c[6:7], *c[1:6], *c[7:12]) for c in bench.CONFIGS.values()}
    assert len(names) == len(bench.CONFIGS)
    B, Hq, Hkv, Sq, Skv, D, dts, causal, window, cap, alibi, scale, _ = bench.CONFIGS["all_primitives_d64"]
    m = bench.metric_name(dts, Hq, Hkv, Sq, Skv, D, causal, window, cap, alibi, scale)
    assert m.startswith("fwd+bwd attention TFLOPS & % MFMA peak, fp16 ") and "D=64" in m and "ALiBi" in m
