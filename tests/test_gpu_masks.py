"""GPU tests of PrefixLM (``prefix_len``) and block-sparse masks
(``block_mask``), which the reference lists as unsupported (README.md:198,
:219); both act on top of every other primitive, in every kernel.

* forward (O, LSE) and backward (dQ, dK, dV) against the float64 oracle at
  the north-star bounds, for every dtype and head dim: the D = 128 staged
  backward, its recomputing dQ kernel, the general MFMA kernels (D = 32, 64,
  256) and the fp32 kernels; PrefixLM per batch row, with a window, with
  document masks and with Sq != Skv; per-head and shared block maps, with
  row blocks that see no key (O = 0, LSE = -inf, dQ = 0);
* decode-shaped problems (few query rows) with a mask take the regular
  forward and still match;
* a block-diagonal map equals the document mask of 128-aligned documents,
  an all-ones map equals no map;
* the autograd, AttentionConfig and torch.library entry points carry the
  masks.
"""
import pytest
import torch

import npu_flash_attention as nfa
from gpu_helpers import alibi_slopes, check, draw
from oracle import attention_oracle as orc

pytestmark = pytest.mark.gpu


def _block_map(seed, b, h, sq, skv, density=0.6, dead_row=None):
    g = torch.Generator().manual_seed(seed)
    m = (torch.rand(b, h, -(-sq // 128), -(-skv // 128), generator=g) < density).to(torch.uint8)
    if dead_row is not None:
        m[0, 0, dead_row] = 0  # head 0 of batch 0: these query rows see no key
    return m


# name: (dtype, D, B, Hq, Hkv, Sq, Skv, kwargs); "prefix" is a list per batch
# row, "blocks" a (seed, heads, dead row block) triple
CASES = {
    "bf16_d128_prefix": (torch.bfloat16, 128, 2, 8, 2, 500, 500, dict(causal=True, prefix=[37, 300])),
    "fp16_d128_prefix_window_sq_lt_skv": (torch.float16, 128, 1, 4, 1, 260, 450,
                                          dict(causal=True, sliding_window=100, prefix=[200])),
    "bf16_d128_blocks_causal_dead": (torch.bfloat16, 128, 1, 6, 2, 600, 600, dict(causal=True, blocks=(1, 6, 1))),
    "fp16_d128_blocks_shared_all": (torch.float16, 128, 2, 4, 2, 384, 300,
                                    dict(sliding_window=200, alibi=True, soft_cap=20.0, scale=0.07, blocks=(2, 1, None))),
    "bf16_d128_prefix_blocks_doc": (torch.bfloat16, 128, 1, 4, 4, 512, 512,
                                    dict(causal=True, prefix=[150], doc=[100, 200, 212], blocks=(3, 4, None))),
    "fp16_d64_prefix_blocks": (torch.float16, 64, 2, 4, 2, 400, 400, dict(causal=True, prefix=[0, 130], blocks=(4, 4, 2))),
    "bf16_d32_blocks_window_alibi": (torch.bfloat16, 32, 1, 4, 1, 300, 520,
                                     dict(sliding_window=150, alibi=True, blocks=(5, 4, 0))),
    "bf16_d256_prefix_cap": (torch.bfloat16, 256, 1, 2, 1, 300, 300, dict(causal=True, soft_cap=30.0, prefix=[90])),
    "fp16_d256_blocks": (torch.float16, 256, 1, 2, 2, 300, 300, dict(causal=True, blocks=(6, 2, None))),
    "fp32_d64_prefix_doc": (torch.float32, 64, 1, 4, 2, 300, 300, dict(causal=True, prefix=[120], doc=[50, 150, 100])),
    "fp32_d128_blocks": (torch.float32, 128, 1, 2, 1, 260, 260, dict(blocks=(7, 2, 1))),
    # walk lists longer than one 64-lane compaction round in every kernel
    # (66 forward KV tiles, 132 dK/dV query tiles, 66 dQ sub-blocks)
    "bf16_d128_blocks_long": (torch.bfloat16, 128, 1, 2, 1, 4224, 4224, dict(causal=True, blocks=(8, 2, None))),
    "fp16_d64_blocks_long_shared": (torch.float16, 64, 1, 2, 2, 4160, 4200, dict(blocks=(9, 1, 3))),
    # the D = 256 forward's wave pairs walk 32-key tiles: 82 listed tiles
    "bf16_d256_blocks_long_cap": (torch.bfloat16, 256, 1, 2, 1, 2600, 2600, dict(causal=True, soft_cap=30.0,
                                                                              blocks=(10, 2, None))),
    # the fp32 forward's list of 32-key tiles: 72 tiles
    "fp32_d64_blocks_long": (torch.float32, 64, 1, 2, 1, 2200, 2300, dict(causal=True, blocks=(11, 2, None))),
}


def _setup(case, seed=0):
    dtype, d, b, hq, hkv, sq, skv, kw = CASES[case]
    kw = dict(kw)
    cpu, dev = draw(seed + 110, b, hq, hkv, sq, skv, d, dtype)
    ref = {}  # the oracle's mask arguments
    if kw.pop("alibi", False):
        kw["alibi_slope"] = alibi_slopes(hq).to("cuda")
    if "prefix" in kw:
        pl = torch.tensor(kw.pop("prefix"))
        kw["prefix_len"] = pl.cuda()
        ref["prefix_len"] = pl.expand(b) if pl.numel() == 1 else pl
    if "doc" in kw:
        lengths = kw.pop("doc")
        ids = torch.cat([torch.full((n,), i, dtype=torch.int32) for i, n in enumerate(lengths)]).expand(b, -1)
        kw["document_ids"] = ids.cuda()
        ref["document_ids"] = ids
    if "blocks" in kw:
        s, h, dead = kw.pop("blocks")
        bm = _block_map(s, b, h, sq, skv, dead_row=dead)
        kw["block_mask"] = bm.cuda()
        ref["block_map"] = bm
    return dtype, cpu, dev, kw, ref


def _oracle(cpu, kw, ref):
    sl = None if kw.get("alibi_slope") is None else kw["alibi_slope"].cpu()
    args = (kw.get("causal", False), kw.get("sliding_window", 0), sl, kw.get("scale"), kw.get("soft_cap", 0.0))
    o, lse = orc.forward(*cpu[:3], *args, **ref)
    return (o, lse) + tuple(orc.backward(*cpu, *args, **ref))


def _run(q, k, v, do, kw):
    o, lse = nfa.npu_flash_attention_forward(q, k, v, return_lse=True, **kw)
    dq, dk, dv = nfa.npu_flash_attention_backward(q, k, v, o, lse, do, **kw)
    torch.cuda.synchronize()
    return o, lse, dq, dk, dv


@pytest.mark.parametrize("case", list(CASES))
def test_masks_match_oracle(gpu_device, case):
    dtype, cpu, (q, k, v, do), kw, ref = _setup(case)
    got = _run(q, k, v, do, kw)
    want = _oracle(cpu, kw, ref)
    for name, x, r in zip(("o", "lse", "dq", "dk", "dv"), got, want):
        check(name, x, r, dtype)
    if case == "bf16_d128_blocks_causal_dead":  # rows 128..255 of head 0 see no key
        o, lse, dq = got[:3]
        assert torch.isneginf(lse[0, 0, 128:256]).all()
        assert (o[0, 0, 128:256] == 0).all() and (dq[0, 0, 128:256] == 0).all()


@pytest.mark.parametrize("case", ["bf16_d128_prefix", "bf16_d128_blocks_causal_dead", "bf16_d128_prefix_blocks_doc",
                                  "fp32_d64_prefix_doc", "fp32_d128_blocks", "fp32_d64_blocks_long"])
def test_masks_recompute_dq_kernel(gpu_device, case):
    """The backward without dS staging (the recomputing dQ kernels: D = 128
    fp16/bf16 and the fp32 kernels)."""
    dtype, cpu, (q, k, v, do), kw, ref = _setup(case, seed=1)
    nfa.ds_staging_enabled = False
    try:
        got = _run(q, k, v, do, kw)
    finally:
        nfa.ds_staging_enabled = True
    want = _oracle(cpu, kw, ref)
    for name, x, r in zip(("o", "lse", "dq", "dk", "dv"), got, want):
        check(name, x, r, dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_masks_decode_shape(gpu_device, dtype):
    """(Hq / Hkv) * Sq <= 32 would take the split-KV decode kernels; with a
    prefix or a block map the regular forward runs and still matches."""
    cpu, (q, k, v, do) = draw(9, 2, 8, 2, 4, 700, 128, dtype)
    bm = _block_map(11, 2, 8, 4, 700, density=0.5)
    for kw, ref in ((dict(causal=True, prefix_len=torch.tensor([2, 650]).cuda()),
                     dict(prefix_len=torch.tensor([2, 650]))),
                    (dict(block_mask=bm.cuda()), dict(block_map=bm))):
        o, lse = nfa.npu_flash_attention_forward(q, k, v, return_lse=True, **kw)
        ro, rl = orc.forward(*cpu[:3], kw.get("causal", False), 0, None, None, 0.0, **ref)
        torch.cuda.synchronize()
        check("o", o, ro, dtype)
        check("lse", lse, rl, dtype)


@pytest.mark.parametrize("d", [128, 64])
def test_block_map_special_cases(gpu_device, d):
    """A block-diagonal map is the document mask of 128-aligned documents; an
    all-ones map is no map (kernel against kernel, at the oracle bounds)."""
    dtype = torch.bfloat16
    cpu, (q, k, v, do) = draw(12, 1, 4, 2, 384, 384, d, dtype)
    diag = torch.eye(3, dtype=torch.uint8).view(1, 1, 3, 3).cuda()
    ids = (torch.arange(384, dtype=torch.int32) // 128).view(1, -1).cuda()
    a = _run(q, k, v, do, dict(causal=True, block_mask=diag))
    b = _run(q, k, v, do, dict(causal=True, document_ids=ids))
    c = _run(q, k, v, do, dict(causal=True, block_mask=torch.ones(1, 1, 3, 3, dtype=torch.uint8).cuda()))
    e = _run(q, k, v, do, dict(causal=True))
    for name, x, y in zip(("o", "lse", "dq", "dk", "dv"), a, b):
        check(name, x, y.double(), dtype)
    for name, x, y in zip(("o", "lse", "dq", "dk", "dv"), c, e):
        check(name, x, y.double(), dtype)


def test_masks_through_autograd_config_and_ops(gpu_device):
    """npu_flex_attention, flex_attention(AttentionConfig) and
    flexatt_ops.attention give the results of the direct calls."""
    import flexatt_ops

    dtype = torch.bfloat16
    cpu, (q, k, v, do) = draw(13, 1, 4, 2, 300, 300, 128, dtype)
    bm = _block_map(14, 1, 4, 300, 300, density=0.7).cuda()
    kw = dict(causal=True, prefix_len=50, block_mask=bm)
    o, lse, dq, dk, dv = _run(q, k, v, do, kw)
    for fn in (lambda a, b_, c: nfa.npu_flex_attention(a, b_, c, **kw),
               lambda a, b_, c: nfa.flex_attention(a, b_, c, config=nfa.AttentionConfig(**kw)),
               lambda a, b_, c: flexatt_ops.attention(a, b_, c, **kw)):
        qq, kk, vv = (t.detach().clone().requires_grad_() for t in (q, k, v))
        out = fn(qq, kk, vv)
        out.backward(do)
        torch.cuda.synchronize()
        assert torch.equal(out, o)
        assert torch.equal(qq.grad, dq) and torch.equal(kk.grad, dk) and torch.equal(vv.grad, dv)
