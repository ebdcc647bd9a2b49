"""GPU tests of document masks (``document_ids``), which the reference lists
as future work and this build adds on top of every other primitive.

* forward (O, LSE) and backward (dQ, dK, dV) against the oracle with
  document masks, for every dtype and head dim, under causal / window /
  soft-cap / ALiBi / GQA, with one-position documents, one document spanning
  everything, many short documents and a different layout per batch row;
* a row of a document is unaffected by the other documents: attention over
  the packed sequence equals attention run on each document alone;
* the autograd and AttentionConfig entry points carry the mask.
"""
import pytest
import torch

import npu_flash_attention as nfa
from gpu_helpers import alibi_slopes, check, draw, oracle_fwd_bwd
from oracle import attention_oracle as orc

pytestmark = pytest.mark.gpu


def doc_ids(lengths_per_batch):
    """[B, S] ids from document lengths (ids repeat across documents on
    purpose: documents are runs, not values)."""
    rows = []
    for lengths in lengths_per_batch:
        rows.append(torch.cat([torch.full((n,), i % 3, dtype=torch.int32) for i, n in enumerate(lengths)]))
    return torch.stack(rows)


S1 = 300
LAYOUTS = {
    "mixed": [[1, 57, 64, 3, 100, 75], [150, 150]],
    "one_doc": [[S1], [S1]],
    "short_docs": [[7] * 42 + [6], [1] * S1],
}

# name: (dtype, D, Hq, Hkv, layout, kwargs)
CASES = {
    "bf16_d128_causal_gqa_mixed": (torch.bfloat16, 128, 8, 2, "mixed", dict(causal=True)),
    "bf16_d128_full_one_doc": (torch.bfloat16, 128, 4, 4, "one_doc", {}),
    "fp16_d64_window_cap_short": (torch.float16, 64, 6, 2, "short_docs", dict(causal=True, sliding_window=5, soft_cap=20.0)),
    "fp16_d32_alibi_mixed": (torch.float16, 32, 4, 1, "mixed", dict(alibi=True, scale=0.2)),
    "bf16_d256_causal_window_mixed": (torch.bfloat16, 256, 2, 1, "mixed", dict(causal=True, sliding_window=40)),
    "fp32_d64_causal_mixed": (torch.float32, 64, 4, 2, "mixed", dict(causal=True)),
    "fp32_d128_short": (torch.float32, 128, 2, 2, "short_docs", {}),
}


def _setup(case, seed=0):
    dtype, d, hq, hkv, layout, kw = CASES[case]
    kw = dict(kw)
    ids = doc_ids(LAYOUTS[layout])
    cpu, dev = draw(seed + 70, ids.shape[0], hq, hkv, S1, S1, d, dtype)
    if kw.pop("alibi", False):
        kw["alibi_slope"] = alibi_slopes(hq).to("cuda")
    return dtype, ids, cpu, dev, kw


@pytest.mark.parametrize("case", list(CASES))
def test_document_mask_matches_oracle(gpu_device, case):
    dtype, ids, cpu, (q, k, v, do), kw = _setup(case)
    o, lse = nfa.npu_flash_attention_forward(q, k, v, return_lse=True, document_ids=ids.cuda(), **kw)
    dq, dk, dv = nfa.npu_flash_attention_backward(q, k, v, o, lse, do, document_ids=ids.cuda(), **kw)
    torch.cuda.synchronize()
    sl = None if kw.get("alibi_slope") is None else kw["alibi_slope"].cpu()
    ref_o, ref_lse = orc.forward(*cpu[:3], kw.get("causal", False), kw.get("sliding_window", 0), sl,
                                 kw.get("scale"), kw.get("soft_cap", 0.0), document_ids=ids)
    ref_g = orc.backward(*cpu, kw.get("causal", False), kw.get("sliding_window", 0), sl, kw.get("scale"),
                         kw.get("soft_cap", 0.0), document_ids=ids)
    check("o", o, ref_o, dtype)
    check("lse", lse, ref_lse, dtype)
    for name, x, r in zip(("dq", "dk", "dv"), (dq, dk, dv), ref_g):
        check(name, x, r, dtype)


def test_documents_are_independent(gpu_device):
    """Each document of the packed sequence equals an unmasked run over that
    document alone (kernel against kernel, same tolerance as the oracle)."""
    dtype, ids, cpu, (q, k, v, do), kw = _setup("bf16_d128_causal_gqa_mixed", seed=5)
    o, lse = nfa.npu_flash_attention_forward(q, k, v, return_lse=True, document_ids=ids.cuda(), **kw)
    start = 0
    for n in LAYOUTS["mixed"][0]:
        sl = slice(start, start + n)
        qs, ks, vs = (t[0:1, :, sl].contiguous() for t in (q, k, v))
        os_, lses = nfa.npu_flash_attention_forward(qs, ks, vs, return_lse=True, **kw)
        check("o", o[0:1, :, sl], os_.float(), dtype)
        check("lse", lse[0:1, :, sl], lses, dtype)
        start += n


def test_autograd_and_config_carry_documents(gpu_device):
    dtype, ids, cpu, (q, k, v, do), kw = _setup("fp16_d64_window_cap_short", seed=6)
    idc = ids.cuda()
    q, k, v = (t.clone().requires_grad_(True) for t in (q, k, v))
    cfg = nfa.AttentionConfig(document_ids=idc, **kw)
    o = nfa.flex_attention(q, k, v, config=cfg)
    o.backward(do)
    o2, lse2 = nfa.npu_flash_attention_forward(q.detach(), k.detach(), v.detach(), return_lse=True,
                                               document_ids=idc, **kw)
    g2 = nfa.npu_flash_attention_backward(q.detach(), k.detach(), v.detach(), o2, lse2, do, document_ids=idc, **kw)
    assert torch.equal(o, o2)
    for a, b in zip((q.grad, k.grad, v.grad), g2):
        assert torch.equal(a, b)
