"""GPU tests of the staged backward under a workspace budget
(``npu_flash_attention.ds_workspace_limit``, flexatt_bwd_workspace_limited):
when the whole dS band exceeds the budget, flexatt_bwd_ws runs in passes over
chunks of whole (batch, KV-head) groups, each pass a problem of its own whose
tensors, LSE / Delta rows, ALiBi slopes, interval bounds and block-map rows
are offset to the chunk; when not even one group fits, the recomputing
backward runs.

* every pass plan (whole batches per pass, KV heads of one batch per pass
  with a short last pass, the recomputing fallback) against the float64
  oracle at the north-star bounds, with per-head ALiBi slopes, per-batch
  document bounds, PrefixLM column bounds and per-head block maps, so that a
  wrong offset in any of them shows;
* the passes against the one-pass result of the same call (same kernels,
  fp32 summation order aside).
"""
import pytest
import torch

import flexatt_lib as L
import npu_flash_attention as nfa
from gpu_helpers import alibi_slopes, check, draw
from oracle import attention_oracle as orc

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _stage_wherever_in_range(monkeypatch):
    # the pass plans under test, not flexatt_bwd_prefers_staging's choice, and
    # under the fixed ds_workspace_limit alone (no share of free memory)
    monkeypatch.setattr(nfa, "ds_staging_auto", False)
    monkeypatch.setattr(nfa, "ds_workspace_free_fraction", 0.0)


def _units(sq, skv, causal, window):
    """Staged units per query head (closed form of the band)."""
    nkb = -(-skv // 128)
    n = 0
    for t in range(-(-sq // 32)):
        lo = min(nkb, max(0, (32 * t - window) // 128)) if window > 0 else 0
        hi = min(nkb, t // 4 + 1) if causal else nkb
        n += max(0, hi - lo)
    return n


# name: (dtype, D, B, Hq, Hkv, Sq, Skv, groups per pass (0: recompute), kwargs)
CASES = {
    # 3 KV heads per pass over Hkv = 4: passes of 3 and 1 heads in each batch
    "bf16_d128_heads_3_1_alibi_cap_blocks": (torch.bfloat16, 128, 2, 8, 4, 300, 300, 3,
                                             dict(causal=True, alibi=True, soft_cap=30.0, blocks=(1, 8))),
    # one batch per pass (4 groups per pass, Hkv = 2 -> 2 batches of 2 groups; B = 3: 2 + 1)
    "fp16_d64_batches_docs_window": (torch.float16, 64, 3, 4, 2, 400, 400, 4,
                                     dict(sliding_window=150, doc=[[100, 250, 50], [400], [10, 390]])),
    # one KV head per pass, PrefixLM per batch row (column bounds), Sq != Skv not allowed with prefix
    "bf16_d256_heads_1_prefix": (torch.bfloat16, 256, 2, 4, 2, 260, 260, 1, dict(causal=True, prefix=[30, 200])),
    # fp32 stages 4 bytes per pair: two KV heads per pass over Hkv = 3 (2 + 1)
    "fp32_d64_heads_2_1_shared_blocks": (torch.float32, 64, 1, 6, 3, 257, 300, 2,
                                         dict(causal=True, sliding_window=100, blocks=(2, 1))),
    # below one group's band: the recomputing backward
    "bf16_d128_recompute": (torch.bfloat16, 128, 2, 4, 2, 300, 300, 0, dict(causal=True, alibi=True)),
}


def _setup(case):
    dtype, d, b, hq, hkv, sq, skv, groups, kw = CASES[case]
    kw = dict(kw)
    cpu, dev = draw(150, b, hq, hkv, sq, skv, d, dtype)
    ref = {}
    if kw.pop("alibi", False):
        kw["alibi_slope"] = alibi_slopes(hq).to("cuda")
    if "prefix" in kw:
        pl = torch.tensor(kw.pop("prefix"))
        kw["prefix_len"] = pl.cuda()
        ref["prefix_len"] = pl
    if "doc" in kw:
        ids = torch.stack([torch.cat([torch.full((n,), i, dtype=torch.int32) for i, n in enumerate(row)])
                           for row in kw.pop("doc")])
        kw["document_ids"] = ids.cuda()
        ref["document_ids"] = ids
    if "blocks" in kw:
        seed, heads = kw.pop("blocks")
        g = torch.Generator().manual_seed(seed)
        bm = (torch.rand(b, heads, -(-sq // 128), -(-skv // 128), generator=g) < 0.6).to(torch.uint8)
        kw["block_mask"] = bm.cuda()
        ref["block_map"] = bm
    per_pair = 4 if dtype == torch.float32 else 2
    group_bytes = (hq // hkv) * _units(sq, skv, kw.get("causal", False), kw.get("sliding_window", 0)) * 32 * 128 * per_pair
    return dtype, cpu, dev, kw, ref, groups, group_bytes


def _backward(q, k, v, do, kw, limit):
    o, lse = nfa.npu_flash_attention_forward(q, k, v, return_lse=True, **kw)
    old = nfa.ds_workspace_limit
    nfa.ds_workspace_limit = limit
    try:
        grads = nfa.npu_flash_attention_backward(q, k, v, o, lse, do, **kw)
    finally:
        nfa.ds_workspace_limit = old
    torch.cuda.synchronize()
    return (o, lse) + tuple(grads)


@pytest.mark.parametrize("case", list(CASES))
def test_bounded_workspace_passes_match_oracle(gpu_device, case):
    dtype, cpu, (q, k, v, do), kw, ref, groups, gb = _setup(case)
    b, hkv = q.shape[0], k.shape[1]
    limit = groups * gb + L.BWD_QUEUE_BYTES if groups else gb - 1
    # the plan the budget selects: fewer groups per pass than the problem has
    p = nfa._problem(q, k, kw.get("scale") or q.shape[-1] ** -0.5, kw.get("causal", False),
                     kw.get("sliding_window", 0), kw.get("soft_cap", 0.0), None)
    old = nfa.ds_workspace_limit
    nfa.ds_workspace_limit = limit
    try:
        n = nfa._staged_workspace_bytes(L.load(), p)
    finally:
        nfa.ds_workspace_limit = old
    assert n == (groups * gb + L.BWD_QUEUE_BYTES if groups else 0) and groups < b * hkv
    got = _backward(q, k, v, do, kw, limit)
    sl = None if kw.get("alibi_slope") is None else kw["alibi_slope"].cpu()
    args = (kw.get("causal", False), kw.get("sliding_window", 0), sl, kw.get("scale"), kw.get("soft_cap", 0.0))
    want = orc.forward(*cpu[:3], *args, **ref) + tuple(orc.backward(*cpu, *args, **ref))
    for name, x, r in zip(("o", "lse", "dq", "dk", "dv"), got, want):
        check(name, x, r, dtype)
    # against the one-pass call (same kernels; dK/dV may differ in the last
    # bits, where a work item's walk direction depends on its slot in the grid)
    whole = _backward(q, k, v, do, kw, 1 << 40)
    for name, x, r in zip(("dq", "dk", "dv"), got[2:], whole[2:]):
        check(name, x, r.double(), dtype)


def test_free_memory_share_keeps_the_whole_band(gpu_device, monkeypatch):
    """With the fixed limit below one group's band but a share of the free
    device memory above the whole band, the backward stages the whole band in
    one pass (instead of the recomputing fallback) and matches the oracle."""
    dtype, cpu, (q, k, v, do), kw, ref, _, gb = _setup("bf16_d128_recompute")
    monkeypatch.setattr(nfa, "ds_workspace_free_fraction", 0.25)
    lib = L.load()
    p = nfa._problem(q, k, q.shape[-1] ** -0.5, kw.get("causal", False), kw.get("sliding_window", 0),
                     kw.get("soft_cap", 0.0), kw.get("alibi_slope"))
    full = lib.flexatt_bwd_workspace(p)
    assert 0.25 * nfa._free_device_bytes(q.device) > full
    old = nfa.ds_workspace_limit
    nfa.ds_workspace_limit = gb - 1
    try:
        assert nfa._staged_workspace_bytes(lib, p) == 0           # the fixed limit alone: recompute
        assert nfa._staged_workspace_bytes(lib, p, q.device) == full  # with the free-memory share: staged
    finally:
        nfa.ds_workspace_limit = old
    got = _backward(q, k, v, do, kw, gb - 1)
    sl = kw["alibi_slope"].cpu()
    args = (kw.get("causal", False), kw.get("sliding_window", 0), sl, kw.get("scale"), kw.get("soft_cap", 0.0))
    want = orc.forward(*cpu[:3], *args, **ref) + tuple(orc.backward(*cpu, *args, **ref))
    for name, x, r in zip(("o", "lse", "dq", "dk", "dv"), got, want):
        check(name, x, r, dtype)
