"""flexatt_fwd_decode_noalloc: the split-KV decode forward with its partial
results in the library's fixed per-GPU scratch buffer instead of a caller
workspace.

* CPU: problems outside the decode range, or whose partials exceed the fixed
  buffer, are rejected before anything touches the GPU;
* GPU: calls through the C ABI match flexatt_fwd_decode (caller workspace) on
  the same inputs bitwise, and the oracle within the forward tolerance, on
  consecutive calls where a later call is smaller than an earlier one (the
  buffer keeps the last call's contents; each call overwrites every partial
  it reads).
"""
import pytest
import torch

import flexatt_lib as L
import npu_flash_attention as nfa
from gpu_helpers import alibi_slopes, check, draw, oracle_fwd_bwd

FAKE = 1 << 20  # aligned, never dereferenced: every CPU call below fails its checks first


def _problem(**kw):
    p = L.Problem()
    vals = dict(dtype=L.BF16, batch=1, heads_q=32, heads_kv=8, seqlen_q=1, seqlen_kv=4096, head_dim=128,
                scale=0.088, causal=0, sliding_window=0, soft_cap=0.0, alibi_slopes=None, doc_bounds=None)
    vals.update(kw)
    for k, v in vals.items():
        setattr(p, k, v)
    return p


def _fake(hd=128, s=4096):
    return L.Tensor(FAKE, 64 * s * hd, s * hd, hd, 1)


@pytest.mark.parametrize("kw,code", [
    (dict(seqlen_q=64), -6),                           # (Hq / Hkv) * Sq > 32: not a decode problem
    (dict(dtype=L.F32), -6),                           # fp32 has no decode kernels
    (dict(batch=128, heads_q=64, heads_kv=8, seqlen_q=4), -7),  # partials of 16.9 MB > 16 MiB
])
def test_noalloc_rejections_before_gpu(kw, code):
    lib = L.load()
    p = _problem(**kw)
    hd = p.head_dim
    if code == -7:
        assert lib.flexatt_fwd_decode_workspace(p) > L.NOALLOC_SCRATCH_BYTES
    t = _fake(hd)
    assert lib.flexatt_fwd_decode_noalloc(p, t, t, t, t, FAKE, None) == code


def test_noalloc_status_string():
    assert b"scratch" in L.load().flexatt_status_string(-7)


# Consecutive calls: (dtype, B, Hq, Hkv, Sq, Skv, D, kwargs); the second is
# smaller than the first, the third repeats the first.
CALLS = [
    (torch.bfloat16, 4, 32, 8, 1, 8000, 128, dict(causal=False)),
    (torch.float16, 2, 28, 4, 4, 700, 64, dict(sliding_window=300, soft_cap=30.0, alibi=True, scale=0.05)),
    (torch.bfloat16, 4, 32, 8, 1, 8000, 128, dict(causal=False)),
]


def _decode_both(lib, dtype, b, hq, hkv, sq, skv, d, kw, seed):
    cpu, (q, k, v, _) = draw(seed, b, hq, hkv, sq, skv, d, dtype)
    kw = dict(kw)
    if kw.pop("alibi", False):
        kw["alibi_slope"] = alibi_slopes(hq).to("cuda")
    slopes = kw.get("alibi_slope")
    scale = kw.get("scale") or 1.0 / d ** 0.5
    p = nfa._problem(q, k, scale, kw.get("causal", False), kw.get("sliding_window", 0), kw.get("soft_cap", 0.0),
                     slopes)
    n = lib.flexatt_fwd_decode_workspace(p)
    assert 0 < n <= L.NOALLOC_SCRATCH_BYTES
    st = torch.cuda.current_stream().cuda_stream
    o_ws, o_na = torch.empty_like(q), torch.empty_like(q)
    l_ws = torch.empty(b, hq, sq, dtype=torch.float32, device=q.device)
    l_na = torch.empty_like(l_ws)
    ws = torch.empty(n, dtype=torch.uint8, device=q.device)
    T = L.tensor
    L.check(lib.flexatt_fwd_decode(p, T(q), T(k), T(v), T(o_ws), l_ws.data_ptr(), ws.data_ptr(), n, st),
            "flexatt_fwd_decode")
    L.check(lib.flexatt_fwd_decode_noalloc(p, T(q), T(k), T(v), T(o_na), l_na.data_ptr(), st),
            "flexatt_fwd_decode_noalloc")
    torch.cuda.synchronize()
    return cpu, kw, (o_ws, l_ws), (o_na, l_na)


@pytest.mark.gpu
def test_noalloc_matches_workspace_entry(gpu_device):
    lib = L.load()
    for i, (dtype, b, hq, hkv, sq, skv, d, kw) in enumerate(CALLS):
        print(f"noalloc call {i}: {dtype} B={b} Hq={hq} Hkv={hkv} Sq={sq} Skv={skv} D={d} {kw}", flush=True)
        cpu, kw2, (o_ws, l_ws), (o_na, l_na) = _decode_both(lib, dtype, b, hq, hkv, sq, skv, d, kw, seed=70 + i)
        assert torch.equal(o_na, o_ws), f"call {i}: O differs from flexatt_fwd_decode"
        assert torch.equal(l_na, l_ws), f"call {i}: LSE differs from flexatt_fwd_decode"
        ref = oracle_fwd_bwd(*cpu, **kw2)
        check("o", o_na, ref[0], dtype)
        check("lse", l_na, ref[1], dtype)
