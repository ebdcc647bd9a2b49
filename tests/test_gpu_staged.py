"""GPU tests of the backward with dS staged through HBM (flexatt_bwd_ws: the
dK/dV kernel writes its rounded dS, the dQ kernel streams dS K), the path
npu_flash_attention_backward takes for fp16/bf16 with head_dim 64, 128 or 256.

* the five outputs against the float64 oracle at the north-star bounds, over
  GQA ratios 1, 2, 3, 4, 7 and 8 (head groups that do not fill a workgroup),
  Sq != Skv, single keys and every mask primitive;
* the staged dS itself, decoded from the workspace, against the oracle's
  P (dP - Delta) (1 - tanh^2);
* the same problem through the recomputing dQ kernel (flexatt_bwd);
* dK/dV of the staging kernel bitwise equal to flexatt_bwd_dkdv, the two
  kernels on their own bitwise equal to flexatt_bwd_ws, and repeat calls
  bitwise equal;
* rows with no allowed key (O = 0, LSE = -inf) give zero gradients.

The default backward stages only where flexatt_bwd_prefers_staging reports
that staging pays (not at head_dim 64 without soft-cap or interval/block
masks); these tests stage wherever the staged range covers the problem
(ds_staging_auto off), so that the head_dim 64 staged kernels stay covered.
"""
import pytest
import torch

import flexatt_lib as L
import npu_flash_attention as nfa
from gpu_helpers import alibi_slopes, check, draw, fwd_bwd, oracle_fwd_bwd
from oracle import attention_oracle as orc

pytestmark = pytest.mark.gpu


@pytest.fixture(autouse=True)
def _stage_wherever_in_range(monkeypatch):
    monkeypatch.setattr(nfa, "ds_staging_auto", False)

# name: (dtype, B, Hq, Hkv, Sq, Skv, kwargs)
CASES = {
    "bf16_g3_causal": (torch.bfloat16, 1, 6, 2, 300, 257, dict(causal=True)),
    "fp16_g7_full_sq_lt_skv": (torch.float16, 1, 7, 1, 200, 333, {}),
    "bf16_g8_causal_window": (torch.bfloat16, 1, 16, 2, 257, 190, dict(causal=True, sliding_window=70)),
    "fp16_g1_window_alibi_cap": (torch.float16, 2, 2, 2, 333, 333,
                                 dict(sliding_window=100, alibi=True, soft_cap=20.0, scale=0.07)),
    "bf16_g4_all": (torch.bfloat16, 1, 8, 2, 1000, 1000,
                    dict(causal=True, sliding_window=300, alibi=True, soft_cap=30.0, scale=0.05)),
    "fp16_g2_one_key": (torch.float16, 1, 4, 2, 65, 1, {}),
    "bf16_g7_causal_sq_gt_skv": (torch.bfloat16, 1, 14, 2, 520, 130, dict(causal=True, scale=-0.08)),
    "fp16_g8_window_long": (torch.float16, 1, 8, 1, 1500, 1600, dict(sliding_window=513)),
    # head_dim 64
    "d64_bf16_g3_causal": (torch.bfloat16, 1, 6, 2, 300, 257, dict(causal=True, d=64)),
    "d64_fp16_g7_all": (torch.float16, 1, 7, 1, 700, 650,
                        dict(causal=True, sliding_window=200, alibi=True, soft_cap=30.0, scale=0.05, d=64)),
    "d64_bf16_g1_full_sq_lt_skv": (torch.bfloat16, 2, 2, 2, 200, 333, dict(d=64)),
    "d64_fp16_g4_window": (torch.float16, 1, 8, 2, 1000, 1000, dict(sliding_window=300, d=64)),
    "d64_fp16_g2_one_key": (torch.float16, 1, 4, 2, 65, 1, dict(d=64)),
    # head_dim 256 (dV and dK in two passes)
    "d256_bf16_g2_causal_window_cap": (torch.bfloat16, 1, 4, 2, 600, 600,
                                       dict(causal=True, sliding_window=300, soft_cap=50.0, scale=1 / 16, d=256)),
    "d256_fp16_g3_all_sq_gt_skv": (torch.float16, 1, 6, 2, 333, 257,
                                   dict(causal=True, alibi=True, soft_cap=20.0, scale=0.05, d=256)),
    "d256_bf16_g1_full": (torch.bfloat16, 2, 2, 2, 200, 300, dict(d=256)),
    "d256_fp16_g8_one_key": (torch.float16, 1, 8, 1, 40, 1, dict(d=256)),
}


def _inputs(case, seed=0):
    dtype, b, hq, hkv, sq, skv, kw = CASES[case]
    kw = dict(kw)
    d = kw.pop("d", 128)
    cpu, dev = draw(seed + 90, b, hq, hkv, sq, skv, d, dtype)
    if kw.pop("alibi", False):
        kw["alibi_slope"] = alibi_slopes(hq).to("cuda")
    return dtype, cpu, dev, kw


def _problem(q, k, kw):
    s = kw.get("scale") or 1.0 / q.shape[-1] ** 0.5
    return nfa._problem(q, k, s, kw.get("causal", False), kw.get("sliding_window", 0), kw.get("soft_cap", 0.0),
                        kw.get("alibi_slope"))


@pytest.mark.parametrize("case", list(CASES))
def test_staged_matches_oracle(gpu_device, case):
    dtype, cpu, (q, k, v, do), kw = _inputs(case)
    assert L.load().flexatt_bwd_workspace(_problem(q, k, kw)) > 0
    got = fwd_bwd(nfa, q, k, v, do, **kw)
    ref = oracle_fwd_bwd(*cpu, **kw)
    for name, x, r in zip(("o", "lse", "dq", "dk", "dv"), got, ref):
        check(name, x, r, dtype)


@pytest.mark.parametrize("case", ["bf16_g3_causal", "fp16_g1_window_alibi_cap", "bf16_g7_causal_sq_gt_skv",
                                  "d64_fp16_g7_all", "d256_fp16_g3_all_sq_gt_skv"])
def test_staged_ds_values(gpu_device, case):
    """Decode the workspace: unit (b, h, t, kb) fragment f, lane l, element e
    holds dS/scale of query row 32 t + l % 32 and KV row
    128 kb + 16 f + 4 (l / 32) + e (+ 4 for e >= 4)."""
    dtype, cpu, (q, k, v, do), kw = _inputs(case)
    lib = L.load()
    B, Hq, Sq, D = q.shape
    Skv = k.shape[2]
    p = _problem(q, k, kw)
    n = lib.flexatt_bwd_workspace(p)
    o, lse = nfa.npu_flash_attention_forward(q, k, v, return_lse=True, **kw)
    delta = torch.empty(B, Hq, Sq, dtype=torch.float32, device=q.device)
    ws = torch.zeros(n, dtype=torch.uint8, device=q.device)
    dk, dv = torch.empty_like(k), torch.empty_like(v)
    st = torch.cuda.current_stream().cuda_stream
    T = L.tensor
    L.check(lib.flexatt_bwd_delta(p, T(o), T(do), delta.data_ptr(), st), "delta")
    L.check(lib.flexatt_bwd_dkdv_ds(p, T(q), T(k), T(v), T(do), lse.data_ptr(), delta.data_ptr(), T(dk), T(dv),
                                    ws.data_ptr(), n, st), "dkdv_ds")
    torch.cuda.synchronize()
    units = ws[: n - L.BWD_QUEUE_BYTES].view(dtype).view(-1, 8, 64, 8).cpu().double()  # [unit, fragment, lane, element]
    causal, window = kw.get("causal", False), kw.get("sliding_window", 0)
    nqt, nkb = -(-Sq // 32), -(-Skv // 128)
    # (t, kb) units of one head in storage order
    order = []
    for t in range(nqt):
        lo = min(nkb, max(0, (32 * t - window) // 128)) if window > 0 else 0
        hi = min(nkb, t // 4 + 1) if causal else nkb
        order += [(t, kb) for kb in range(lo, hi)]
    assert units.shape[0] == B * Hq * len(order)
    ref = orc.score_grad(*cpu, causal=causal, sliding_window=window,
                         alibi_slope=None if kw.get("alibi_slope") is None else kw["alibi_slope"].cpu(),
                         scale=kw.get("scale"), soft_cap=kw.get("soft_cap", 0.0))
    dense = torch.zeros(B, Hq, nqt * 32, nkb * 128, dtype=torch.float64)
    lanes = torch.arange(64)
    el = torch.arange(8)
    row = (lanes % 32).view(64, 1).expand(64, 8)
    col = (4 * (lanes // 32)).view(64, 1) + el.view(1, 8) + 4 * (el.view(1, 8) >= 4)
    for bh in range(B * Hq):
        for u, (t, kb) in enumerate(order):
            blk = units[bh * len(order) + u]  # [8, 64, 8]
            for f in range(8):
                dense[bh // Hq, bh % Hq, 32 * t + row, 128 * kb + 16 * f + col] = blk[f]
    got = dense[:, :, :Sq, :Skv]
    tol = {torch.bfloat16: 2e-2, torch.float16: 5e-3}[dtype]
    scale = max(1.0, ref.abs().max().item())
    e = (got - ref).abs().max().item() / scale
    assert e <= tol, f"staged dS err {e:.3e} > {tol}"


@pytest.mark.parametrize("case", ["bf16_g8_causal_window", "fp16_g7_full_sq_lt_skv", "bf16_g4_all", "d64_fp16_g4_window",
                                  "d256_bf16_g2_causal_window_cap"])
def test_staged_against_recompute_path(gpu_device, case):
    dtype, cpu, (q, k, v, do), kw = _inputs(case)
    o, lse = nfa.npu_flash_attention_forward(q, k, v, return_lse=True, **kw)
    staged = nfa.npu_flash_attention_backward(q, k, v, o, lse, do, **kw)
    nfa.ds_staging_enabled = False
    try:
        recomp = nfa.npu_flash_attention_backward(q, k, v, o, lse, do, **kw)
    finally:
        nfa.ds_staging_enabled = True
    torch.cuda.synchronize()
    # (dK/dV differ in the last bits: the recomputing dQ kernel forms Delta
    # in its own summation order; with one Delta the dK/dV kernels agree
    # bitwise, see test_staged_kernels_and_repeats_bitwise)
    for name, x, r in zip(("dq", "dk", "dv"), staged, recomp):
        check(name, x, r.double(), dtype)


@pytest.mark.parametrize("case", ["bf16_g3_causal", "fp16_g1_window_alibi_cap", "d64_bf16_g3_causal",
                                  "d256_bf16_g1_full"])
def test_staged_kernels_and_repeats_bitwise(gpu_device, case):
    dtype, cpu, (q, k, v, do), kw = _inputs(case)
    lib = L.load()
    B, Hq, Sq, D = q.shape
    p = _problem(q, k, kw)
    n = lib.flexatt_bwd_workspace(p)
    o, lse = nfa.npu_flash_attention_forward(q, k, v, return_lse=True, **kw)
    st = torch.cuda.current_stream().cuda_stream
    T = L.tensor

    def whole():
        delta = torch.empty(B, Hq, Sq, dtype=torch.float32, device=q.device)
        ws = torch.empty(n, dtype=torch.uint8, device=q.device)
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        L.check(lib.flexatt_bwd_ws(p, T(q), T(k), T(v), T(o), T(do), lse.data_ptr(), delta.data_ptr(), T(dq), T(dk),
                                   T(dv), ws.data_ptr(), n, st), "bwd_ws")
        return dq, dk, dv, delta

    def parts():
        delta = torch.empty(B, Hq, Sq, dtype=torch.float32, device=q.device)
        ws = torch.full((n,), 0x7f, dtype=torch.uint8, device=q.device)  # stale contents must not matter
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        dk2, dv2 = torch.empty_like(k), torch.empty_like(v)
        L.check(lib.flexatt_bwd_delta(p, T(o), T(do), delta.data_ptr(), st), "delta")
        L.check(lib.flexatt_bwd_dkdv_ds(p, T(q), T(k), T(v), T(do), lse.data_ptr(), delta.data_ptr(), T(dk), T(dv),
                                        ws.data_ptr(), n, st), "dkdv_ds")
        L.check(lib.flexatt_bwd_dq_ds(p, T(k), ws.data_ptr(), n, T(dq), st), "dq_ds")
        L.check(lib.flexatt_bwd_dkdv(p, T(q), T(k), T(v), T(do), lse.data_ptr(), delta.data_ptr(), T(dk2), T(dv2),
                                     st), "dkdv")
        return dq, dk, dv, delta, dk2, dv2

    a = whole()
    b_ = whole()
    c = parts()
    torch.cuda.synchronize()
    for x, y in zip(a, b_):
        assert torch.equal(x, y), "repeat call differs"
    for x, y in zip(a, c[:4]):
        assert torch.equal(x, y), "separate kernels differ from flexatt_bwd_ws"
    assert torch.equal(c[1], c[4]) and torch.equal(c[2], c[5]), "staging changed dK/dV"


@pytest.mark.parametrize("d", [128, 64, 256])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_staged_fully_masked_rows(gpu_device, dtype, d):
    """Non-causal window W = 30 over Skv = 100 keys: query rows >= 131 see
    none (O = 0, LSE = -inf) and get dQ = 0; the others match the oracle."""
    cpu, (q, k, v, do) = draw(5, 1, 4, 2, 400, 100, d, dtype)
    kw = dict(sliding_window=30)
    o, lse, dq, dk, dv = fwd_bwd(nfa, q, k, v, do, **kw)
    ref = oracle_fwd_bwd(*cpu, **kw)
    assert torch.isneginf(lse[:, :, 131:]).all()
    assert (dq[:, :, 131:] == 0).all() and (o[:, :, 131:] == 0).all()
    for name, x, r in zip(("o", "lse", "dq", "dk", "dv"), (o, lse, dq, dk, dv), ref):
        check(name, x, r, dtype)


# Grids with more workgroups than CUs: flexatt_bwd_ws hands the workgroups
# past the first per CU their work items from the queue counters in the
# workspace (cleared by its Delta pass); the two kernels called on their own
# keep the static order.  Each item is computed the same way wherever it
# runs, so the results are bitwise equal, over repeated calls too.
QUEUE_CASES = {
    "bf16_d128_causal_gqa4": (torch.bfloat16, 128, 2, 32, 8, 4096, dict(causal=True)),
    "bf16_d256_window_cap": (torch.bfloat16, 256, 1, 16, 8, 8192, dict(causal=True, sliding_window=4096,
                                                                       soft_cap=50.0)),
    "fp16_d64_g7_window": (torch.float16, 64, 2, 28, 4, 8192, dict(causal=True, sliding_window=2048)),
}


@pytest.mark.parametrize("case", list(QUEUE_CASES))
def test_work_queue_matches_static_order(gpu_device, case):
    dtype, d, b, hq, hkv, s, kw = QUEUE_CASES[case]
    g = torch.Generator().manual_seed(21)
    q, do = (torch.randn(b, hq, s, d, generator=g).to(dtype).cuda() for _ in range(2))
    k, v = (torch.randn(b, hkv, s, d, generator=g).to(dtype).cuda() for _ in range(2))
    lib = L.load()
    p = _problem(q, k, kw)
    n = lib.flexatt_bwd_workspace(p)
    assert n > L.BWD_QUEUE_BYTES
    o, lse = nfa.npu_flash_attention_forward(q, k, v, return_lse=True, **kw)
    st = torch.cuda.current_stream().cuda_stream
    T = L.tensor

    def run(whole):
        delta = torch.empty(b, hq, s, dtype=torch.float32, device=q.device)
        ws = torch.full((n,), 0x55, dtype=torch.uint8, device=q.device)  # stale counters must not matter
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        if whole:
            L.check(lib.flexatt_bwd_ws(p, T(q), T(k), T(v), T(o), T(do), lse.data_ptr(), delta.data_ptr(), T(dq),
                                       T(dk), T(dv), ws.data_ptr(), n, st), "bwd_ws")
        else:
            L.check(lib.flexatt_bwd_delta(p, T(o), T(do), delta.data_ptr(), st), "delta")
            L.check(lib.flexatt_bwd_dkdv_ds(p, T(q), T(k), T(v), T(do), lse.data_ptr(), delta.data_ptr(), T(dk),
                                            T(dv), ws.data_ptr(), n, st), "dkdv_ds")
            L.check(lib.flexatt_bwd_dq_ds(p, T(k), ws.data_ptr(), n, T(dq), st), "dq_ds")
        torch.cuda.synchronize()
        return dq, dk, dv

    a, b2, c = run(True), run(True), run(False)
    for name, x, y, z in zip(("dq", "dk", "dv"), a, b2, c):
        assert bool(torch.isfinite(x).all()), name
        assert torch.equal(x, y), f"{name}: repeat call differs"
        assert torch.equal(x, z), f"{name}: queue order differs from the static order"
