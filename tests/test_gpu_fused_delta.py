"""GPU tests of flexatt_bwd_dq_delta, the entry point that forms Delta inside
the dQ kernel (D = 64 and 128 fp16/bf16) instead of in a separate pass.

Against the separate passes (flexatt_bwd_delta, then flexatt_bwd_dq) on the
same inputs: Delta agrees to fp32 summation-order rounding, dQ within the
dtype's dQ tolerance (the two differ only through that rounding), and the
problems outside the fused range (another head dim) take the separate passes,
bitwise.  Oracle parity of the whole backward through this entry point is in
the backward tests of test_gpu_parity.py, which run npu_flash_attention_backward
(flexatt_bwd calls flexatt_bwd_dq_delta).
"""
import math

import pytest
import torch

import flexatt_lib as L
import npu_flash_attention as nfa
from gpu_helpers import alibi_slopes, check, draw

pytestmark = pytest.mark.gpu

CASES = {
    "bf16_d128_causal_gqa": (torch.bfloat16, 128, 8, 2, 300, 300, dict(causal=True)),
    "fp16_d128_all": (torch.float16, 128, 8, 4, 333, 257,
                      dict(causal=True, sliding_window=97, soft_cap=20.0, scale=0.06, alibi=True)),
    "bf16_d128_noncausal_ragged": (torch.bfloat16, 128, 4, 4, 129, 77, dict(causal=False)),
    "fp16_d64_window_gqa": (torch.float16, 64, 6, 2, 261, 300, dict(causal=True, sliding_window=70)),
    "bf16_d32_separate": (torch.bfloat16, 32, 8, 2, 200, 150, dict(causal=True)),
}


def run_both(dtype, d, hq, hkv, sq, skv, kw):
    _, (q, k, v, do) = draw(5, 2, hq, hkv, sq, skv, d, dtype)
    slopes = alibi_slopes(hq).to(q.device) if kw.get("alibi") else None
    scale = kw.get("scale") or 1.0 / math.sqrt(d)
    fkw = dict(causal=kw.get("causal", False), sliding_window=kw.get("sliding_window", 0),
               soft_cap=kw.get("soft_cap", 0.0), scale=scale, alibi_slope=slopes)
    o, lse = nfa.npu_flash_attention_forward(q, k, v, return_lse=True, **fkw)
    lib = L.load()
    p = nfa._problem(q, k, scale, fkw["causal"], fkw["sliding_window"], fkw["soft_cap"], slopes)
    st = torch.cuda.current_stream(q.device).cuda_stream
    T = L.tensor
    delta_s = torch.empty(2, hq, sq, dtype=torch.float32, device=q.device)
    delta_f = torch.full_like(delta_s, float("nan"))
    dq_s, dq_f = torch.empty_like(q), torch.empty_like(q)
    L.check(lib.flexatt_bwd_delta(p, T(o), T(do), delta_s.data_ptr(), st), "delta")
    L.check(lib.flexatt_bwd_dq(p, T(q), T(k), T(v), T(do), lse.data_ptr(), delta_s.data_ptr(), T(dq_s), st), "dq")
    L.check(lib.flexatt_bwd_dq_delta(p, T(q), T(k), T(v), T(o), T(do), lse.data_ptr(), delta_f.data_ptr(),
                                     T(dq_f), st), "dq_delta")
    torch.cuda.synchronize()
    return o, do, delta_s, delta_f, dq_s, dq_f


@pytest.mark.parametrize("case", list(CASES))
def test_fused_delta_matches_separate_passes(gpu_device, case):
    dtype, d, hq, hkv, sq, skv, kw = CASES[case]
    o, do, delta_s, delta_f, dq_s, dq_f = run_both(dtype, d, hq, hkv, sq, skv, kw)
    assert torch.isfinite(delta_f).all(), "every Delta entry is written"
    # Delta against the float64 sum of the same O and dO
    ref = (o.double() * do.double()).sum(-1)
    scale = max(1.0, ref.abs().max().item())
    assert (delta_f.double() - ref).abs().max().item() <= 1e-5 * scale
    assert (delta_s.double() - ref).abs().max().item() <= 1e-5 * scale
    if d in (64, 128):
        check("dq", dq_f.float(), dq_s.float(), dtype)
    else:  # outside the fused range: the separate passes, bitwise
        assert torch.equal(delta_f, delta_s)
        assert torch.equal(dq_f, dq_s)


def test_fused_delta_repeatable(gpu_device):
    first = run_both(*CASES["bf16_d128_causal_gqa"])
    second = run_both(*CASES["bf16_d128_causal_gqa"])
    assert torch.equal(first[3], second[3]) and torch.equal(first[5], second[5])
