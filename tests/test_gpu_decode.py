"""GPU tests of the split-KV decode forward (flexatt_fwd_decode), which the
forward takes when (Hq / Hkv) * Sq <= 32 for fp16 / bf16 and D <= 128.

* O and LSE against the oracle over head dims, GQA ratios, query counts, KV
  lengths (one tile, ragged tails, many splits) and every mask primitive;
* against the regular forward kernel on the same inputs (same tolerance: the
  split changes the summation order, not the math);
* bitwise repeatability, and the backward fed by the decode forward's O / LSE.
"""
import pytest
import torch

import flexatt_lib as L
import npu_flash_attention as nfa
from gpu_helpers import alibi_slopes, check, draw, oracle_fwd_bwd

pytestmark = pytest.mark.gpu

# name: (dtype, D, Hq, Hkv, Sq, Skv, kwargs)
CASES = {
    "bf16_d128_g4_sq1_long": (torch.bfloat16, 128, 32, 8, 1, 4113, {}),
    "fp16_d128_g4_sq2_causal": (torch.float16, 128, 8, 2, 2, 1000, dict(causal=True)),
    "bf16_d64_g7_sq4_all": (torch.bfloat16, 64, 28, 4, 4, 2047, dict(sliding_window=300, soft_cap=30.0,
                                                                        alibi=True, scale=0.05)),
    "fp16_d64_mha_sq32_window": (torch.float16, 64, 4, 4, 32, 777, dict(sliding_window=45)),
    "bf16_d32_g8_sq4_cap": (torch.bfloat16, 32, 16, 2, 4, 3001, dict(soft_cap=20.0)),
    "fp16_d32_g1_sq1_tiny": (torch.float16, 32, 2, 2, 1, 1, {}),
    "bf16_d128_g2_sq16_one_tile": (torch.bfloat16, 128, 4, 2, 16, 33, dict(causal=False, scale=-0.1)),
    "fp16_d128_g8_sq4_alibi_causal": (torch.float16, 128, 8, 1, 4, 5000, dict(causal=True, alibi=True)),
    "bf16_d64_g4_sq8_b3": (torch.bfloat16, 64, 8, 2, 8, 9000, {}),
}


def _run(case, seed=0):
    dtype, d, hq, hkv, sq, skv, kw = CASES[case]
    kw = dict(kw)
    b = 3 if case.endswith("_b3") else 1
    cpu, dev = draw(seed + 50, b, hq, hkv, sq, skv, d, dtype)
    if kw.pop("alibi", False):
        kw["alibi_slope"] = alibi_slopes(hq).to("cuda")
    return dtype, cpu, dev, kw


def _uses_decode(q, k, kw):
    s = kw.get("scale") or 1.0 / q.shape[-1] ** 0.5
    p = nfa._problem(q, k, s, kw.get("causal", False), kw.get("sliding_window", 0), kw.get("soft_cap", 0.0),
                     kw.get("alibi_slope"))
    return L.load().flexatt_fwd_decode_workspace(p) > 0


@pytest.mark.parametrize("case", list(CASES))
def test_decode_matches_oracle(gpu_device, case):
    dtype, cpu, (q, k, v, do), kw = _run(case)
    assert _uses_decode(q, k, kw), "case is outside the decode range"
    o, lse = nfa.npu_flash_attention_forward(q, k, v, return_lse=True, **kw)
    torch.cuda.synchronize()
    ref = oracle_fwd_bwd(*cpu, **kw)
    check("o", o, ref[0], dtype)
    check("lse", lse, ref[1], dtype)


@pytest.mark.parametrize("case", ["bf16_d128_g4_sq1_long", "bf16_d64_g7_sq4_all", "fp16_d128_g8_sq4_alibi_causal"])
def test_decode_matches_regular_forward(gpu_device, case):
    dtype, cpu, (q, k, v, do), kw = _run(case, seed=1)
    o, lse = nfa.npu_flash_attention_forward(q, k, v, return_lse=True, **kw)
    nfa.decode_enabled = False
    try:
        o2, lse2 = nfa.npu_flash_attention_forward(q, k, v, return_lse=True, **kw)
    finally:
        nfa.decode_enabled = True
    torch.cuda.synchronize()
    check("o", o, o2.float(), dtype)
    check("lse", lse, lse2, dtype)


def test_decode_bitwise_repeatable(gpu_device):
    _, _, (q, k, v, _), kw = _run("bf16_d64_g7_sq4_all", seed=2)
    a = nfa.npu_flash_attention_forward(q, k, v, return_lse=True, **kw)
    b = nfa.npu_flash_attention_forward(q, k, v, return_lse=True, **kw)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_backward_after_decode_forward(gpu_device):
    dtype, cpu, (q, k, v, do), kw = _run("fp16_d128_g4_sq2_causal", seed=3)
    o, lse = nfa.npu_flash_attention_forward(q, k, v, return_lse=True, **kw)
    dq, dk, dv = nfa.npu_flash_attention_backward(q, k, v, o, lse, do, **kw)
    torch.cuda.synchronize()
    ref = oracle_fwd_bwd(*cpu, **kw)
    for name, x, r in zip(("dq", "dk", "dv"), (dq, dk, dv), ref[2:]):
        check(name, x, r, dtype)
