"""GPU tests of the API contract and of the BASELINE configurations.

* bitwise determinism of repeated calls (reference tests R06, R11);
* strided inputs: [B, S, H, D] storage viewed as [B, H, S, D] (R01-R03) and
  K / V broadcast over the batch with stride 0 (S09), against the contiguous
  run, bitwise;
* the autograd entry point (npu_flex_attention) and flex_attention with an
  AttentionConfig, against the direct forward / backward calls, bitwise;
* BASELINE.json configs 2 (all sequence lengths), 4 and 5 (reduced sequence
  lengths, every other parameter as specified) against the oracle, and
  config 3 at full size with the oracle evaluated on one (batch, KV-head)
  group.
"""
import pytest
import torch

import npu_flash_attention as nfa
from gpu_helpers import alibi_slopes, check, draw, fwd_bwd, oracle_fwd_bwd
from oracle import attention_oracle as orc

pytestmark = pytest.mark.gpu

NAMES = ("o", "lse", "dq", "dk", "dv")

REPEAT_CASES = {
    "bf16_d128_causal_gqa": (torch.bfloat16, 128, 8, 2, dict(causal=True)),
    "fp16_d64_all": (torch.float16, 64, 7, 1, dict(causal=True, sliding_window=61, soft_cap=20.0, scale=0.07)),
    "bf16_d256_window": (torch.bfloat16, 256, 4, 4, dict(causal=False, sliding_window=45)),
}


@pytest.mark.parametrize("case", list(REPEAT_CASES))
def test_bitwise_repeatable(gpu_device, case):
    dtype, d, hq, hkv, kw = REPEAT_CASES[case]
    _, dev = draw(21, 2, hq, hkv, 333, 301, d, dtype)
    first = fwd_bwd(nfa, *dev, **kw)
    second = fwd_bwd(nfa, *dev, **kw)
    for name, x, y in zip(NAMES, first, second):
        assert torch.equal(x, y), f"{case}: {name} differs between two identical calls"


def _bsnd_view(x):
    """Same values, stored as [B, S, H, D] and viewed as [B, H, S, D]."""
    return x.transpose(1, 2).contiguous().transpose(1, 2)


@pytest.mark.parametrize("dtype,d", [(torch.bfloat16, 128), (torch.float16, 64)], ids=["bf16_d128", "fp16_d64"])
def test_bsnd_views_match_contiguous(gpu_device, dtype, d):
    _, (q, k, v, do) = draw(22, 2, 4, 2, 257, 250, d, dtype)
    views = [_bsnd_view(t) for t in (q, k, v, do)]
    assert not views[0].is_contiguous() and views[0].stride(2) == 4 * d
    ref = fwd_bwd(nfa, q, k, v, do, causal=True, sliding_window=100)
    got = fwd_bwd(nfa, *views, causal=True, sliding_window=100)
    for name, x, y in zip(NAMES, got, ref):
        assert torch.equal(x.contiguous(), y), f"{name}: strided result differs"


def test_kv_broadcast_over_batch(gpu_device):
    _, (q, k, v, do) = draw(23, 3, 4, 2, 130, 130, 64, torch.bfloat16)
    kb = k[:1].expand(3, -1, -1, -1)
    vb = v[:1].expand(3, -1, -1, -1)
    assert kb.stride(0) == 0
    ref = fwd_bwd(nfa, q, kb.contiguous(), vb.contiguous(), do, causal=True)
    got = fwd_bwd(nfa, q, kb, vb, do, causal=True)
    for name, x, y in zip(NAMES, got, ref):
        assert torch.equal(x, y), f"{name}: broadcast result differs"


def test_autograd_matches_direct(gpu_device):
    _, (q, k, v, do) = draw(24, 1, 8, 2, 300, 280, 128, torch.bfloat16)
    kw = dict(causal=True, sliding_window=90, soft_cap=15.0)
    o_ref, lse = nfa.npu_flash_attention_forward(q, k, v, return_lse=True, **kw)
    dq_ref, dk_ref, dv_ref = nfa.npu_flash_attention_backward(q, k, v, o_ref, lse, do, **kw)
    qa, ka, va = (t.clone().requires_grad_(True) for t in (q, k, v))
    o = nfa.npu_flex_attention(qa, ka, va, True, 90, None, None, 16, 64, 15.0)
    o.backward(do)
    assert torch.equal(o.detach(), o_ref)
    for name, g, r in (("dq", qa.grad, dq_ref), ("dk", ka.grad, dk_ref), ("dv", va.grad, dv_ref)):
        assert torch.equal(g, r), f"{name}: autograd result differs from the direct backward"


def test_flex_attention_config(gpu_device):
    _, (q, k, v, _) = draw(25, 2, 6, 3, 190, 200, 64, torch.float16)
    cfg = nfa.AttentionConfig(causal=True, sliding_window=33, soft_cap=7.0, scale=0.11)
    got = nfa.flex_attention(q, k, v, cfg)
    ref = nfa.npu_flash_attention_forward(q, k, v, causal=True, sliding_window=33, soft_cap=7.0, scale=0.11)
    assert torch.equal(got, ref)
    got_kw = nfa.flex_attention(q, k, v, causal=True, sliding_window=33, soft_cap=7.0, scale=0.11)
    assert torch.equal(got_kw, ref)


# ------------------------------------------------------ BASELINE configurations --
@pytest.mark.parametrize("s", [128, 512, 1024, 2048])
def test_config2_mha_fp16(gpu_device, s):
    """fp16, B=1 H=2 D=64, causal."""
    cpu, dev = draw(42, 1, 2, 2, s, s, 64, torch.float16)
    got = fwd_bwd(nfa, *dev, causal=True)
    ref = oracle_fwd_bwd(*cpu, causal=True)
    rep = {}
    for name, x, r in zip(NAMES, got, ref):
        check(name, x, r, torch.float16, rep)
    print(f"[config2 S={s}] " + " ".join(f"{k}={v:.2e}" for k, v in rep.items()))


def test_config4_d256_reduced(gpu_device):
    """configs[3] at S=1024: bf16, Hq=16 Hkv=8 D=256, causal, W=512, cap=50, scale=1/16, inputs x2."""
    cpu, dev = draw(42, 1, 16, 8, 1024, 1024, 256, torch.bfloat16, scale_inputs=2.0)
    kw = dict(causal=True, sliding_window=512, soft_cap=50.0, scale=1.0 / 16)
    got = fwd_bwd(nfa, *dev, **kw)
    ref = oracle_fwd_bwd(*cpu, dtype=torch.float32, **kw)
    rep = {}
    for name, x, r in zip(NAMES, got, ref):
        check(name, x, r, torch.bfloat16, rep)
    print("[config4 S=1024] " + " ".join(f"{k}={v:.2e}" for k, v in rep.items()))


def test_config5_gqa7_reduced(gpu_device):
    """configs[4] at Sq=2049, Skv=2048: fp16, Hq=28 Hkv=4 (G=7) D=64, causal, W=512, ALiBi, cap=30, scale=0.05."""
    cpu, dev = draw(42, 1, 28, 4, 2049, 2048, 64, torch.float16)
    slopes = alibi_slopes(28)
    kw = dict(causal=True, sliding_window=512, soft_cap=30.0, scale=0.05)
    got = fwd_bwd(nfa, *dev, alibi_slope=slopes.to(gpu_device), **kw)
    ref = oracle_fwd_bwd(*cpu, alibi_slope=slopes, dtype=torch.float32, **kw)
    rep = {}
    for name, x, r in zip(NAMES, got, ref):
        check(name, x, r, torch.float16, rep)
    print("[config5 Sq=2049] " + " ".join(f"{k}={v:.2e}" for k, v in rep.items()))


@pytest.fixture(scope="module")
def config3_full():
    """configs[2], the bench workload, at full size: bf16 B=2 Hq=32 Hkv=8
    S=4096 D=128 causal, the whole problem on the GPU (outputs moved to the
    CPU once for every group check)."""
    cpu, dev = draw(42, 2, 32, 8, 4096, 4096, 128, torch.bfloat16)
    got = fwd_bwd(nfa, *dev, causal=True)
    for x in got:
        assert bool(torch.isfinite(x).all())
    return cpu, [x.cpu() for x in got]


# (batch, KV head) groups spread over the grid: the work order gives each XCD
# two whole groups (flexatt_device.h xcd_lpt_item), so these land on
# different XCDs and in both batches
@pytest.mark.parametrize("bi,hk", [(0, 0), (0, 7), (1, 0), (1, 5), (1, 7)])
def test_config3_full_size(gpu_device, config3_full, bi, hk):
    """The oracle checks one (batch, KV-head) group of the full-size run."""
    cpu, got = config3_full
    g = 4
    hs = slice(hk * g, (hk + 1) * g)
    part = [t[bi:bi + 1, hs] if t.shape[1] == 32 else t[bi:bi + 1, hk:hk + 1] for t in cpu]
    ref = orc.forward_backward_chunked(*part, causal=True, dtype=torch.float32)[0][2:]
    sel = (got[0][bi:bi + 1, hs], got[1][bi:bi + 1, hs], got[2][bi:bi + 1, hs],
           got[3][bi:bi + 1, hk:hk + 1], got[4][bi:bi + 1, hk:hk + 1])
    rep = {}
    for name, x, r in zip(NAMES, sel, ref):
        check(name, x, r, torch.bfloat16, rep)
    print(f"[config3 full, group ({bi}, {hk})] " + " ".join(f"{k}={v:.2e}" for k, v in rep.items()))
