"""BASELINE configurations 4 and 5 at their full sizes on the GPU, with the
oracle evaluated on one (batch, KV-head) group over query-row chunks
(oracle.forward_backward_rows, pinned in tests/test_oracle.py).

* config 4: bf16 B=1 Hq=16 Hkv=8 S=8192 D=256, causal + window 4096 + tanh
  soft-cap 50, scale 1/16, inputs N(0,1)*2 so the cap saturates;
* config 5: fp16 B=1 Hq=28 Hkv=4 (G=7) D=64, Sq=16384, Skv=16383 (not a tile
  multiple), causal + window 2048 + ALiBi slopes 2^(-8(h+1)/Hq) + soft-cap 30
  + scale 0.05.
"""
import pytest
import torch

import npu_flash_attention as nfa
from gpu_helpers import alibi_slopes, check, draw, fwd_bwd
from oracle import attention_oracle as orc

pytestmark = pytest.mark.gpu

NAMES = ("o", "lse", "dq", "dk", "dv")


def _group_check(tag, dtype, got, cpu, hk, g, kw, slopes=None):
    for x in got:
        assert bool(torch.isfinite(x).all()), f"{tag}: non-finite output"
    hs = slice(hk * g, (hk + 1) * g)
    q, k, v, do = cpu
    ref = orc.forward_backward_rows(q[:, hs], k[:, hk:hk + 1], v[:, hk:hk + 1], do[:, hs],
                                    kw.get("causal", False), kw.get("sliding_window", 0),
                                    None if slopes is None else slopes[hs], kw.get("scale"),
                                    kw.get("soft_cap", 0.0), dtype=torch.float32)
    sel = (got[0][:, hs], got[1][:, hs], got[2][:, hs], got[3][:, hk:hk + 1], got[4][:, hk:hk + 1])
    rep = {}
    for name, x, r in zip(NAMES, sel, ref):
        check(name, x, r, dtype, rep)
    print(f"[{tag}, group (0, {hk})] " + " ".join(f"{k_}={v_:.2e}" for k_, v_ in rep.items()))


C4_KW = dict(causal=True, sliding_window=4096, soft_cap=50.0, scale=1.0 / 16)
C5_KW = dict(causal=True, sliding_window=2048, soft_cap=30.0, scale=0.05)


@pytest.fixture(scope="module")
def config4_full():
    cpu, dev = draw(42, 1, 16, 8, 8192, 8192, 256, torch.bfloat16, scale_inputs=2.0)
    got = fwd_bwd(nfa, *dev, **C4_KW)
    return cpu, [x.cpu() for x in got]


@pytest.fixture(scope="module")
def config5_full():
    slopes = alibi_slopes(28)
    cpu, dev = draw(42, 1, 28, 4, 16384, 16383, 64, torch.float16)
    got = fwd_bwd(nfa, *dev, alibi_slope=slopes.to("cuda"), **C5_KW)
    return cpu, [x.cpu() for x in got], slopes


# two KV heads each, at both ends of the head range (different XCDs)
@pytest.mark.parametrize("hk", [0, 7])
def test_config4_full_size(gpu_device, config4_full, hk):
    cpu, got = config4_full
    _group_check("config4 full", torch.bfloat16, got, cpu, hk=hk, g=2, kw=C4_KW)


@pytest.mark.parametrize("hk", [0, 3])
def test_config5_full_size(gpu_device, config5_full, hk):
    cpu, got, slopes = config5_full
    _group_check("config5 full", torch.float16, got, cpu, hk=hk, g=7, kw=C5_KW, slopes=slopes)
