"""Write tests/golden/attention_golden.npz from the CPU oracle.

The reference stores no golden vectors (its tests compare against on-device
eager math on the fly), so these fixtures are produced by this repository's
float64 oracle (oracle/attention_oracle.py) on seeded CPU inputs and serve as
fixed anchors for the GPU parity tests and as a regression check of the
oracle itself.  Inputs are drawn with torch.Generator().manual_seed(seed) as
fp32 N(0,1) in the order q, k, v, dO (the reference's backward seed 42,
test/test_comprehensive.py:272).

Cases
  config1      B=1 H=1 S=128 D=64 fp32, causal, default scale
  combo_*      B=1 Hq=4 Hkv=2 Sq=19 Skv=17 D=32 with mask-primitive
               combinations, including a KV length that is not a tile multiple
               and Sq != Skv.

Run: python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import attention_oracle as orc  # noqa: E402

OUT = os.path.join(HERE, "attention_golden.npz")

COMBOS = {
    # name: (causal, window, alibi, soft_cap, scale)
    "combo_full": (False, 0, False, 0.0, None),
    "combo_causal": (True, 0, False, 0.0, None),
    "combo_causal_window": (True, 5, False, 0.0, None),
    "combo_window_noncausal": (False, 4, False, 0.0, 0.3),
    "combo_causal_alibi_cap": (True, 0, True, 2.5, 0.4),
    "combo_all": (True, 6, True, 1.5, 0.25),
}


def inputs(seed, b, hq, hkv, sq, skv, d):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(b, hq, sq, d, generator=g)
    k = torch.randn(b, hkv, skv, d, generator=g)
    v = torch.randn(b, hkv, skv, d, generator=g)
    do = torch.randn(b, hq, sq, d, generator=g)
    return q, k, v, do


def case(prefix, q, k, v, do, causal, window, alibi, cap, scale, arrays):
    o, lse = orc.forward(q, k, v, causal, window, alibi, scale, cap)
    dq, dk, dv = orc.backward(q, k, v, do, causal, window, alibi, scale, cap)
    for name, t in (("o", o), ("lse", lse), ("dq", dq), ("dk", dk), ("dv", dv)):
        arrays[f"{prefix}/{name}"] = t.to(torch.float32).numpy()


def main():
    arrays = {}
    q, k, v, do = inputs(42, 1, 1, 1, 128, 128, 64)
    for name, t in (("q", q), ("k", k), ("v", v), ("do", do)):
        arrays[f"config1/{name}"] = t.numpy()
    case("config1", q, k, v, do, True, 0, None, 0.0, None, arrays)

    q, k, v, do = inputs(7, 1, 4, 2, 19, 17, 32)
    slopes = torch.tensor([0.5, 0.25, 0.125, 0.0625], dtype=torch.float32)
    for name, t in (("q", q), ("k", k), ("v", v), ("do", do), ("alibi", slopes)):
        arrays[f"combo/{name}"] = t.numpy()
    for name, (causal, window, alibi, cap, scale) in COMBOS.items():
        arrays[f"{name}/flags"] = np.array(
            [int(causal), window, int(alibi), cap, -1.0 if scale is None else scale], dtype=np.float64)
        case(name, q, k, v, do, causal, window, slopes if alibi else None, cap, scale, arrays)
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes, {len(arrays)} arrays)")


if __name__ == "__main__":
    main()
