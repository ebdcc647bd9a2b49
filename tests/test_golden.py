"""The committed fixtures (tests/golden/attention_golden.npz) still equal what
the oracle computes — CPU only.  The fixtures anchor the GPU parity tests, so a
change to the oracle that moved them would show up here first."""
import os

import numpy as np
import pytest
import torch

from oracle import attention_oracle as orc

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "attention_golden.npz")
COMBOS = ["combo_full", "combo_causal", "combo_causal_window", "combo_window_noncausal",
          "combo_causal_alibi_cap", "combo_all"]


@pytest.fixture(scope="module")
def gold():
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def t(a):
    return torch.from_numpy(np.asarray(a))


def test_config1_inputs_are_the_seeded_draws(gold):
    g = torch.Generator().manual_seed(42)
    for name, shape in (("q", (1, 1, 128, 64)), ("k", (1, 1, 128, 64)), ("v", (1, 1, 128, 64)), ("do", (1, 1, 128, 64))):
        assert torch.equal(t(gold[f"config1/{name}"]), torch.randn(*shape, generator=g))


def test_config1_matches_oracle(gold):
    q, k, v, do = (t(gold[f"config1/{n}"]) for n in ("q", "k", "v", "do"))
    o, lse = orc.forward(q, k, v, causal=True)
    dq, dk, dv = orc.backward(q, k, v, do, causal=True)
    for name, x in (("o", o), ("lse", lse), ("dq", dq), ("dk", dk), ("dv", dv)):
        assert torch.allclose(x.float(), t(gold[f"config1/{name}"]), rtol=1e-6, atol=1e-6), name


@pytest.mark.parametrize("name", COMBOS)
def test_combo_matches_oracle(gold, name):
    q, k, v, do, slopes = (t(gold[f"combo/{n}"]) for n in ("q", "k", "v", "do", "alibi"))
    causal, window, alibi, cap, scale = gold[f"{name}/flags"].tolist()
    scale = None if scale < 0 else scale
    sl = slopes if alibi else None
    o, lse = orc.forward(q, k, v, bool(causal), int(window), sl, scale, cap)
    dq, dk, dv = orc.backward(q, k, v, do, bool(causal), int(window), sl, scale, cap)
    for nm, x in (("o", o), ("lse", lse), ("dq", dq), ("dk", dk), ("dv", dv)):
        assert torch.allclose(x.float(), t(gold[f"{name}/{nm}"]), rtol=1e-6, atol=1e-6), nm
