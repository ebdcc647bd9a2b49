"""GPU parity of the HIP kernels against the CPU oracle over the primitive grid.

Every dtype x head dim x mask combination, with GQA, Sq != Skv and a KV
length that is not a tile multiple, forward (O, LSE) and backward
(dQ, dK, dV), through the public API (and so through the C ABI).
"""
import os

import numpy as np
import pytest
import torch

import npu_flash_attention as nfa
from gpu_helpers import TOL, alibi_slopes, check, draw, fp32_score_factor, fwd_bwd, oracle_fwd_bwd

pytestmark = pytest.mark.gpu

DTYPES = [torch.bfloat16, torch.float16, torch.float32]
HEAD_DIMS = [32, 64, 128, 256]
# name: (causal, window, alibi, soft_cap, scale)
FLAGS = {
    "full": (False, 0, False, 0.0, None),
    "causal": (True, 0, False, 0.0, None),
    "causal_window": (True, 37, False, 0.0, None),
    "window": (False, 29, False, 0.0, 0.09),
    "causal_alibi_cap": (True, 0, True, 5.0, None),
    "all": (True, 41, True, 3.0, 0.05),
}


@pytest.mark.parametrize("flags", list(FLAGS))
@pytest.mark.parametrize("d", HEAD_DIMS)
@pytest.mark.parametrize("dtype", DTYPES, ids=["bf16", "fp16", "fp32"])
def test_primitive_grid(gpu_device, dtype, d, flags):
    causal, window, alibi, cap, scale = FLAGS[flags]
    b, hq, hkv, sq, skv = 2, 4, 2, 200, 173
    cpu, dev = draw(11, b, hq, hkv, sq, skv, d, dtype)
    slopes = alibi_slopes(hq) if alibi else None
    kw = dict(causal=causal, sliding_window=window, soft_cap=cap, scale=scale,
              alibi_slope=None if slopes is None else slopes.to(gpu_device))
    got = fwd_bwd(nfa, *dev, **kw)
    ref = oracle_fwd_bwd(*cpu, causal=causal, sliding_window=window, alibi_slope=slopes, scale=scale, soft_cap=cap)
    rep = {}
    for name, x, r in zip(("o", "lse", "dq", "dk", "dv"), got, ref):
        check(name, x, r, dtype, rep)
    print(f"[grid] {dtype} D={d} {flags}: " + " ".join(f"{k}={v:.2e}" for k, v in rep.items()))


GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "attention_golden.npz")


@pytest.fixture(scope="module")
def gold():
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def test_golden_config1_fp32(gpu_device, gold):
    q, k, v, do = (torch.from_numpy(gold[f"config1/{n}"]).to(gpu_device) for n in ("q", "k", "v", "do"))
    got = fwd_bwd(nfa, q, k, v, do, causal=True)
    for name, x in zip(("o", "lse", "dq", "dk", "dv"), got):
        check(name, x, torch.from_numpy(gold[f"config1/{name}"]), torch.float32)


@pytest.mark.parametrize("name", ["combo_full", "combo_causal", "combo_causal_window", "combo_window_noncausal",
                                  "combo_causal_alibi_cap", "combo_all"])
def test_golden_combos_fp32(gpu_device, gold, name):
    q, k, v, do, slopes = (torch.from_numpy(gold[f"combo/{n}"]).to(gpu_device)
                           for n in ("q", "k", "v", "do", "alibi"))
    causal, window, alibi, cap, scale = gold[f"{name}/flags"].tolist()
    got = fwd_bwd(nfa, q, k, v, do, causal=bool(causal), sliding_window=int(window),
                  alibi_slope=slopes if alibi else None, soft_cap=cap, scale=None if scale < 0 else scale)
    for nm, x in zip(("o", "lse", "dq", "dk", "dv"), got):
        check(nm, x, torch.from_numpy(gold[f"{name}/{nm}"]), torch.float32)


@pytest.mark.parametrize("dtype", DTYPES, ids=["bf16", "fp16", "fp32"])
@pytest.mark.parametrize("sq,skv", [(1, 1), (16, 16), (33, 33), (65, 47), (47, 300), (300, 47), (129, 127)])
def test_ragged_lengths(gpu_device, dtype, sq, skv):
    cpu, dev = draw(5, 1, 2, 1, sq, skv, 64, dtype)
    for causal, window in ((True, 0), (False, 0), (True, 9), (False, 9)):
        got = fwd_bwd(nfa, *dev, causal=causal, sliding_window=window)
        ref = oracle_fwd_bwd(*cpu, causal=causal, sliding_window=window)
        for name, x, r in zip(("o", "lse", "dq", "dk", "dv"), got, ref):
            check(name, x, r, dtype)


@pytest.mark.parametrize("flags", ["full", "causal", "causal_window", "window"])
@pytest.mark.parametrize("d", HEAD_DIMS)
def test_fp32_several_tiles(gpu_device, d, flags):
    # fp32 matrix-core kernels over several work items per head (the forward
    # takes 256 query rows per workgroup, dQ and dK/dV 128 or 256 rows), G = 3,
    # Sq != Skv, lengths off the tile grid.
    causal, window, alibi, cap, scale = FLAGS[flags]
    window = 90 if window else 0
    cpu, dev = draw(17, 1, 6, 2, 600, 563, d, torch.float32)
    kw = dict(causal=causal, sliding_window=window, scale=scale)
    got = fwd_bwd(nfa, *dev, **kw)
    ref = oracle_fwd_bwd(*cpu, causal=causal, sliding_window=window, scale=scale)
    for name, x, r in zip(("o", "lse", "dq", "dk", "dv"), got, ref):
        check(name, x, r, torch.float32)


@pytest.mark.parametrize("flags", ["causal", "window", "causal_alibi_cap", "all"])
@pytest.mark.parametrize("d", HEAD_DIMS)
def test_fp32_recompute_path(gpu_device, d, flags):
    # The fp32 backward without a dS workspace (flexatt_bwd: dQ recomputes S
    # and dP with 16 query rows per wave, dK/dV without dS stores), which the
    # staged default never runs: G = 3, B = 2, Sq != Skv off the tile grid,
    # several work items per head.
    causal, window, alibi, cap, scale = FLAGS[flags]
    window = 70 if window else 0
    cpu, dev = draw(31, 2, 6, 2, 300, 277, d, torch.float32)
    slopes = alibi_slopes(6) if alibi else None
    kw = dict(causal=causal, sliding_window=window, soft_cap=cap, scale=scale)
    nfa.ds_staging_enabled = False
    try:
        got = fwd_bwd(nfa, *dev, alibi_slope=None if slopes is None else slopes.to(gpu_device), **kw)
    finally:
        nfa.ds_staging_enabled = True
    ref = oracle_fwd_bwd(*cpu, alibi_slope=slopes, **kw)
    for name, x, r in zip(("o", "lse", "dq", "dk", "dv"), got, ref):
        check(name, x, r, torch.float32)


@pytest.mark.parametrize("flags", ["full", "causal", "window", "causal_alibi_cap", "all"])
@pytest.mark.parametrize("d", [64, 128])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_recompute_path_16bit(gpu_device, dtype, d, flags):
    # The fp16/bf16 backward without a dS workspace (flexatt_bwd: the query-
    # stationary dQ kernel that recomputes S and dP and forms Delta itself,
    # then dK/dV without dS stores), which the staged default runs only when
    # even one (batch, KV-head) group's band exceeds the workspace budget:
    # G = 3, B = 2, Sq != Skv off the tile grid, several work items per head.
    causal, window, alibi, cap, scale = FLAGS[flags]
    window = 70 if window else 0
    cpu, dev = draw(37, 2, 6, 2, 300, 277, d, dtype)
    slopes = alibi_slopes(6) if alibi else None
    kw = dict(causal=causal, sliding_window=window, soft_cap=cap, scale=scale)
    nfa.ds_staging_enabled = False
    try:
        got = fwd_bwd(nfa, *dev, alibi_slope=None if slopes is None else slopes.to(gpu_device), **kw)
    finally:
        nfa.ds_staging_enabled = True
    ref = oracle_fwd_bwd(*cpu, alibi_slope=slopes, **kw)
    for name, x, r in zip(("o", "lse", "dq", "dk", "dv"), got, ref):
        check(name, x, r, dtype)


@pytest.mark.parametrize("case", ["bf16_g8_causal_window", "fp16_g3_alibi_noncausal"])
def test_d256_head_groups(gpu_device, case):
    # The D = 256 forward's wave pairs pack gp = min(G & -G, 4) heads per
    # workgroup: G = 8 gives four heads of 32 rows each and two workgroups
    # per group, G = 3 one head of 128 rows and three; Sq != Skv, lengths off
    # the tile grid, several work items per head; the two-pass backward too.
    dtype, hq, hkv, sq, skv, kw = {
        "bf16_g8_causal_window": (torch.bfloat16, 8, 1, 150, 333, dict(causal=True, sliding_window=70)),
        "fp16_g3_alibi_noncausal": (torch.float16, 6, 2, 300, 217, dict(causal=False, alibi=True, scale=0.05)),
    }[case]
    cpu, dev = draw(29, 2, hq, hkv, sq, skv, 256, dtype)
    slopes = alibi_slopes(hq) if kw.pop("alibi", False) else None
    got = fwd_bwd(nfa, *dev, alibi_slope=slopes.to(gpu_device) if slopes is not None else None, **kw)
    ref = oracle_fwd_bwd(*cpu, alibi_slope=slopes, **kw)
    for name, x, r in zip(("o", "lse", "dq", "dk", "dv"), got, ref):
        check(name, x, r, dtype)


@pytest.mark.parametrize("dtype", DTYPES, ids=["bf16", "fp16", "fp32"])
def test_relative_position_score_mod(gpu_device, dtype):
    # FlexAttention's relative-position score_mod, score + (q_idx - kv_idx),
    # is ALiBi with slope 1 in this API's sign convention (+slope * (i - j)).
    # 96 positions: the bias reaches 95, where an fp32 score carries a rounding
    # error of half an ulp (3.8e-6) -- any fp32 softmax over scores of a few
    # hundred exceeds the 1e-5 bound on O by its input rounding alone.
    hq = 4
    cpu, dev = draw(23, 1, hq, 2, 96, 96, 64, dtype)
    ones = torch.ones(hq, dtype=torch.float32)
    for causal, window in ((True, 0), (False, 0), (True, 20)):
        got = fwd_bwd(nfa, *dev, causal=causal, sliding_window=window, scale=0.1, alibi_slope=ones.to(gpu_device))
        ref = oracle_fwd_bwd(*cpu, causal=causal, sliding_window=window, scale=0.1, alibi_slope=ones)
        for name, x, r in zip(("o", "lse", "dq", "dk", "dv"), got, ref):
            check(name, x, r, dtype)


def test_relative_position_long_fp32(gpu_device):
    # The same score_mod over 600 positions: the bias reaches 599, and the
    # fp32 bound scales with the largest attended score (fp32_score_factor):
    # exp(x - m) inherits the half-ulp rounding of a score x, which grows
    # with |x|.
    hq = 4
    cpu, dev = draw(24, 1, hq, 2, 600, 600, 64, torch.float32)
    ones = torch.ones(hq, dtype=torch.float32)
    for causal, window in ((True, 0), (False, 0)):
        got = fwd_bwd(nfa, *dev, causal=causal, sliding_window=window, scale=0.1, alibi_slope=ones.to(gpu_device))
        ref = oracle_fwd_bwd(*cpu, causal=causal, sliding_window=window, scale=0.1, alibi_slope=ones)
        f = fp32_score_factor(cpu[0], cpu[1], scale=0.1, alibi_slope=ones, causal=causal, sliding_window=window)
        assert f > 5.0
        for name, x, r in zip(("o", "lse", "dq", "dk", "dv"), got, ref):
            check(name, x, r, torch.float32, factor=f)


def test_fully_masked_rows(gpu_device):
    # Sq > Skv with a window: rows past Skv-1+W see no key -> O=0, LSE=-inf, finite grads.
    cpu, dev = draw(6, 1, 2, 2, 150, 40, 64, torch.bfloat16)
    got = fwd_bwd(nfa, *dev, causal=True, sliding_window=10)
    ref = oracle_fwd_bwd(*cpu, causal=True, sliding_window=10)
    assert torch.all(torch.isneginf(got[1][0, :, 50:].cpu()))
    assert torch.all(got[0][0, :, 50:].float().cpu() == 0)
    for name, x, r in zip(("o", "lse", "dq", "dk", "dv"), got, ref):
        check(name, x, r, torch.bfloat16)
