"""Pins of the CPU oracle (oracle/attention_oracle.py) — CPU only.

Each check is independent of the oracle's own vectorised formulas:
  * library routine: torch's scaled_dot_product_attention (causal/full/scale);
  * the reference tests' per-row sliding-window loop
    (test/test_comprehensive.py:63-73) and logsumexp LSE
    (test/test_real_world.py:183-199);
  * scalar brute force (math.exp / math.tanh loops) over every primitive
    combination, Sq != Skv and GQA;
  * finite differences (torch.autograd.gradcheck) for the backward;
  * closed forms: V=0, Q=0, S=1, dV = P^T dO, the Delta identity, GQA as
    expanded MHA, degenerate primitives;
  * planted mistakes: wrong variants of the oracle fail the brute-force check.
"""
import itertools
import math

import pytest
import torch
import torch.nn.functional as F

from oracle import attention_oracle as orc



@pytest.fixture(autouse=True)
def _float64_default():
    old = torch.get_default_dtype()
    torch.set_default_dtype(torch.float64)
    yield
    torch.set_default_dtype(old)


def rnd(*shape, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g, dtype=torch.float64)


# ------------------------------------------------------------------ brute force --
def brute_forward(q, k, v, causal, window, slopes, scale, cap):
    """Scalar loops over (b, h, i, j) with the reference's score order
    (npu_flash_attention.py:102-109, :138-141)."""
    b, hq, sq, d = q.shape
    hkv, skv = k.shape[1], k.shape[2]
    g = hq // hkv
    if scale is None:
        scale = 1.0 / math.sqrt(d)
    o = torch.zeros(b, hq, sq, d)
    lse = torch.zeros(b, hq, sq)
    for bi in range(b):
        for h in range(hq):
            kh = h // g
            for i in range(sq):
                xs = []
                for j in range(skv):
                    if causal and j > i:
                        continue
                    if window > 0 and i - j > window:
                        continue
                    x = scale * float(sum(q[bi, h, i, t] * k[bi, kh, j, t] for t in range(d)))
                    if cap > 0:
                        x = cap * math.tanh(x / cap)
                    if slopes is not None:
                        x += float(slopes[h]) * (i - j)
                    xs.append((j, x))
                if not xs:
                    lse[bi, h, i] = float("-inf")
                    continue
                mx = max(x for _, x in xs)
                den = sum(math.exp(x - mx) for _, x in xs)
                lse[bi, h, i] = mx + math.log(den)
                for j, x in xs:
                    o[bi, h, i] += math.exp(x - mx) / den * v[bi, kh, j]
    return o, lse


COMBOS = list(itertools.product([False, True], [0, 2], [False, True], [0.0, 1.3]))


@pytest.mark.parametrize("causal,window,alibi,cap", COMBOS)
def test_forward_matches_brute_force(causal, window, alibi, cap):
    q, k, v = rnd(1, 4, 7, 4, seed=1), rnd(1, 2, 6, 4, seed=2), rnd(1, 2, 6, 4, seed=3)
    slopes = torch.tensor([0.3, -0.2, 0.5, 0.1]) if alibi else None
    o, lse = orc.forward(q, k, v, causal, window, slopes, 0.7, cap)
    bo, blse = brute_forward(q, k, v, causal, window, slopes, 0.7, cap)
    assert torch.allclose(o, bo, atol=1e-12)
    finite = torch.isfinite(blse)
    assert torch.equal(torch.isfinite(lse), finite)
    assert torch.allclose(lse[finite], blse[finite], atol=1e-12)


def test_fully_masked_rows_give_zero_and_neg_inf():
    # Sq > Skv with a window: rows i > Skv-1+W see no key (npu_flash_attention.py:152-161).
    q, k, v = rnd(1, 1, 9, 4, seed=4), rnd(1, 1, 3, 4, seed=5), rnd(1, 1, 3, 4, seed=6)
    o, lse = orc.forward(q, k, v, True, 2, None, None, 0.0)
    assert torch.all(o[0, 0, 5:] == 0) and torch.all(torch.isneginf(lse[0, 0, 5:]))
    assert torch.all(torch.isfinite(lse[0, 0, :5]))
    dq, dk, dv = orc.backward(q, k, v, rnd(1, 1, 9, 4, seed=7), True, 2)
    assert torch.all(torch.isfinite(dq)) and torch.all(dq[0, 0, 5:] == 0)


# ---------------------------------------------------------- library / tests' math --
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("scale", [None, 0.05, 0.2])
def test_forward_matches_sdpa(causal, scale):
    q, k, v = rnd(2, 6, 33, 16, seed=8), rnd(2, 2, 33, 16, seed=9), rnd(2, 2, 33, 16, seed=10)
    o, _ = orc.forward(q, k, v, causal=causal, scale=scale)
    ref = F.scaled_dot_product_attention(
        q, k.repeat_interleave(3, 1), v.repeat_interleave(3, 1), is_causal=causal, scale=scale)
    assert torch.allclose(o, ref, atol=1e-12)


def test_causal_top_left_for_sq_ne_skv():
    # test A14: Sq=128 < Skv=256 matches SDPA(is_causal=True), top-left aligned.
    q, k, v = rnd(1, 1, 12, 8, seed=11), rnd(1, 1, 20, 8, seed=12), rnd(1, 1, 20, 8, seed=13)
    o, _ = orc.forward(q, k, v, causal=True)
    ref = F.scaled_dot_product_attention(q, k, v, is_causal=True)
    assert torch.allclose(o, ref, atol=1e-12)


def test_sliding_window_matches_row_loop():
    # test/test_comprehensive.py:63-73 (causal window of W+1 keys)
    q, k, v = rnd(1, 2, 40, 8, seed=14), rnd(1, 2, 40, 8, seed=15), rnd(1, 2, 40, 8, seed=16)
    w = 6
    o, _ = orc.forward(q, k, v, causal=True, sliding_window=w)
    scale = 1 / math.sqrt(8)
    ref = torch.zeros_like(v)
    for m in range(40):
        s = max(0, m - w)
        a = torch.softmax(q[:, :, m:m + 1] @ k[:, :, s:m + 1].transpose(-2, -1) * scale, -1)
        ref[:, :, m:m + 1] = a @ v[:, :, s:m + 1]
    assert torch.allclose(o, ref, atol=1e-12)


def test_lse_matches_logsumexp():
    # test/test_real_world.py:183-199
    q, k, v = rnd(1, 1, 32, 16, seed=17), rnd(1, 1, 32, 16, seed=18), rnd(1, 1, 32, 16, seed=19)
    _, lse = orc.forward(q, k, v, causal=True)
    qk = q @ k.transpose(-2, -1) / 4.0
    qk = qk.masked_fill(torch.triu(torch.ones(32, 32, dtype=torch.bool), 1), float("-inf"))
    assert torch.allclose(lse, torch.logsumexp(qk, -1), atol=1e-12)


# ------------------------------------------------------------------- backward --
@pytest.mark.parametrize("causal,window,alibi,cap", COMBOS)
def test_backward_closed_form_matches_autograd(causal, window, alibi, cap):
    q, k, v, do = rnd(2, 4, 9, 8, seed=20), rnd(2, 2, 7, 8, seed=21), rnd(2, 2, 7, 8, seed=22), rnd(2, 4, 9, 8, seed=23)
    slopes = torch.tensor([0.3, -0.2, 0.5, 0.1]) if alibi else None
    a = orc.backward(q, k, v, do, causal, window, slopes, 0.6, cap)
    b = orc.backward_autograd(q, k, v, do, causal, window, slopes, 0.6, cap)
    for x, y in zip(a, b):
        assert torch.allclose(x, y, atol=1e-11)


@pytest.mark.parametrize("causal,window,alibi,cap", [(True, 0, False, 0.0), (True, 2, True, 1.1), (False, 3, True, 0.9)])
def test_backward_finite_differences(causal, window, alibi, cap):
    q = rnd(1, 2, 5, 3, seed=24).requires_grad_(True)
    k = rnd(1, 1, 5, 3, seed=25).requires_grad_(True)
    v = rnd(1, 1, 5, 3, seed=26).requires_grad_(True)
    slopes = torch.tensor([0.4, -0.3]) if alibi else None
    do = rnd(1, 2, 5, 3, seed=27)

    def fn(q_, k_, v_):
        g = q_.shape[1] // k_.shape[1]
        x, _ = orc.scores(q_, k_.repeat_interleave(g, 1), 0.8, cap, slopes)
        ok = orc.allowed_mask(5, 5, causal, window)
        x = x.masked_fill(~ok, float("-inf"))
        return torch.softmax(x, -1) @ v_.repeat_interleave(g, 1)

    assert torch.autograd.gradcheck(fn, (q, k, v), eps=1e-6, atol=1e-7)
    # the closed form equals the finite-difference-checked autograd gradient
    o = fn(q, k, v)
    o.backward(do)
    dq, dk, dv = orc.backward(q, k, v, do, causal, window, slopes, 0.8, cap)
    assert torch.allclose(dq, q.grad, atol=1e-11)
    assert torch.allclose(dk, k.grad, atol=1e-11)
    assert torch.allclose(dv, v.grad, atol=1e-11)


def test_dv_is_pt_do_and_delta_identity():
    # B06 (dV = P^T dO) and Delta = rowsum(P * dP) = rowsum(O * dO) (DESIGN.md:131-138 of the reference)
    q, k, v, do = rnd(1, 1, 24, 8, seed=28), rnd(1, 1, 24, 8, seed=29), rnd(1, 1, 24, 8, seed=30), rnd(1, 1, 24, 8, seed=31)
    o, lse = orc.forward(q, k, v, causal=True)
    x = (q @ k.transpose(-2, -1)) / math.sqrt(8)
    x = x.masked_fill(~orc.allowed_mask(24, 24, True, 0), float("-inf"))
    p = torch.exp(x - lse.unsqueeze(-1))
    _, _, dv = orc.backward(q, k, v, do, causal=True)
    assert torch.allclose(dv, p.transpose(-2, -1) @ do, atol=1e-12)
    dp = do @ v.transpose(-2, -1)
    assert torch.allclose((p * dp).sum(-1), orc.delta(o, do), atol=1e-12)


def test_gqa_equals_expanded_mha():
    # test/test_comprehensive.py:333-338: GQA grads = expanded-MHA grads summed over the group
    q, k, v, do = rnd(1, 6, 10, 8, seed=32), rnd(1, 2, 10, 8, seed=33), rnd(1, 2, 10, 8, seed=34), rnd(1, 6, 10, 8, seed=35)
    dq, dk, dv = orc.backward(q, k, v, do, causal=True)
    ke, ve = k.repeat_interleave(3, 1), v.repeat_interleave(3, 1)
    dqe, dke, dve = orc.backward(q, ke, ve, do, causal=True)
    assert torch.allclose(dq, dqe, atol=1e-12)
    assert torch.allclose(dk, dke.view(1, 2, 3, 10, 8).sum(2), atol=1e-12)
    assert torch.allclose(dv, dve.view(1, 2, 3, 10, 8).sum(2), atol=1e-12)


# --------------------------------------------------------------- closed forms --
def test_zero_value_gives_zero_output():  # C04
    q, k = rnd(1, 1, 16, 8, seed=36), rnd(1, 1, 16, 8, seed=37)
    o, _ = orc.forward(q, k, torch.zeros(1, 1, 16, 8), causal=True)
    assert torch.all(o == 0)


def test_zero_query_gives_causal_running_mean():  # C05
    k, v = rnd(1, 1, 16, 8, seed=38), rnd(1, 1, 16, 8, seed=39)
    o, lse = orc.forward(torch.zeros(1, 1, 16, 8), k, v, causal=True)
    mean = torch.cumsum(v, 2) / torch.arange(1, 17).view(1, 1, -1, 1)
    assert torch.allclose(o, mean, atol=1e-12)
    assert torch.allclose(lse[0, 0], torch.log(torch.arange(1, 17, dtype=torch.float64)), atol=1e-12)


def test_single_token_returns_value():  # D03
    q, k, v = rnd(1, 1, 1, 8, seed=40), rnd(1, 1, 1, 8, seed=41), rnd(1, 1, 1, 8, seed=42)
    o, _ = orc.forward(q, k, v, causal=True)
    assert torch.allclose(o, v, atol=1e-15)


def test_degenerate_primitives():
    q, k, v = rnd(1, 2, 12, 8, seed=43), rnd(1, 2, 12, 8, seed=44), rnd(1, 2, 12, 8, seed=45)
    base, _ = orc.forward(q, k, v, causal=True)
    wide, _ = orc.forward(q, k, v, causal=True, sliding_window=12)
    zero_slope, _ = orc.forward(q, k, v, causal=True, alibi_slope=torch.zeros(2))
    huge_cap, _ = orc.forward(q, k, v, causal=True, soft_cap=1e7)
    assert torch.allclose(base, wide, atol=1e-14)
    assert torch.allclose(base, zero_slope, atol=1e-14)
    assert torch.allclose(base, huge_cap, atol=1e-9)


def test_attention_pairs_closed_forms():
    assert orc.attention_pairs(4096, 4096, True, 0) == 4096 * 4097 // 2
    assert orc.attention_pairs(100, 80, False, 0) == 8000
    assert orc.attention_pairs(10, 10, True, 3) == sum(min(i, 3) + 1 for i in range(10))
    assert orc.attention_pairs(20, 20, False, 4) == int(orc.allowed_mask(20, 20, False, 4).sum())


# ----------------------------------------------------------- planted mistakes --
def _mismatch(fn):
    q, k, v = rnd(1, 2, 7, 4, seed=46), rnd(1, 1, 6, 4, seed=47), rnd(1, 1, 6, 4, seed=48)
    slopes = torch.tensor([0.3, 0.5])
    o, _ = fn(q, k, v, True, 2, slopes, 0.7, 1.3)
    bo, _ = brute_forward(q, k, v, True, 2, slopes, 0.7, 1.3)
    return not torch.allclose(o, bo, atol=1e-9)


def test_planted_mistakes_are_caught(monkeypatch):
    good = orc.forward
    assert not _mismatch(good)

    real_scores = orc.scores

    def alibi_sign_flipped(q, k, scale, soft_cap=0.0, alibi_slope=None):
        return real_scores(q, k, scale, soft_cap, None if alibi_slope is None else -alibi_slope)

    monkeypatch.setattr(orc, "scores", alibi_sign_flipped)
    assert _mismatch(orc.forward)
    monkeypatch.setattr(orc, "scores", real_scores)

    real_mask = orc.allowed_mask

    def window_off_by_one(sq, skv, causal, w):
        return real_mask(sq, skv, causal, max(w - 1, 0))

    monkeypatch.setattr(orc, "allowed_mask", window_off_by_one)
    assert _mismatch(orc.forward)

    def causal_transposed(sq, skv, causal, w):
        return real_mask(sq, skv, False, w) & real_mask(skv, sq, causal, 0).T

    monkeypatch.setattr(orc, "allowed_mask", causal_transposed)
    assert _mismatch(orc.forward)
    monkeypatch.setattr(orc, "allowed_mask", real_mask)

    def cap_after_alibi(q, k, scale, soft_cap=0.0, alibi_slope=None):
        x, _ = real_scores(q, k, scale, 0.0, alibi_slope)
        t = torch.tanh(x / soft_cap)
        return soft_cap * t, t

    monkeypatch.setattr(orc, "scores", cap_after_alibi)
    assert _mismatch(orc.forward)
    monkeypatch.setattr(orc, "scores", real_scores)

    def gqa_modulo(q, k, v, causal, window, slopes, scale, cap):
        # query head h reading KV head h % Hkv instead of h // G
        hq = q.shape[1]
        return good(q, k.repeat(1, hq // k.shape[1], 1, 1)[:, :hq], v.repeat(1, hq // v.shape[1], 1, 1)[:, :hq],
                    causal, window, slopes, scale, cap)

    q, k, v = rnd(1, 4, 5, 4, seed=49), rnd(1, 2, 5, 4, seed=50), rnd(1, 2, 5, 4, seed=51)
    bo, _ = brute_forward(q, k, v, True, 0, None, None, 0.0)
    wrong, _ = gqa_modulo(q, k, v, True, 0, None, None, 0.0)
    assert not torch.allclose(wrong, bo, atol=1e-9)


# ------------------------------------------------------------- document masks --
DOC_IDS = torch.tensor([[0, 0, 0, 1, 1, 2, 2, 2, 2, 3, 0, 0, 0],
                        [5, 5, 5, 5, 5, 5, 5, 6, 6, 6, 6, 6, 6]])


def _runs(ids_row):
    """[(start, end)] of the maximal runs of equal values."""
    out, s = [], 0
    for t in range(1, len(ids_row) + 1):
        if t == len(ids_row) or ids_row[t] != ids_row[t - 1]:
            out.append((s, t))
            s = t
    return out


@pytest.mark.parametrize("causal,window,alibi,cap", [(False, 0, False, 0.0), (True, 0, False, 0.0),
                                                      (True, 2, True, 1.3), (False, 3, False, 0.9)])
def test_document_mask_equals_independent_segments(causal, window, alibi, cap):
    """Attention with document masks = attention run on each document alone
    (the primitives depend only on i - j, so slicing preserves them); rows and
    gradients of one document do not see any other."""
    b, hq, hkv, s, d = 2, 4, 2, DOC_IDS.shape[1], 8
    q, k, v, do = rnd(b, hq, s, d, seed=60), rnd(b, hkv, s, d, seed=61), rnd(b, hkv, s, d, seed=62), rnd(b, hq, s, d, seed=63)
    slopes = torch.tensor([0.3, -0.2, 0.5, 0.1]) if alibi else None
    o, lse = orc.forward(q, k, v, causal, window, slopes, 0.6, cap, document_ids=DOC_IDS)
    dq, dk, dv = orc.backward(q, k, v, do, causal, window, slopes, 0.6, cap, document_ids=DOC_IDS)
    for bi in range(b):
        for a, e in _runs(DOC_IDS[bi].tolist()):
            sl = (slice(bi, bi + 1), slice(None), slice(a, e))
            os_, ls_ = orc.forward(q[sl], k[sl], v[sl], causal, window, slopes, 0.6, cap)
            dqs, dks, dvs = orc.backward(q[sl], k[sl], v[sl], do[sl], causal, window, slopes, 0.6, cap)
            assert torch.allclose(o[sl], os_, atol=1e-12)
            assert torch.equal(torch.isinf(lse[sl]), torch.isinf(ls_))
            fin = torch.isfinite(ls_)
            assert torch.allclose(lse[sl][fin], ls_[fin], atol=1e-12)
            assert torch.allclose(dq[sl], dqs, atol=1e-12)
            assert torch.allclose(dk[sl], dks, atol=1e-12)
            assert torch.allclose(dv[sl], dvs, atol=1e-12)


def test_document_runs_not_values():
    """A repeated id after another one starts a new document (runs, not equal
    values): positions 0-2 and 10-12 of row 0 above do not attend to each
    other."""
    m = orc.document_mask(DOC_IDS)
    assert m.shape == (2, 1, 13, 13)
    assert not bool(m[0, 0, 0, 11]) and not bool(m[0, 0, 12, 1])
    assert bool(m[0, 0, 11, 12]) and bool(m[1, 0, 0, 6]) and not bool(m[1, 0, 6, 7])


def test_document_backward_closed_form_matches_autograd():
    q, k, v, do = rnd(2, 4, 13, 8, seed=64), rnd(2, 2, 13, 8, seed=65), rnd(2, 2, 13, 8, seed=66), rnd(2, 4, 13, 8, seed=67)
    a = orc.backward(q, k, v, do, True, 0, None, 0.5, 0.0, document_ids=DOC_IDS)
    b = orc.backward_autograd(q, k, v, do, True, 0, None, 0.5, 0.0, document_ids=DOC_IDS)
    for x, y in zip(a, b):
        assert torch.allclose(x, y, atol=1e-11)


@pytest.mark.parametrize("causal,window,alibi,cap", [(True, 0, False, 0.0), (True, 3, True, 1.2), (False, 4, False, 0.7)])
def test_row_chunked_group_equals_full(causal, window, alibi, cap):
    """forward_backward_rows (query-row chunks, one GQA group) equals the
    whole-matrix forward + backward, Sq != Skv, chunk not dividing Sq."""
    q, k, v, do = rnd(1, 3, 13, 8, seed=80), rnd(1, 1, 11, 8, seed=81), rnd(1, 1, 11, 8, seed=82), rnd(1, 3, 13, 8, seed=83)
    slopes = torch.tensor([0.3, -0.2, 0.5]) if alibi else None
    o, lse = orc.forward(q, k, v, causal, window, slopes, 0.7, cap)
    g = orc.backward(q, k, v, do, causal, window, slopes, 0.7, cap)
    got = orc.forward_backward_rows(q, k, v, do, causal, window, slopes, 0.7, cap, dtype=torch.float64, chunk=5)
    for x, y in zip(got, (o, lse) + tuple(g)):
        fin = torch.isfinite(y)
        assert torch.equal(torch.isfinite(x), fin)
        assert torch.allclose(x[fin], y[fin], atol=1e-12)


def test_row_chunked_group_with_window_skipping_columns():
    """Chunks whose window excludes leading keys (and causal chunks that stop
    early) give the whole-matrix result."""
    q, k, v, do = rnd(1, 2, 40, 8, seed=84), rnd(1, 1, 37, 8, seed=85), rnd(1, 1, 37, 8, seed=86), rnd(1, 2, 40, 8, seed=87)
    for causal, window in ((True, 6), (False, 9), (True, 0)):
        o, lse = orc.forward(q, k, v, causal, window, None, 0.5, 0.0)
        g = orc.backward(q, k, v, do, causal, window, None, 0.5, 0.0)
        got = orc.forward_backward_rows(q, k, v, do, causal, window, None, 0.5, 0.0, dtype=torch.float64, chunk=7)
        for x, y in zip(got, (o, lse) + tuple(g)):
            fin = torch.isfinite(y)
            assert torch.equal(torch.isfinite(x), fin)
            assert torch.allclose(x[fin], y[fin], atol=1e-12)


# ------------------------------------------------ PrefixLM and block maps --
def brute_forward_masked(q, k, v, causal, window, scale, prefix=None, keep=None):
    """Scalar loops with the PrefixLM relaxation of the causal term (key j is
    visible to every row when j < prefix[b]) and an arbitrary keep(b, h, i, j)
    predicate (the block map), written as per-pair conditions."""
    b, hq, sq, d = q.shape
    hkv, skv = k.shape[1], k.shape[2]
    g = hq // hkv
    o = torch.zeros(b, hq, sq, d)
    lse = torch.zeros(b, hq, sq)
    for bi in range(b):
        for h in range(hq):
            for i in range(sq):
                xs = []
                for j in range(skv):
                    if causal and j > i and not (prefix is not None and j < prefix[bi]):
                        continue
                    if window > 0 and i - j > window:
                        continue
                    if keep is not None and not keep(bi, h, i, j):
                        continue
                    x = scale * float(sum(q[bi, h, i, t] * k[bi, h // g, j, t] for t in range(d)))
                    xs.append((j, x))
                if not xs:
                    lse[bi, h, i] = float("-inf")
                    continue
                mx = max(x for _, x in xs)
                den = sum(math.exp(x - mx) for _, x in xs)
                lse[bi, h, i] = mx + math.log(den)
                for j, x in xs:
                    o[bi, h, i] += math.exp(x - mx) / den * v[bi, h // g, j]
    return o, lse


def _close(o, lse, bo, blse):
    assert torch.allclose(o, bo, atol=1e-12)
    fin = torch.isfinite(blse)
    assert torch.equal(torch.isfinite(lse), fin)
    assert torch.allclose(lse[fin], blse[fin], atol=1e-12)


@pytest.mark.parametrize("window", [0, 2])
def test_prefix_lm_matches_brute_force(window):
    q, k, v = rnd(2, 2, 9, 3, seed=11), rnd(2, 1, 9, 3, seed=12), rnd(2, 1, 9, 3, seed=13)
    prefix = [3, 0]
    o, lse = orc.forward(q, k, v, True, window, None, 0.6, 0.0, prefix_len=torch.tensor(prefix))
    _close(o, lse, *brute_forward_masked(q, k, v, True, window, 0.6, prefix=prefix))


def test_prefix_lm_special_cases():
    q, k, v = rnd(1, 2, 10, 4, seed=14), rnd(1, 2, 10, 4, seed=15), rnd(1, 2, 10, 4, seed=16)
    # prefix 0 is plain causal, a prefix covering every key is no mask at all
    for pl, causal_ref in ((0, True), (10, False), (25, False)):
        o, lse = orc.forward(q, k, v, True, 0, None, None, 0.0, prefix_len=torch.tensor([pl]))
        ro, rl = orc.forward(q, k, v, causal_ref, 0, None, None, 0.0)
        assert torch.equal(o, ro) and torch.equal(lse, rl)
    # without causal the prefix changes nothing
    o, _ = orc.forward(q, k, v, False, 0, None, None, 0.0, prefix_len=torch.tensor([4]))
    assert torch.equal(o, orc.forward(q, k, v, False, 0, None, None, 0.0)[0])


@pytest.mark.parametrize("causal,window", [(False, 0), (True, 0), (True, 3)])
def test_block_map_matches_brute_force(causal, window):
    q, k, v = rnd(1, 4, 11, 3, seed=17), rnd(1, 2, 9, 3, seed=18), rnd(1, 2, 9, 3, seed=19)
    bs = 4  # tiny blocks: 3 x 3 map
    gen = torch.Generator().manual_seed(5)
    bm = (torch.rand(1, 4, 3, 3, generator=gen) > 0.4).to(torch.uint8)
    bm[0, 1, 0] = 0  # a head whose first row block sees no key at all
    o, lse = orc.forward(q, k, v, causal, window, None, 0.8, 0.0, block_map=bm, block_size=bs)
    keep = lambda bi, h, i, j: bool(bm[bi, h, i // bs, j // bs])
    _close(o, lse, *brute_forward_masked(q, k, v, causal, window, 0.8, keep=keep))
    assert torch.isneginf(lse[0, 1, :4]).all() and (o[0, 1, :4] == 0).all()


def test_block_map_special_cases():
    q, k, v = rnd(1, 2, 300, 4, seed=20), rnd(1, 2, 300, 4, seed=21), rnd(1, 2, 300, 4, seed=22)
    ones = torch.ones(1, 1, 3, 3, dtype=torch.uint8)
    o, lse = orc.forward(q, k, v, True, 0, None, None, 0.0, block_map=ones)
    ro, rl = orc.forward(q, k, v, True, 0, None, None, 0.0)
    assert torch.equal(o, ro) and torch.equal(lse, rl)
    # a block-diagonal map is a document mask with 128-aligned documents
    diag = torch.eye(3, dtype=torch.uint8).view(1, 1, 3, 3)
    ids = (torch.arange(300) // 128).view(1, -1)
    o, lse = orc.forward(q, k, v, True, 0, None, None, 0.0, block_map=diag)
    ro, rl = orc.forward(q, k, v, True, 0, None, None, 0.0, document_ids=ids)
    assert torch.equal(o, ro) and torch.equal(lse, rl)


def test_prefix_and_block_backward_closed_form_matches_autograd():
    q, k, v, do = (rnd(1, 2, 8, 3, seed=s) for s in (23, 24, 25, 26))
    bm = torch.tensor([[[[1, 0], [1, 1]]]], dtype=torch.uint8)
    kw = dict(causal=True, sliding_window=0, scale=0.9, prefix_len=torch.tensor([3]), block_map=bm, block_size=4)
    a = orc.backward(q, k, v, do, **kw)
    b = orc.backward_autograd(q, k, v, do, **kw)
    for x, y in zip(a, b):
        assert torch.allclose(x, y, atol=1e-12)
