"""CPU oracle for the flash-attention forward/backward hot path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker.  The product path (``npu_flash_attention`` and the HIP library under
it) never imports it and has no CPU fallback.

What it restates
----------------
The reference (dropletzhu/npu-flex-att) defines the semantics of the path in
its Triton kernels and checks them in its tests against PyTorch eager math.
This module is that eager math, in float64 on the CPU by default, extended to
every primitive the kernels implement:

* score order ``x = scale * q.k`` -> soft-cap ``cap*tanh(x/cap)`` -> ALiBi
  ``+ slope[h]*(i-j)`` -> mask  (npu_flash_attention.py:102-109, :129-141);
* mask ``allowed(i,j) = (j<=i if causal) & (i-j<=W if W>0) & (j<Skv)``
  (npu_flash_attention.py:65-80, :138-141; the ``j<Skv`` term is the tail
  handling the reference lacks, README.md:199);
* softmax with natural-log LSE, fully-masked rows give ``O=0, LSE=-inf``
  (npu_flash_attention.py:152-166);
* GQA: query head ``h`` reads KV head ``h // G`` (npu_flash_attention.py:42);
* document masks (no counterpart in the reference, see :func:`document_mask`):
  pairs in different runs of ``document_ids`` are masked;
* PrefixLM (see :func:`prefix_mask`): with ``causal``, keys below
  ``prefix_len[b]`` are visible to every query row;
* block maps (see :func:`block_mask_dense`): whole blocks of (query rows,
  keys) removed from the attention;
* backward: ``Delta = rowsum(O*dO)`` (npu_flash_attention.py:681-685),
  ``dS = P*(dP-Delta)*scale*(1-tanh^2)`` (npu_flash_attention.py:386-399,
  :502-516), dK/dV summed over the G query heads of a group
  (npu_flash_attention.py:734-737).  Unlike the reference kernels, the ALiBi
  bias is part of the recomputed P (the reference drops it in backward); the
  oracle follows the eager autograd math, which is what the reference's tests
  compare against (test/test_comprehensive.py:54-60).

Pinning (the checks that make this module trustworthy live in
``tests/test_oracle.py``): library SDPA equality, per-row brute-force loops,
``torch.logsumexp``, closed forms (V=0, Q=0, S=1, dV=P^T dO, the Delta
identity), finite-difference gradient checks and planted-mistake checks.
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import torch

__all__ = [
    "allowed_mask",
    "document_mask",
    "scores",
    "forward",
    "delta",
    "backward",
    "backward_autograd",
    "forward_backward_chunked",
    "forward_backward_rows",
    "attention_pairs",
    "prefix_mask",
    "block_mask_dense",
]


def allowed_mask(sq: int, skv: int, causal: bool, sliding_window: int) -> torch.Tensor:
    """Boolean [Sq, Skv] mask of attended (i, j) pairs.

    Follows npu_flash_attention.py:138-141: causal keeps ``j <= i`` (top-left
    aligned, the same as ``F.scaled_dot_product_attention(is_causal=True)``
    used by test A14), a window ``W > 0`` keeps ``i - j <= W`` (W+1 keys when
    causal; future keys are not masked without causal).  Columns never exceed
    ``Skv`` here because the matrix is exactly [Sq, Skv].
    """
    i = torch.arange(sq).view(-1, 1)
    j = torch.arange(skv).view(1, -1)
    ok = torch.ones(sq, skv, dtype=torch.bool)
    if causal:
        ok &= j <= i
    if sliding_window > 0:
        ok &= (i - j) <= sliding_window
    return ok


def document_mask(document_ids: torch.Tensor) -> torch.Tensor:
    """Boolean [B, 1, S, S] mask of pairs in the same document.

    Document masking has no counterpart in the reference (it is one of the
    future candidates it lists, its README.md:219 and DESIGN.md:374, :382).  Here a
    document is a maximal run of equal values along a row of
    ``document_ids`` [B, S]: positions i and j attend to each other only
    inside one run (on top of the other primitives).
    """
    ids = document_ids.detach().to("cpu").long()
    change = torch.zeros_like(ids)
    change[:, 1:] = (ids[:, 1:] != ids[:, :-1]).long()
    run = torch.cumsum(change, dim=1)
    return (run.unsqueeze(-1) == run.unsqueeze(-2)).unsqueeze(1)


def prefix_mask(sq: int, skv: int, prefix_len) -> torch.Tensor:
    """Boolean [B, 1, Sq, Skv] PrefixLM relaxation of the causal mask: key j
    is visible to every query row when ``j < prefix_len[b]`` (a bidirectional
    prefix), otherwise only to rows ``i >= j``.  PrefixLM has no counterpart
    in the reference (a future candidate in its DESIGN.md:374); it replaces
    the causal term of :func:`allowed_mask`, the other primitives still
    apply."""
    pl = torch.as_tensor(prefix_len).reshape(-1).to("cpu", torch.long)
    i = torch.arange(sq).view(1, -1, 1)
    j = torch.arange(skv).view(1, 1, -1)
    return ((j <= i) | (j < pl.view(-1, 1, 1))).unsqueeze(1)


def block_mask_dense(block_map: torch.Tensor, sq: int, skv: int, block_size: int = 128) -> torch.Tensor:
    """Boolean [B, H, Sq, Skv] mask of a block map [B, H, ceil(Sq / bs),
    ceil(Skv / bs)] (nonzero = block computed): pair (i, j) is kept when block
    (i // bs, j // bs) is.  The reference lists block-sparse masks as
    unsupported (README.md:198); here a block map only removes whole blocks,
    on top of the other primitives."""
    m = block_map.detach().to("cpu") != 0
    m = m.repeat_interleave(block_size, dim=-2).repeat_interleave(block_size, dim=-1)
    return m[..., :sq, :skv]


def _mask(sq, skv, causal, sliding_window, document_ids, prefix_len=None, block_map=None, block_size=128):
    if prefix_len is not None and causal:
        ok = allowed_mask(sq, skv, False, sliding_window) & prefix_mask(sq, skv, prefix_len)
    else:
        ok = allowed_mask(sq, skv, causal, sliding_window)
    if document_ids is not None:
        ok = ok & document_mask(document_ids)
    if block_map is not None:
        ok = ok & block_mask_dense(block_map, sq, skv, block_size)
    return ok


def _expand_kv(x: torch.Tensor, groups: int) -> torch.Tensor:
    """[B, Hkv, S, D] -> [B, Hkv*G, S, D]; consecutive query heads share a KV
    head (npu_flash_attention.py:42, test/test_comprehensive.py:189)."""
    return x if groups == 1 else x.repeat_interleave(groups, dim=1)


def scores(
    q: torch.Tensor,
    k: torch.Tensor,
    scale: float,
    soft_cap: float = 0.0,
    alibi_slope: Optional[torch.Tensor] = None,
) -> Tuple[torch.Tensor, Optional[torch.Tensor]]:
    """Unmasked logits ``x`` [B, Hq, Sq, Skv] and ``tanh(scale*qk/cap)``.

    Order follows npu_flash_attention.py:102-109: scale, then soft-cap, then
    ``+ slope[h] * (i - j)`` (the reference's sign: the bias grows with
    distance for positive slopes).  ``k`` must already be expanded to Hq heads.
    """
    x = torch.matmul(q, k.transpose(-2, -1)) * scale
    t = None
    if soft_cap > 0.0:
        t = torch.tanh(x / soft_cap)
        x = soft_cap * t
    if alibi_slope is not None:
        sq, skv = x.shape[-2], x.shape[-1]
        i = torch.arange(sq, dtype=x.dtype).view(-1, 1)
        j = torch.arange(skv, dtype=x.dtype).view(1, -1)
        slope = alibi_slope.to(x.dtype).view(1, -1, 1, 1)
        x = x + slope * (i - j)
    return x, t


def _prep(q, k, v, scale, dtype):
    b, hq, sq, d = q.shape
    hkv = k.shape[1]
    assert hq % hkv == 0
    g = hq // hkv
    if scale is None:
        scale = 1.0 / math.sqrt(d)  # npu_flash_attention.py:625-626
    q = q.detach().to("cpu", dtype)
    k = _expand_kv(k.detach().to("cpu", dtype), g)
    v = _expand_kv(v.detach().to("cpu", dtype), g)
    return q, k, v, float(scale), g


def _softmax_masked(x: torch.Tensor, ok: torch.Tensor):
    """Masked softmax with natural-log LSE; fully masked rows -> P=0, LSE=-inf
    (npu_flash_attention.py:152-161)."""
    x = x.masked_fill(~ok, float("-inf"))
    lse = torch.logsumexp(x, dim=-1)
    safe = torch.where(torch.isfinite(lse), lse, torch.zeros_like(lse))
    p = torch.exp(x - safe.unsqueeze(-1))
    p = torch.where(ok, p, torch.zeros_like(p))
    return p, lse


def forward(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    causal: bool = False,
    sliding_window: int = 0,
    alibi_slope: Optional[torch.Tensor] = None,
    scale: Optional[float] = None,
    soft_cap: float = 0.0,
    dtype: torch.dtype = torch.float64,
    document_ids: Optional[torch.Tensor] = None,
    prefix_len=None,
    block_map: Optional[torch.Tensor] = None,
    block_size: int = 128,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Eager attention forward: returns (O [B,Hq,Sq,D], LSE [B,Hq,Sq]).

    Semantics of npu_flash_attention.py:17-166 (flash_attn_fwd_kernel) as the
    eager math of test/test_comprehensive.py:42-51 and :63-73 and
    test/test_real_world.py:183-199 compute it, in ``dtype`` on the CPU.
    """
    qf, kf, vf, scale, _ = _prep(q, k, v, scale, dtype)
    x, _ = scores(qf, kf, scale, soft_cap, alibi_slope)
    ok = _mask(x.shape[-2], x.shape[-1], causal, sliding_window, document_ids, prefix_len, block_map, block_size)
    p, lse = _softmax_masked(x, ok)
    return torch.matmul(p, vf), lse


def delta(o: torch.Tensor, do: torch.Tensor, dtype: torch.dtype = torch.float64) -> torch.Tensor:
    """``Delta[b,h,i] = sum_d O*dO`` (npu_flash_attention.py:681-685)."""
    return (o.detach().to("cpu", dtype) * do.detach().to("cpu", dtype)).sum(-1)


def _score_grad(qf, kf, vf, dof, causal, sliding_window, alibi_slope, scale, soft_cap, o, dtype, document_ids,
                prefix_len=None, block_map=None, block_size=128):
    """(dS / scale, P) [B, Hq, Sq, Skv] from prepared (expanded) inputs:
    ``P (dP - Delta) (1 - tanh^2)``, 0 at masked pairs (npu_flash_attention.py
    :386-397, :502-513)."""
    sq = qf.shape[2]
    x, t = scores(qf, kf, scale, soft_cap, alibi_slope)
    ok = _mask(sq, x.shape[-1], causal, sliding_window, document_ids, prefix_len, block_map, block_size)
    p, _ = _softmax_masked(x, ok)
    of = torch.matmul(p, vf) if o is None else o.detach().to("cpu", dtype)
    dl = (of * dof).sum(-1, keepdim=True)
    dp = torch.matmul(dof, vf.transpose(-2, -1))
    ds = p * (dp - dl)
    if t is not None:
        ds = ds * (1.0 - t * t)
    return ds, p


def score_grad(q, k, v, do, causal=False, sliding_window=0, alibi_slope=None, scale=None, soft_cap=0.0,
               dtype=torch.float64, document_ids=None, prefix_len=None, block_map=None, block_size=128):
    """Gradient of the loss with respect to the scaled, capped, biased logits
    before the scale factor: ``dS / scale = P (dP - Delta) (1 - tanh^2)``,
    [B, Hq, Sq, Skv], 0 at masked pairs.  :func:`backward` forms
    ``dQ = scale dS K`` and ``dK = scale dS^T Q`` from exactly this tensor, so
    it is pinned by backward's checks."""
    qf, kf, vf, scale, _ = _prep(q, k, v, scale, dtype)
    return _score_grad(qf, kf, vf, do.detach().to("cpu", dtype), causal, sliding_window, alibi_slope, scale,
                       soft_cap, None, dtype, document_ids, prefix_len, block_map, block_size)[0]


def backward(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    do: torch.Tensor,
    causal: bool = False,
    sliding_window: int = 0,
    alibi_slope: Optional[torch.Tensor] = None,
    scale: Optional[float] = None,
    soft_cap: float = 0.0,
    dtype: torch.dtype = torch.float64,
    o: Optional[torch.Tensor] = None,
    document_ids: Optional[torch.Tensor] = None,
    prefix_len=None,
    block_map: Optional[torch.Tensor] = None,
    block_size: int = 128,
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Closed-form attention backward: (dQ, dK, dV), dK/dV in [B,Hkv,Skv,D].

    Formulas of npu_flash_attention.py:386-399 (dQ) and :502-516 (dK/dV):
    ``P = exp(x - LSE)``, ``dP = dO V^T``, ``Delta = rowsum(O*dO)``,
    ``dS = P*(dP - Delta)*scale*(1 - tanh^2)``, ``dQ = dS K``,
    ``dK = dS^T Q``, ``dV = P^T dO``, summed over each GQA group
    (npu_flash_attention.py:734-737).  ``o`` may be given to use a specific
    forward output for Delta (as the reference's wrapper does); by default the
    oracle's own O is used.
    """
    b, hq, sq, d = q.shape
    hkv = k.shape[1]
    qf, kf, vf, scale, g = _prep(q, k, v, scale, dtype)
    dof = do.detach().to("cpu", dtype)
    ds, p = _score_grad(qf, kf, vf, dof, causal, sliding_window, alibi_slope, scale, soft_cap, o, dtype,
                        document_ids, prefix_len, block_map, block_size)
    ds = ds * scale
    dq = torch.matmul(ds, kf)
    dk = torch.matmul(ds.transpose(-2, -1), qf)
    dv = torch.matmul(p.transpose(-2, -1), dof)
    skv = kf.shape[2]
    dk = dk.view(b, hkv, g, skv, d).sum(2)
    dv = dv.view(b, hkv, g, skv, d).sum(2)
    return dq, dk, dv


def backward_autograd(q, k, v, do, causal=False, sliding_window=0, alibi_slope=None,
                      scale=None, soft_cap=0.0, dtype=torch.float64, document_ids=None, prefix_len=None,
                      block_map=None, block_size=128):
    """(dQ, dK, dV) by autograd through :func:`forward` — the form of the
    reference's oracle ``ref_sdpa_backward`` (test/test_comprehensive.py:54-60);
    GQA K/V gradients come out summed over the group because the expansion is
    part of the graph (test/test_comprehensive.py:333-338)."""
    qr = q.detach().to("cpu", dtype).requires_grad_(True)
    kr = k.detach().to("cpu", dtype).requires_grad_(True)
    vr = v.detach().to("cpu", dtype).requires_grad_(True)
    hq, hkv = q.shape[1], k.shape[1]
    g = hq // hkv
    sc = (1.0 / math.sqrt(q.shape[-1])) if scale is None else float(scale)
    x, _ = scores(qr, _expand_kv(kr, g), sc, soft_cap, alibi_slope)
    ok = _mask(x.shape[-2], x.shape[-1], causal, sliding_window, document_ids, prefix_len, block_map, block_size)
    p, _ = _softmax_masked(x, ok)
    o = torch.matmul(p, _expand_kv(vr, g))
    o.backward(do.detach().to("cpu", dtype))
    return qr.grad, kr.grad, vr.grad


def attention_pairs(sq: int, skv: int, causal: bool, sliding_window: int) -> int:
    """Number of attended (i, j) pairs per head — the FLOP-count numerator."""
    total = 0
    for i in range(sq):
        lo = 0
        hi = skv - 1
        if causal:
            hi = min(hi, i)
        if sliding_window > 0:
            lo = max(lo, i - sliding_window)
        if hi >= lo:
            total += hi - lo + 1
    return total


def forward_backward_chunked(q, k, v, do, causal=False, sliding_window=0, alibi_slope=None,
                             scale=None, soft_cap=0.0, dtype=torch.float32, with_backward=True,
                             max_groups=None):
    """Forward (+ backward) evaluated one (batch, KV-head group) at a time.

    Bounds memory at the large configurations (the score matrix of one group
    is G*Sq*Skv elements).  ``max_groups`` evaluates only the first N groups
    (the bounded sample the CPU baseline times).  Returns the list of per-group
    results ``(b, hkv, O, LSE, dQ, dK, dV)``.
    """
    b, hq, sq, d = q.shape
    hkv = k.shape[1]
    g = hq // hkv
    out = []
    count = 0
    for bi in range(b):
        for h in range(hkv):
            if max_groups is not None and count >= max_groups:
                return out
            hs = slice(h * g, (h + 1) * g)
            qs, ks, vs = q[bi:bi + 1, hs], k[bi:bi + 1, h:h + 1], v[bi:bi + 1, h:h + 1]
            sl = None if alibi_slope is None else alibi_slope[hs]
            o, lse = forward(qs, ks, vs, causal, sliding_window, sl, scale, soft_cap, dtype)
            grads = (None, None, None)
            if with_backward:
                grads = backward(qs, ks, vs, do[bi:bi + 1, hs], causal, sliding_window, sl,
                                 scale, soft_cap, dtype, o=o)
            out.append((bi, h, o, lse) + tuple(grads))
            count += 1
    return out


def forward_backward_rows(q, k, v, do, causal=False, sliding_window=0, alibi_slope=None, scale=None,
                          soft_cap=0.0, dtype=torch.float32, chunk=1024):
    """Forward and closed-form backward of one (batch, KV-head) group,
    evaluated over chunks of ``chunk`` query rows so that memory stays
    bounded at full sequence lengths (a [G, chunk, Skv] score block at a
    time).  Same formulas and results as :func:`forward` + :func:`backward`
    (``q``, ``do``: [1, G, Sq, D]; ``k``, ``v``: [1, 1, Skv, D]).  Returns
    (O, LSE, dQ, dK, dV) with dK / dV summed over the G heads.  Each chunk
    only scores the keys a causal mask or a window leaves to it.
    """
    d = q.shape[-1]
    sc = (1.0 / math.sqrt(d)) if scale is None else float(scale)
    qf = q.detach().to("cpu", dtype)[0]
    dof = do.detach().to("cpu", dtype)[0]
    kf = k.detach().to("cpu", dtype)[0, 0]
    vf = v.detach().to("cpu", dtype)[0, 0]
    g, sq, _ = qf.shape
    skv = kf.shape[0]
    sl = None if alibi_slope is None else alibi_slope.detach().to("cpu", dtype).view(g, 1, 1)
    o = torch.empty(g, sq, d, dtype=dtype)
    lse = torch.empty(g, sq, dtype=dtype)
    dq = torch.empty(g, sq, d, dtype=dtype)
    dk = torch.zeros(skv, d, dtype=dtype)
    dv = torch.zeros(skv, d, dtype=dtype)
    for r0 in range(0, sq, chunk):
        r1 = min(sq, r0 + chunk)
        # keys outside [c0, c1) are masked for every row of the chunk
        c0 = max(0, r0 - sliding_window) if sliding_window > 0 else 0
        c1 = min(skv, r1) if causal else skv
        c1 = max(c1, c0 + 1)  # keep one column so that fully masked rows stay defined
        i = torch.arange(r0, r1).view(-1, 1)
        j = torch.arange(c0, c1).view(1, -1)
        kc, vc = kf[c0:c1], vf[c0:c1]
        x = torch.matmul(qf[:, r0:r1], kc.transpose(0, 1)) * sc
        t = None
        if soft_cap > 0.0:
            t = torch.tanh(x / soft_cap)
            x = soft_cap * t
        if sl is not None:
            x = x + sl * (i - j).to(dtype)
        ok = torch.ones(r1 - r0, c1 - c0, dtype=torch.bool)
        if causal:
            ok &= j <= i
        if sliding_window > 0:
            ok &= (i - j) <= sliding_window
        p, ls = _softmax_masked(x, ok)
        oc = torch.matmul(p, vc)
        o[:, r0:r1] = oc
        lse[:, r0:r1] = ls
        dl = (oc * dof[:, r0:r1]).sum(-1, keepdim=True)
        ds = p * (torch.matmul(dof[:, r0:r1], vc.transpose(0, 1)) - dl)
        if t is not None:
            ds = ds * (1.0 - t * t)
        ds = ds * sc
        dq[:, r0:r1] = torch.matmul(ds, kc)
        dk[c0:c1] += torch.matmul(ds.transpose(1, 2), qf[:, r0:r1]).sum(0)
        dv[c0:c1] += torch.matmul(p.transpose(1, 2), dof[:, r0:r1]).sum(0)
    return o[None], lse[None], dq[None], dk[None, None], dv[None, None]
