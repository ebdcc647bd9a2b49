"""Flash attention forward/backward for AMD Instinct MI355X (gfx950).

Drop-in replacement for the reference module ``npu_flash_attention``
(dropletzhu/npu-flex-att, npu_flash_attention.py): the same public names,
signatures, defaults, return values and argument errors, with tensors on a
ROCm device (``"cuda"`` in PyTorch-ROCm) instead of ``"npu"``.  Every call
goes through the C ABI of ``libflexatt.so`` (include/flexatt.h) to
hand-written HIP kernels; there is no Triton, no CPU fallback and no second
backend.

Public API (reference file:line):
  npu_flash_attention_forward   npu_flash_attention.py:606-656
  npu_flash_attention_backward  npu_flash_attention.py:659-739
  NPUFlexAttention              npu_flash_attention.py:742-781
  npu_flex_attention            npu_flash_attention.py:784-794
  AttentionConfig               npu_flash_attention.py:820-844
  flex_attention                npu_flash_attention.py:847-886

``block_m`` / ``block_n`` are accepted for signature compatibility; they were
tiling hints of the Triton kernels and do not change results here (the HIP
kernels use fixed gfx950 tilings).

Masks beyond the reference's primitives (its README.md:198, :219 and
DESIGN.md:374 list them as unsupported or future work), on every entry point:

* ``document_ids`` [B, S]: positions of different runs of equal ids do not
  attend to each other;
* ``prefix_len`` (int or [B]): PrefixLM, with ``causal``; keys below the
  prefix are visible to every query row, the rest stay causal;
* ``block_mask``: block-sparse mask over 128 x 128 blocks of (query rows,
  keys), given as a dense block map [B|1, Hq|1, ceil(Sq/128), ceil(Skv/128)]
  (bool or integer), as ``(kv_num_blocks, kv_indices)`` index tensors, or as
  a ``torch.nn.attention.flex_attention.BlockMask`` with BLOCK_SIZE 128 whose
  listed blocks are whole (no ``mask_mod`` other than the no-op).
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import torch

import flexatt_lib as _lib

__all__ = [
    "npu_flash_attention_forward",
    "npu_flash_attention_backward",
    "NPUFlexAttention",
    "npu_flex_attention",
    "AttentionConfig",
    "flex_attention",
]

_DTYPES = {torch.float32: _lib.F32, torch.float16: _lib.F16, torch.bfloat16: _lib.BF16}

# The forward takes the split-KV decode kernels (flexatt_fwd_decode) whenever
# the problem is in their range: fp16/bf16, D <= 128 and (Hq / Hkv) * Sq <= 32.
# Set to False to force the regular forward kernel (tests compare the two).
decode_enabled = True
# The backward stages dS through a workspace (flexatt_bwd_ws) whenever the
# library supports it for the problem (fp16/bf16 at head_dim 64, 128 and 256;
# fp32 at every head_dim) and reports that staging pays (below).  Set to
# False to run the recomputing dQ kernel (flexatt_bwd).
ds_staging_enabled = True
# Stage only where flexatt_bwd_prefers_staging reports that staging pays:
# not at head_dim 64 fp16/bf16 without soft-cap or interval/block masks,
# where the recomputing backward measured 2-15% faster.  False: stage
# wherever the staged range covers the problem.
ds_staging_auto = True
# Byte budget of that workspace for one backward call.  The whole dS band
# (about one byte per attended (query row, key) pair of each query head for
# fp16/bf16, two for fp32) is used when it fits; otherwise the staged backward
# runs in passes over chunks of whole (batch, KV-head) groups whose band fits,
# and when not even one group fits the recomputing backward runs, whose memory
# is O(S) like the reference's (npu_flash_attention.py:675-685).  The budget
# is the larger of ds_workspace_limit and ds_workspace_free_fraction of the
# device memory free at the call (the driver's free bytes plus what torch's
# caching allocator holds unused), so that long sequences stay on the staged
# backward on a large-memory device; a fraction of 0 keeps the fixed limit.
ds_workspace_limit = 4 << 30
ds_workspace_free_fraction = 0.25
_HEAD_DIMS = (32, 64, 128, 256)
_BLOCK = 128  # block edge of the block-sparse map (flexatt_problem.block_map)


# ----------------------------------------------------------------- helpers --
def _kernel_ready(t: torch.Tensor) -> bool:
    """True if the kernels can read ``t`` in place: innermost stride 1 and
    every row on a 16-byte boundary (batch/head strides may be 0)."""
    if t.dim() != 4 or t.stride(-1) != 1:
        return False
    es = t.element_size()
    if t.data_ptr() % 16:
        return False
    return all((s * es) % 16 == 0 and s >= 0 for s in t.stride()[:3])


def _prepare(t: torch.Tensor) -> torch.Tensor:
    return t if _kernel_ready(t) else t.contiguous()


def _check_device_dtype(name_tensors, dtype):
    for name, t in name_tensors:
        if not isinstance(t, torch.Tensor):
            raise RuntimeError(f"{name} must be a torch.Tensor")
        if t.device.type != "cuda":
            raise RuntimeError(f"{name} must be on a ROCm GPU device (got {t.device})")
        if t.dtype != dtype:
            raise RuntimeError(f"{name} has dtype {t.dtype}, expected {dtype}")


class _Masks:
    """Device tensors of the interval and block masks of one call (kept alive
    for the duration of the kernels) and the causal flag the kernels see:
    PrefixLM is encoded in the row / column bounds with the flag cleared."""

    __slots__ = ("causal", "rows", "cols", "blocks")

    def __init__(self, causal, rows=None, cols=None, blocks=None):
        self.causal = bool(causal)
        self.rows, self.cols, self.blocks = rows, cols, blocks


def _problem(query, key, scale, causal, sliding_window, soft_cap, alibi, masks=None):
    B, Hq, Sq, D = query.shape
    Hkv, Sk = key.shape[1], key.shape[2]
    if query.dtype not in _DTYPES:
        raise RuntimeError(f"unsupported dtype {query.dtype} (expected float32, float16 or bfloat16)")
    if D not in _HEAD_DIMS:
        raise RuntimeError(f"unsupported head dim {D} (expected one of {_HEAD_DIMS})")
    p = _lib.Problem()
    p.dtype = _DTYPES[query.dtype]
    p.batch, p.heads_q, p.heads_kv, p.seqlen_q, p.seqlen_kv, p.head_dim = B, Hq, Hkv, Sq, Sk, D
    p.scale = float(scale)
    if masks is not None:
        causal = masks.causal
    p.causal = 1 if causal else 0
    # The reference enables a primitive only for a positive value
    # (npu_flash_attention.py:70, :648).
    p.sliding_window = int(sliding_window) if sliding_window and sliding_window > 0 else 0
    p.soft_cap = float(soft_cap) if soft_cap and soft_cap > 0.0 else 0.0
    p.alibi_slopes = alibi.data_ptr() if alibi is not None else None
    if masks is not None:
        p.doc_bounds = masks.rows.data_ptr() if masks.rows is not None else None
        p.col_bounds = masks.cols.data_ptr() if masks.cols is not None else None
        if masks.blocks is not None:
            p.block_map = masks.blocks.data_ptr()
            p.block_heads = masks.blocks.shape[1]
    return p


def _alibi(alibi_slope, hq, device):
    if alibi_slope is None:
        return None
    s = torch.as_tensor(alibi_slope, dtype=torch.float32, device=device).reshape(-1).contiguous()
    if s.numel() != hq:
        raise RuntimeError(f"alibi_slope must have Hq={hq} entries, got {s.numel()}")
    return s


def _doc_bounds(document_ids, B, Sq, Sk, device):
    """Document masks: ``document_ids`` [B, S] (S = Sq = Skv) -> int32
    [B, S, 2] holding, per position, the range [lo, hi) of its document, a
    maximal run of equal ids.  Positions of different documents do not attend
    to each other."""
    if document_ids is None:
        return None
    ids = torch.as_tensor(document_ids, device=device)
    if ids.dim() != 2 or ids.shape[0] != B or ids.shape[1] != Sk or Sq != Sk:
        raise RuntimeError(f"document_ids must be [B, S] = [{B}, {Sk}] with Sq == Skv (got {tuple(ids.shape)}, Sq={Sq})")
    if ids.dtype.is_floating_point or ids.dtype == torch.bool:
        raise RuntimeError("document_ids must be an integer tensor")
    S = Sk
    pos = torch.arange(S, device=device, dtype=torch.int32).expand(B, S)
    start = torch.ones(B, S, dtype=torch.bool, device=device)
    start[:, 1:] = ids[:, 1:] != ids[:, :-1]
    end = torch.ones(B, S, dtype=torch.bool, device=device)
    end[:, :-1] = start[:, 1:]
    lo = torch.where(start, pos, torch.zeros_like(pos)).cummax(dim=1).values
    hi = torch.where(end, pos + 1, torch.full_like(pos, S)).flip(1).cummin(dim=1).values.flip(1)
    return torch.stack((lo, hi), dim=-1).to(torch.int32).contiguous()


def _prefix_bounds(prefix_len, doc, B, Sq, Sk, device):
    """PrefixLM with causal: query row i sees keys j <= i and every key
    j < P[b], i.e. the keys [0, max(i + 1, P)); key j is seen by the rows
    [0, Sq) when j < P, else [j, Sq).  Intersected with the document bounds
    ``doc`` (symmetric, Sq == Skv) when given.  Returns int32 row bounds
    [B, Sq, 2] and column bounds [B, Skv, 2], both non-decreasing."""
    pl = torch.as_tensor(prefix_len, device=device)
    if pl.dtype.is_floating_point or pl.dtype == torch.bool:
        raise RuntimeError("prefix_len must be an int or an integer tensor")
    pl = pl.reshape(-1).to(torch.int64)
    if pl.numel() == 1:
        pl = pl.expand(B)
    if pl.numel() != B:
        raise RuntimeError(f"prefix_len must be an int or have B={B} entries, got {pl.numel()}")
    pl = pl.clamp(0, Sk).view(B, 1)
    i = torch.arange(Sq, device=device, dtype=torch.int64).view(1, Sq)
    j = torch.arange(Sk, device=device, dtype=torch.int64).view(1, Sk)
    r_lo = torch.zeros(B, Sq, dtype=torch.int64, device=device)
    r_hi = torch.maximum(i + 1, pl).clamp(max=Sk)
    c_lo = torch.where(j < pl, torch.zeros_like(j), j).expand(B, Sk)
    c_hi = torch.full((B, Sk), Sq, dtype=torch.int64, device=device)
    if doc is not None:
        r_lo = torch.maximum(r_lo, doc[..., 0])
        r_hi = torch.minimum(r_hi, doc[..., 1])
        c_lo = torch.maximum(c_lo, doc[..., 0])
        c_hi = torch.minimum(c_hi, doc[..., 1])
    rows = torch.stack((r_lo, r_hi), dim=-1).to(torch.int32).contiguous()
    cols = torch.stack((c_lo, c_hi), dim=-1).to(torch.int32).contiguous()
    return rows, cols


def _dense_blocks(num, idx, nk, name):
    """(kv_num_blocks [.., nq], kv_indices [.., nq, K]) -> bool [.., nq, nk]:
    the first num[...] entries of each index row are the listed blocks."""
    if num.dtype.is_floating_point or idx.dtype.is_floating_point:
        raise RuntimeError(f"{name}: kv_num_blocks / kv_indices must be integer tensors")
    if idx.dim() != num.dim() + 1 or idx.shape[:-1] != num.shape:
        raise RuntimeError(f"{name}: kv_indices {tuple(idx.shape)} does not extend kv_num_blocks {tuple(num.shape)}")
    K = idx.shape[-1]
    idx = idx.to(torch.int64)
    listed = torch.arange(K, device=idx.device) < num.to(torch.int64).unsqueeze(-1)
    if bool(((idx < 0) | (idx >= nk))[listed].any()):
        raise RuntimeError(f"{name}: a listed block index is outside [0, {nk})")
    out = torch.zeros(*num.shape, nk + 1, dtype=torch.bool, device=idx.device)
    out.scatter_(-1, torch.where(listed, idx, nk), True)  # unlisted slots land in a spare column
    return out[..., :nk]


def _block_map(block_mask, B, Hq, Sq, Sk, device):
    """A block mask in any accepted form -> contiguous uint8 block map
    [B, Hm, ceil(Sq/128), ceil(Skv/128)] on ``device`` with Hm in {1, Hq}."""
    nq, nk = -(-Sq // _BLOCK), -(-Sk // _BLOCK)
    if isinstance(block_mask, torch.Tensor):
        m = block_mask
        if m.dtype.is_floating_point:
            raise RuntimeError("a dense block_mask must be bool or integer")
        if m.dim() != 4 or m.shape[2] != nq or m.shape[3] != nk:
            raise RuntimeError(f"a dense block_mask must be [B|1, Hq|1, {nq}, {nk}] (blocks of {_BLOCK}), "
                               f"got {tuple(m.shape)}")
        m = m != 0
    else:
        if isinstance(block_mask, (tuple, list)) and len(block_mask) == 2:
            parts = [tuple(block_mask)]
        elif hasattr(block_mask, "kv_num_blocks") and hasattr(block_mask, "kv_indices"):
            bs = getattr(block_mask, "BLOCK_SIZE", (_BLOCK, _BLOCK))
            bs = tuple(bs) if isinstance(bs, (tuple, list)) else (bs, bs)
            if bs != (_BLOCK, _BLOCK):
                raise RuntimeError(f"block_mask BLOCK_SIZE must be ({_BLOCK}, {_BLOCK}), got {bs}")
            parts = [(block_mask.kv_num_blocks, block_mask.kv_indices)]
            mm = getattr(block_mask, "mask_mod", None)
            partial = bool((block_mask.kv_num_blocks != 0).any())
            if partial and mm is not None and getattr(mm, "__name__", "") != "noop_mask":
                raise RuntimeError("block_mask: mask_mod functions are not supported; "
                                   "only whole blocks (no mask_mod, or full_kv_* blocks)")
            if getattr(block_mask, "full_kv_num_blocks", None) is not None:
                parts.append((block_mask.full_kv_num_blocks, block_mask.full_kv_indices))
        else:
            raise RuntimeError("block_mask must be a dense block map tensor, a (kv_num_blocks, kv_indices) "
                               "pair or a BlockMask")
        m = None
        for num, idx in parts:
            d = _dense_blocks(torch.as_tensor(num, device=device), torch.as_tensor(idx, device=device), nk,
                              "block_mask")
            if d.dim() != 4 or d.shape[2] < nq:
                raise RuntimeError(f"block_mask must list blocks for [B|1, Hq|1, >= {nq}] query blocks, "
                                   f"got {tuple(d.shape[:3])}")
            d = d[:, :, :nq]
            m = d if m is None else (m | d)
    if m.shape[0] not in (1, B) or m.shape[1] not in (1, Hq):
        raise RuntimeError(f"block_mask must have batch 1 or {B} and heads 1 or {Hq}, got {tuple(m.shape[:2])}")
    return m.to(device=device, dtype=torch.uint8).expand(B, m.shape[1], nq, nk).contiguous()


def _masks(causal, document_ids, prefix_len, block_mask, B, Hq, Sq, Sk, device):
    """The interval / block masks of one call as kernel inputs, or None."""
    if document_ids is None and block_mask is None and (prefix_len is None or not causal):
        return None
    rows = _doc_bounds(document_ids, B, Sq, Sk, device)
    cols = None
    if prefix_len is not None and causal:
        rows, cols = _prefix_bounds(prefix_len, rows, B, Sq, Sk, device)
        causal = False
    blocks = _block_map(block_mask, B, Hq, Sq, Sk, device) if block_mask is not None else None
    return _Masks(causal, rows, cols, blocks)


def _stream(device):
    return torch.cuda.current_stream(device).cuda_stream


# ------------------------------------------------------------- forward (L2) --
def npu_flash_attention_forward(
    query, key, value,
    causal=False,
    sliding_window=0,
    alibi_slope=None,
    scale=None,
    block_m=16,
    block_n=64,
    return_lse=False,
    soft_cap=0.0,
    document_ids=None,
    prefix_len=None,
    block_mask=None,
):
    """Attention forward; returns ``O`` or ``(O, LSE)``.

    ``O`` has ``query``'s dtype and layout (``empty_like``), ``LSE`` is fp32
    ``[B, Hq, Sq]`` in natural log.  Follows npu_flash_attention.py:606-656:
    the same shape assertions (:620-622) and default scale ``1/sqrt(D)``
    (:625-626).  ``document_ids`` ([B, S] integers, Sq == Skv), ``prefix_len``
    and ``block_mask`` add the masks described in the module docstring (no
    counterpart in the reference).
    """
    B, Hq, Sq, D = query.shape
    Bk, Hkv, Sk, Dk = key.shape
    Bv, Hkv2, Sv, Dv = value.shape
    assert D == Dk, "Q and K head dims must match"
    assert Dv == D, "V head dim must match Q head dim for this kernel"
    assert Hq % Hkv == 0, "Hq must be divisible by Hkv"
    assert Bk == B and Bv == B, "Q, K and V batch sizes must match"
    assert Hkv2 == Hkv and Sv == Sk, "K and V must have the same heads and length"
    _check_device_dtype((("query", query), ("key", key), ("value", value)), query.dtype)

    if scale is None:
        scale = 1.0 / math.sqrt(D)

    O = torch.empty_like(query)
    if not _kernel_ready(O):
        O = torch.empty(query.shape, dtype=query.dtype, device=query.device)
    LSE = torch.empty(B, Hq, Sq, device=query.device, dtype=torch.float32)
    masks = _masks(causal, document_ids, prefix_len, block_mask, B, Hq, Sq, Sk, query.device)
    _forward_into(query, key, value, O, LSE, causal=causal, sliding_window=sliding_window,
                  alibi=alibi_slope, scale=scale, soft_cap=soft_cap, masks=masks)
    if return_lse:
        return O, LSE
    return O


def _forward_into(query, key, value, O, LSE, *, causal, sliding_window, alibi, scale, soft_cap, masks=None):
    """Run the forward kernels into the caller's ``O`` (kernel-ready layout)
    and contiguous fp32 ``LSE``; shapes are already validated."""
    if O.numel() == 0 or key.shape[2] == 0:
        O.zero_()
        LSE.fill_(float("-inf"))
        return
    lib = _lib.load()
    q, k, v = _prepare(query), _prepare(key), _prepare(value)
    slopes = _alibi(alibi, query.shape[1], query.device)
    p = _problem(q, k, scale, causal, sliding_window, soft_cap, slopes, masks)
    # Few query rows per KV head (decoding): the split-KV kernels, with their
    # partial results in a workspace from torch's caching allocator.
    ws_bytes = lib.flexatt_fwd_decode_workspace(p) if decode_enabled else 0
    with torch.cuda.device(query.device):
        if ws_bytes:
            ws = torch.empty(ws_bytes, dtype=torch.uint8, device=query.device)
            st = lib.flexatt_fwd_decode(p, _lib.tensor(q), _lib.tensor(k), _lib.tensor(v), _lib.tensor(O),
                                        LSE.data_ptr(), ws.data_ptr(), ws_bytes, _stream(query.device))
            _lib.check(st, "flexatt_fwd_decode")
            return
        st = lib.flexatt_fwd(p, _lib.tensor(q), _lib.tensor(k), _lib.tensor(v), _lib.tensor(O),
                             LSE.data_ptr(), _stream(query.device))
    _lib.check(st, "flexatt_fwd")


# ------------------------------------------------------------ backward (L2) --
def npu_flash_attention_backward(
    query, key, value, out, lse, grad_out,
    causal=False,
    sliding_window=0,
    alibi_slope=None,
    scale=None,
    block_m=16,
    block_n=32,
    soft_cap=0.0,
    document_ids=None,
    prefix_len=None,
    block_mask=None,
):
    """Attention backward; returns ``(dQ, dK, dV)``.

    ``dQ`` is ``empty_like(query)``; ``dK``/``dV`` are ``[B, Hkv, Skv, D]`` in
    K/V's dtype with the GQA group sum already applied
    (npu_flash_attention.py:659-739).  ``Delta = rowsum(out * grad_out)`` is
    computed on the GPU (:681-685) and ``out`` is required (:684).
    """
    B, Hq, Sq, D = query.shape
    Bk, Hkv, Sk, Dk = key.shape
    assert D == Dk, "Q and K head dims must match"
    assert value.shape == key.shape, "K and V shapes must match"
    assert Hq % Hkv == 0, "Hq must be divisible by Hkv"
    assert out is not None, "backward requires forward output `out` to compute Delta"
    assert out.shape == query.shape and grad_out.shape == query.shape, "out/grad_out must match query's shape"
    assert lse is not None and tuple(lse.shape) == (B, Hq, Sq), "lse must be [B, Hq, Sq]"
    _check_device_dtype((("query", query), ("key", key), ("value", value), ("out", out)), query.dtype)
    if grad_out.dtype != query.dtype:
        grad_out = grad_out.to(query.dtype)
    _check_device_dtype((("grad_out", grad_out),), query.dtype)

    if scale is None:
        scale = 1.0 / math.sqrt(D)

    DQ = torch.empty_like(query)
    if not _kernel_ready(DQ):
        DQ = torch.empty(query.shape, dtype=query.dtype, device=query.device)
    DK = torch.empty(B, Hkv, Sk, D, device=key.device, dtype=key.dtype)
    DV = torch.empty(B, Hkv, Sk, D, device=value.device, dtype=value.dtype)
    masks = _masks(causal, document_ids, prefix_len, block_mask, B, Hq, Sq, Sk, query.device)
    _backward_into(query, key, value, out, lse, grad_out, DQ, DK, DV, causal=causal,
                   sliding_window=sliding_window, alibi=alibi_slope, scale=scale, soft_cap=soft_cap, masks=masks)
    return DQ, DK, DV


def _workspace_budget(free_bytes: int) -> int:
    """Byte budget of the staged-dS workspace given ``free_bytes`` of free
    device memory (0: the fixed ``ds_workspace_limit`` alone)."""
    extra = int(ds_workspace_free_fraction * max(0, int(free_bytes))) if ds_workspace_free_fraction > 0 else 0
    return max(0, int(ds_workspace_limit), extra)


def _free_device_bytes(device) -> int:
    """Device memory a workspace could take now: the driver's free bytes
    plus the bytes torch's caching allocator reserves but does not use."""
    free, _ = torch.cuda.mem_get_info(device)
    return int(free) + int(torch.cuda.memory_reserved(device)) - int(torch.cuda.memory_allocated(device))


def _staged_workspace_bytes(lib, p, device=None) -> int:
    """Workspace bytes of the staged backward for problem ``p`` under the
    workspace budget (``ds_workspace_limit``, or ``ds_workspace_free_fraction``
    of the free memory of ``device`` when that is larger; the whole band, or
    the band of the chunk of whole (batch, KV-head) groups one pass covers);
    0 selects the recomputing backward (staging disabled, outside its range,
    slower for ``p`` under ``ds_staging_auto``, or not even one group's band
    within the budget)."""
    if not ds_staging_enabled:
        return 0
    if ds_staging_auto and not lib.flexatt_bwd_prefers_staging(p):
        return 0
    free = 0
    if device is not None and ds_workspace_free_fraction > 0 and lib.flexatt_bwd_workspace(p) > ds_workspace_limit:
        free = _free_device_bytes(device)  # queried only when the fixed limit does not hold the whole band
    return int(lib.flexatt_bwd_workspace_limited(p, _workspace_budget(free)))


def _backward_into(query, key, value, out, lse, grad_out, DQ, DK, DV, *, causal, sliding_window,
                   alibi, scale, soft_cap, masks=None):
    """Run Delta, dQ and dK/dV into the caller's ``DQ`` (kernel-ready layout)
    and contiguous ``DK`` / ``DV``; shapes are already validated."""
    if DQ.numel() == 0 or DK.numel() == 0:
        DQ.zero_()
        DK.zero_()
        DV.zero_()
        return
    B, Hq, Sq, _ = query.shape
    delta = torch.empty(B, Hq, Sq, device=query.device, dtype=torch.float32)
    lib = _lib.load()
    q, k, v = _prepare(query), _prepare(key), _prepare(value)
    o, do = _prepare(out), _prepare(grad_out)
    lse = lse.to(torch.float32).contiguous()
    slopes = _alibi(alibi, Hq, query.device)
    p = _problem(q, k, scale, causal, sliding_window, soft_cap, slopes, masks)
    ws_bytes = _staged_workspace_bytes(lib, p, query.device)
    with torch.cuda.device(query.device):
        if ws_bytes:
            # the dK/dV kernel stages its dS in a workspace from torch's
            # caching allocator and dQ is formed from it
            ws = torch.empty(ws_bytes, dtype=torch.uint8, device=query.device)
            st = lib.flexatt_bwd_ws(p, _lib.tensor(q), _lib.tensor(k), _lib.tensor(v), _lib.tensor(o),
                                    _lib.tensor(do), lse.data_ptr(), delta.data_ptr(), _lib.tensor(DQ),
                                    _lib.tensor(DK), _lib.tensor(DV), ws.data_ptr(), ws_bytes,
                                    _stream(query.device))
            _lib.check(st, "flexatt_bwd_ws")
            return
        st = lib.flexatt_bwd(p, _lib.tensor(q), _lib.tensor(k), _lib.tensor(v), _lib.tensor(o),
                             _lib.tensor(do), lse.data_ptr(), delta.data_ptr(), _lib.tensor(DQ),
                             _lib.tensor(DK), _lib.tensor(DV), _stream(query.device))
    _lib.check(st, "flexatt_bwd")


# ----------------------------------------------------------- autograd (L3) --
class NPUFlexAttention(torch.autograd.Function):
    """Differentiable attention (npu_flash_attention.py:742-781).

    Forward runs without grad and saves ``(q, k, v, lse, out)``; backward
    recomputes P from the LSE.  Gradients flow to query/key/value only.
    """

    @staticmethod
    def forward(ctx, query, key, value, causal=False, sliding_window=0,
                alibi_slope=None, scale=None, block_m=16, block_n=64, soft_cap=0.0, document_ids=None,
                prefix_len=None, block_mask=None):
        ctx.causal = causal
        ctx.sliding_window = sliding_window
        ctx.alibi_slope = alibi_slope
        ctx.scale = scale
        ctx.block_m = block_m
        ctx.block_n = block_n
        ctx.soft_cap = soft_cap
        ctx.document_ids = document_ids
        ctx.prefix_len = prefix_len
        ctx.block_mask = block_mask
        with torch.no_grad():
            out, lse = npu_flash_attention_forward(
                query, key, value,
                causal=causal, sliding_window=sliding_window,
                alibi_slope=alibi_slope, scale=scale,
                block_m=block_m, block_n=block_n, return_lse=True,
                soft_cap=soft_cap, document_ids=document_ids,
                prefix_len=prefix_len, block_mask=block_mask,
            )
        ctx.save_for_backward(query, key, value, lse, out)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        query, key, value, lse, out = ctx.saved_tensors
        DQ, DK, DV = npu_flash_attention_backward(
            query, key, value, out, lse, grad_out.contiguous(),
            causal=ctx.causal, sliding_window=ctx.sliding_window,
            alibi_slope=ctx.alibi_slope, scale=ctx.scale,
            block_m=ctx.block_m, block_n=ctx.block_n,
            soft_cap=ctx.soft_cap, document_ids=ctx.document_ids,
            prefix_len=ctx.prefix_len, block_mask=ctx.block_mask,
        )
        return DQ, DK, DV, None, None, None, None, None, None, None, None, None, None


def npu_flex_attention(
    query, key, value,
    causal=False, sliding_window=0,
    alibi_slope=None, scale=None,
    block_m=16, block_n=64,
    soft_cap=0.0,
    document_ids=None,
    prefix_len=None,
    block_mask=None,
):
    """Autograd entry point (npu_flash_attention.py:784-794); ``document_ids``,
    ``prefix_len`` and ``block_mask`` as in :func:`npu_flash_attention_forward`."""
    return NPUFlexAttention.apply(
        query, key, value, causal, sliding_window,
        alibi_slope, scale, block_m, block_n, soft_cap, document_ids, prefix_len, block_mask,
    )


# ------------------------------------------------- template config API (L4) --
@dataclass
class AttentionConfig:
    """Composable attention pattern (npu_flash_attention.py:820-844).

    Each combination of primitives selects one ahead-of-time compiled kernel
    instance; the window, cap, scale and GQA ratio are runtime values, so new
    values never trigger a compile.

    Example — Gemma2-style attention::

        config = AttentionConfig(causal=True, sliding_window=1024, soft_cap=50.0)
        out = flex_attention(q, k, v, config=config)
    """

    causal: bool = False
    sliding_window: int = 0
    alibi_slope: Optional[torch.Tensor] = None
    scale: Optional[float] = None
    soft_cap: float = 0.0
    block_m: int = 16
    block_n: int = 64
    # no counterpart in the reference: document, PrefixLM and block masks
    document_ids: Optional[torch.Tensor] = None
    prefix_len: Optional[object] = None
    block_mask: Optional[object] = None

    def __post_init__(self):
        if self.sliding_window < 0:
            raise ValueError("sliding_window must be >= 0")
        if self.soft_cap < 0:
            raise ValueError("soft_cap must be >= 0")
        if self.prefix_len is not None and not self.causal:
            raise ValueError("prefix_len relaxes the causal mask and needs causal=True")


def flex_attention(query, key, value, config: Optional[AttentionConfig] = None, **kwargs):
    """Attention with composable primitives (npu_flash_attention.py:847-886).

    Builds an :class:`AttentionConfig` from ``kwargs`` when ``config`` is None
    (kwargs are ignored when a config is given) and returns ``O`` only;
    differentiable through :class:`NPUFlexAttention`.
    """
    if config is None:
        config = AttentionConfig(**kwargs)
    return npu_flex_attention(
        query, key, value,
        causal=config.causal,
        sliding_window=config.sliding_window,
        alibi_slope=config.alibi_slope,
        scale=config.scale,
        block_m=config.block_m,
        block_n=config.block_n,
        soft_cap=config.soft_cap,
        document_ids=config.document_ids,
        prefix_len=config.prefix_len,
        block_mask=config.block_mask,
    )
