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
# library supports it for the problem (fp16/bf16, head_dim 128, no document
# mask).  Set to False to run the recomputing dQ kernel (flexatt_bwd).
ds_staging_enabled = True
_HEAD_DIMS = (32, 64, 128, 256)


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


def _problem(query, key, scale, causal, sliding_window, soft_cap, alibi, doc=None):
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
    p.causal = 1 if causal else 0
    # The reference enables a primitive only for a positive value
    # (npu_flash_attention.py:70, :648).
    p.sliding_window = int(sliding_window) if sliding_window and sliding_window > 0 else 0
    p.soft_cap = float(soft_cap) if soft_cap and soft_cap > 0.0 else 0.0
    p.alibi_slopes = alibi.data_ptr() if alibi is not None else None
    p.doc_bounds = doc.data_ptr() if doc is not None else None
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
):
    """Attention forward; returns ``O`` or ``(O, LSE)``.

    ``O`` has ``query``'s dtype and layout (``empty_like``), ``LSE`` is fp32
    ``[B, Hq, Sq]`` in natural log.  Follows npu_flash_attention.py:606-656:
    the same shape assertions (:620-622) and default scale ``1/sqrt(D)``
    (:625-626).  ``document_ids`` ([B, S] integers, Sq == Skv; no counterpart
    in the reference) adds a document mask: positions of different runs of
    equal ids do not attend to each other.
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
    doc = _doc_bounds(document_ids, B, Sq, Sk, query.device)
    _forward_into(query, key, value, O, LSE, causal=causal, sliding_window=sliding_window,
                  alibi=alibi_slope, scale=scale, soft_cap=soft_cap, doc=doc)
    if return_lse:
        return O, LSE
    return O


def _forward_into(query, key, value, O, LSE, *, causal, sliding_window, alibi, scale, soft_cap, doc=None):
    """Run the forward kernels into the caller's ``O`` (kernel-ready layout)
    and contiguous fp32 ``LSE``; shapes are already validated."""
    if O.numel() == 0 or key.shape[2] == 0:
        O.zero_()
        LSE.fill_(float("-inf"))
        return
    lib = _lib.load()
    q, k, v = _prepare(query), _prepare(key), _prepare(value)
    slopes = _alibi(alibi, query.shape[1], query.device)
    p = _problem(q, k, scale, causal, sliding_window, soft_cap, slopes, doc)
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
    doc = _doc_bounds(document_ids, B, Sq, Sk, query.device)
    _backward_into(query, key, value, out, lse, grad_out, DQ, DK, DV, causal=causal,
                   sliding_window=sliding_window, alibi=alibi_slope, scale=scale, soft_cap=soft_cap, doc=doc)
    return DQ, DK, DV


def _backward_into(query, key, value, out, lse, grad_out, DQ, DK, DV, *, causal, sliding_window,
                   alibi, scale, soft_cap, doc=None):
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
    p = _problem(q, k, scale, causal, sliding_window, soft_cap, slopes, doc)
    # head_dim 128 fp16/bf16: the dK/dV kernel stages its dS in a workspace
    # from torch's caching allocator and dQ is formed from it
    ws_bytes = lib.flexatt_bwd_workspace(p) if ds_staging_enabled else 0
    with torch.cuda.device(query.device):
        if ws_bytes:
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
                alibi_slope=None, scale=None, block_m=16, block_n=64, soft_cap=0.0, document_ids=None):
        ctx.causal = causal
        ctx.sliding_window = sliding_window
        ctx.alibi_slope = alibi_slope
        ctx.scale = scale
        ctx.block_m = block_m
        ctx.block_n = block_n
        ctx.soft_cap = soft_cap
        ctx.document_ids = document_ids
        with torch.no_grad():
            out, lse = npu_flash_attention_forward(
                query, key, value,
                causal=causal, sliding_window=sliding_window,
                alibi_slope=alibi_slope, scale=scale,
                block_m=block_m, block_n=block_n, return_lse=True,
                soft_cap=soft_cap, document_ids=document_ids,
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
        )
        return DQ, DK, DV, None, None, None, None, None, None, None, None


def npu_flex_attention(
    query, key, value,
    causal=False, sliding_window=0,
    alibi_slope=None, scale=None,
    block_m=16, block_n=64,
    soft_cap=0.0,
    document_ids=None,
):
    """Autograd entry point (npu_flash_attention.py:784-794); ``document_ids``
    as in :func:`npu_flash_attention_forward`."""
    return NPUFlexAttention.apply(
        query, key, value, causal, sliding_window,
        alibi_slope, scale, block_m, block_n, soft_cap, document_ids,
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
    document_ids: Optional[torch.Tensor] = None  # no counterpart in the reference

    def __post_init__(self):
        if self.sliding_window < 0:
            raise ValueError("sliding_window must be >= 0")
        if self.soft_cap < 0:
            raise ValueError("soft_cap must be >= 0")


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
    )
