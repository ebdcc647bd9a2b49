"""``torch.library`` registration of the attention kernels, for ``torch.compile``.

The reference has no compiler integration (its README.md:220 and DESIGN.md:405
list it as a limitation): its autograd.Function is opaque to Dynamo.  This module
registers the same forward / backward as two custom operators with fake
(meta) implementations and an autograd formula, so that a compiled graph
keeps the HIP kernels as single nodes and traces around them without a graph
break:

  flexatt::fwd(q, k, v, alibi, scale, causal, window, soft_cap, rows, cols, blocks)
      -> (O, LSE)
  flexatt::bwd(dO, q, k, v, O, LSE, alibi, scale, causal, window, soft_cap, rows, cols,
               blocks) -> (dQ, dK, dV)

(``rows`` / ``cols``: optional int32 [B, Sq, 2] / [B, Skv, 2] interval bounds,
``blocks``: optional uint8 block map, as built from ``document_ids``,
``prefix_len`` and ``block_mask`` by the npu_flash_attention entry points.)

Both run exactly the kernels of npu_flash_attention_forward / _backward
(npu_flash_attention.py:606-656, :659-739 in the reference), so results are
bitwise identical to those calls.  Outputs of the operators are contiguous
(``O`` and ``dQ`` in ``[B, Hq, Sq, D]``, ``dK`` / ``dV`` in
``[B, Hkv, Skv, D]``, ``LSE`` fp32 ``[B, Hq, Sq]``), which is what the fake
implementations promise.  ``LSE`` is returned for callers that need it but is
not differentiable.

``attention(...)`` is the user-facing entry point with the reference's
argument names and defaults (npu_flex_attention, npu_flash_attention.py:
784-794, without the ``block_m`` / ``block_n`` tiling hints).
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import torch

import npu_flash_attention as _nfa

__all__ = ["attention"]

_NS = "flexatt"


def _check_shapes(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> None:
    # the reference's forward assertions (npu_flash_attention.py:620-622)
    B, Hq, Sq, D = q.shape
    Bk, Hkv, Sk, Dk = k.shape
    assert D == Dk, "Q and K head dims must match"
    assert tuple(v.shape) == tuple(k.shape), "K and V shapes must match"
    assert Hq % Hkv == 0, "Hq must be divisible by Hkv"
    assert Bk == B, "Q, K and V batch sizes must match"


@torch.library.custom_op(f"{_NS}::fwd", mutates_args=(), device_types="cuda")
def _fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, alibi: Optional[torch.Tensor],
         scale: float, causal: bool, window: int, soft_cap: float,
         rows: Optional[torch.Tensor] = None, cols: Optional[torch.Tensor] = None,
         blocks: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    _check_shapes(q, k, v)
    O = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    LSE = torch.empty(q.shape[:3], dtype=torch.float32, device=q.device)
    _nfa._forward_into(q, k, v, O, LSE, causal=causal, sliding_window=window, alibi=alibi,
                       scale=scale, soft_cap=soft_cap, masks=_as_masks(causal, rows, cols, blocks))
    return O, LSE


def _as_masks(causal, rows, cols, blocks):
    if rows is None and cols is None and blocks is None:
        return None
    return _nfa._Masks(causal, rows, cols, blocks)


@_fwd.register_fake
def _fwd_fake(q, k, v, alibi, scale, causal, window, soft_cap, rows=None, cols=None, blocks=None):
    _check_shapes(q, k, v)
    return q.new_empty(q.shape), q.new_empty(q.shape[:3], dtype=torch.float32)


@torch.library.custom_op(f"{_NS}::bwd", mutates_args=(), device_types="cuda")
def _bwd(do: torch.Tensor, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, o: torch.Tensor,
         lse: torch.Tensor, alibi: Optional[torch.Tensor], scale: float, causal: bool, window: int,
         soft_cap: float, rows: Optional[torch.Tensor] = None, cols: Optional[torch.Tensor] = None,
         blocks: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    _check_shapes(q, k, v)
    DQ = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    DK = torch.empty(k.shape, dtype=k.dtype, device=k.device)
    DV = torch.empty(v.shape, dtype=v.dtype, device=v.device)
    _nfa._backward_into(q, k, v, o, lse, do, DQ, DK, DV, causal=causal, sliding_window=window,
                        alibi=alibi, scale=scale, soft_cap=soft_cap, masks=_as_masks(causal, rows, cols, blocks))
    return DQ, DK, DV


@_bwd.register_fake
def _bwd_fake(do, q, k, v, o, lse, alibi, scale, causal, window, soft_cap, rows=None, cols=None, blocks=None):
    _check_shapes(q, k, v)
    return q.new_empty(q.shape), k.new_empty(k.shape), v.new_empty(v.shape)


def _setup_context(ctx, inputs, output):
    q, k, v, alibi, scale, causal, window, soft_cap, rows, cols, blocks = inputs
    o, lse = output
    ctx.mark_non_differentiable(lse)
    ctx.save_for_backward(q, k, v, o, lse, alibi, rows, cols, blocks)
    ctx.params = (scale, causal, window, soft_cap)


def _backward(ctx, do, dlse):
    q, k, v, o, lse, alibi, rows, cols, blocks = ctx.saved_tensors
    dq, dk, dv = torch.ops.flexatt.bwd(do.contiguous(), q, k, v, o, lse, alibi, *ctx.params, rows, cols, blocks)
    return dq, dk, dv, None, None, None, None, None, None, None, None


torch.library.register_autograd(f"{_NS}::fwd", _backward, setup_context=_setup_context)


def attention(query: torch.Tensor, key: torch.Tensor, value: torch.Tensor, causal: bool = False,
              sliding_window: int = 0, alibi_slope=None, scale: Optional[float] = None,
              soft_cap: float = 0.0, document_ids: Optional[torch.Tensor] = None,
              prefix_len=None, block_mask=None) -> torch.Tensor:
    """Differentiable attention through the registered operators; returns O.

    Same arguments and defaults as ``npu_flex_attention`` (default scale
    ``1/sqrt(D)``, primitives enabled by positive values, optional
    ``document_ids``, ``prefix_len`` and ``block_mask``); usable inside
    ``torch.compile(fullgraph=True)`` with mask arguments built outside the
    compiled region or absent.
    """
    if scale is None:
        scale = 1.0 / math.sqrt(query.shape[-1])
    alibi = None
    if alibi_slope is not None:
        alibi = torch.as_tensor(alibi_slope, dtype=torch.float32, device=query.device).reshape(-1)
    window = int(sliding_window) if sliding_window and sliding_window > 0 else 0
    cap = float(soft_cap) if soft_cap and soft_cap > 0.0 else 0.0
    B, Hq, Sq, _ = query.shape
    m = _nfa._masks(causal, document_ids, prefix_len, block_mask, B, Hq, Sq, key.shape[2], query.device)
    if m is None:
        o, _ = torch.ops.flexatt.fwd(query, key, value, alibi, float(scale), bool(causal), window, cap)
    else:
        o, _ = torch.ops.flexatt.fwd(query, key, value, alibi, float(scale), m.causal, window, cap,
                                     m.rows, m.cols, m.blocks)
    return o
