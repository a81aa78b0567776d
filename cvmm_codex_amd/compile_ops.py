"""torch.library custom ops over the native phases, for torch.compile.

The reference registers its forward primitive as ``mylib::cvmm_triton`` with
a fake (meta) implementation (cvmm.py:808-812, :1436-1456) so that compiled
callers can trace through ``CVMM``.  Here every native phase the API calls
is an op with a fake implementation: the selector sort, the expert offsets,
the weight cast, the forward and the backward products, the router (with its
backward registered as the op's autograd formula), plus
``cvmm_codex_amd::cvmm_triton`` with the reference op's schema.  The API
routes through these ops only while torch.compile traces
(``torch.compiler.is_compiling()``); eager calls go to the host glue directly,
which costs less host time per call.  The ops run the same native code.

Ops return tensors of their own: outputs of a custom op may not alias its
inputs or each other, so the sort's outputs (views of two buffers in eager
mode) are separate tensors here, and absent gradients are empty tensors.
"""
from __future__ import annotations

from typing import List, Optional, Tuple

import torch

from . import _native as N

NS = "cvmm_codex_amd"


def _empty(like: torch.Tensor) -> torch.Tensor:
    return like.new_empty((0,))


# ---------------------------------------------------------------------------
# selector sort (cvmm.py:24-27, :1796-1803) and expert offsets (:1108-1120)
# ---------------------------------------------------------------------------
@torch.library.custom_op(f"{NS}::sort_routes", mutates_args=())
def sort_routes(raw: torch.Tensor, n_experts: int, top_k: int) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor,
                                                                          torch.Tensor, torch.Tensor]:
    """(sorted int32 [R], perm int64 [R], perm // top_k int64 [R], inclusive
    offsets int64 [E], inverse permutation int32 [R])."""
    out = N.host().sort_routes(raw.reshape(-1), n_experts, top_k, N.stream_of(raw.device))
    return tuple(t.clone() for t in out)


@sort_routes.register_fake
def _(raw, n_experts, top_k):
    R = raw.numel()
    return (raw.new_empty((R,), dtype=torch.int32), raw.new_empty((R,), dtype=torch.int64),
            raw.new_empty((R,), dtype=torch.int64), raw.new_empty((n_experts,), dtype=torch.int64),
            raw.new_empty((R,), dtype=torch.int32))


@torch.library.custom_op(f"{NS}::expert_offsets", mutates_args=())
def expert_offsets(sorted_experts: torch.Tensor, n_experts: int) -> torch.Tensor:
    return N.host().expert_offsets(sorted_experts, n_experts, N.stream_of(sorted_experts.device))


@expert_offsets.register_fake
def _(sorted_experts, n_experts):
    return sorted_experts.new_empty((n_experts,), dtype=torch.int64)


# ---------------------------------------------------------------------------
# per-step weight cast: kt [E, d_out, d_in], kn [E, d_in, d_out]
# ---------------------------------------------------------------------------
@torch.library.custom_op(f"{NS}::cast_keys", mutates_args=())
def cast_keys(keys: torch.Tensor, op_dtype: torch.dtype) -> Tuple[torch.Tensor, torch.Tensor]:
    kt, kn = N.host().cast_keys(keys, N.dtype_id(op_dtype), True, True, 0, N.stream_of(keys.device))
    return kt, kn


@cast_keys.register_fake
def _(keys, op_dtype):
    E, d_in, d_out = keys.shape
    return keys.new_empty((E, d_out, d_in), dtype=op_dtype), keys.new_empty((E, d_in, d_out), dtype=op_dtype)


# ---------------------------------------------------------------------------
# forward (cvmm.py:1524-1550): [out_rows, d_out] in the op dtype
# ---------------------------------------------------------------------------
@torch.library.custom_op(f"{NS}::forward", mutates_args=())
def forward(x: torch.Tensor, keys: torch.Tensor, keys_op: Optional[torch.Tensor], keys_op_is_t: bool,
            sel: torch.Tensor, sel_index: torch.Tensor, out_index: Optional[torch.Tensor], offsets: torch.Tensor,
            reduction_weight: Optional[torch.Tensor], op_dtype: torch.dtype, flags: int) -> torch.Tensor:
    return N.host().forward(x, keys, keys_op, keys_op_is_t, sel, sel_index, out_index, offsets, None,
                            reduction_weight, N.dtype_id(op_dtype), -1, flags, N.stream_of(x.device))


@forward.register_fake
def _(x, keys, keys_op, keys_op_is_t, sel, sel_index, out_index, offsets, reduction_weight, op_dtype, flags):
    R = sel.numel()
    rows = R if reduction_weight is None else R // reduction_weight.shape[-1]
    return x.new_empty((rows, keys.shape[2]), dtype=op_dtype)


# ---------------------------------------------------------------------------
# backward (cvmm.py:1552-1755): (grad x, grad keys, grad reduction weight),
# an empty tensor for a gradient that is not wanted
# ---------------------------------------------------------------------------
@torch.library.custom_op(f"{NS}::backward", mutates_args=())
def backward(grad_output: torch.Tensor, x: torch.Tensor, keys: torch.Tensor, keys_x: Optional[torch.Tensor],
             keys_x_is_t: bool, sel: torch.Tensor, sel_index: torch.Tensor, out_index: Optional[torch.Tensor],
             offsets: torch.Tensor,
             reduction_weight: Optional[torch.Tensor], top_k: int, op_dtype: torch.dtype, need_grad_x: bool,
             need_grad_keys: bool, need_grad_rw: bool, flags: int) -> Tuple[torch.Tensor, torch.Tensor,
                                                                             torch.Tensor]:
    gx, gw, grw = N.host().backward(grad_output, x, keys, keys_x, keys_x_is_t, sel, sel_index, out_index, offsets,
                                    None,
                                    reduction_weight, top_k, N.dtype_id(op_dtype), need_grad_x, need_grad_keys,
                                    need_grad_rw, flags, N.stream_of(x.device))
    return (gx if gx is not None else _empty(x), gw if gw is not None else _empty(keys),
            grw if grw is not None else _empty(x))


@backward.register_fake
def _(grad_output, x, keys, keys_x, keys_x_is_t, sel, sel_index, out_index, offsets, reduction_weight, top_k, op_dtype,
      need_grad_x, need_grad_keys, need_grad_rw, flags):
    # the real op's grad_x is always a fresh contiguous tensor of x's shape
    gx = x.new_empty(x.shape) if need_grad_x else _empty(x)
    gw = torch.empty_like(keys, memory_format=torch.contiguous_format) if need_grad_keys else _empty(keys)
    grw = (torch.empty_like(reduction_weight, memory_format=torch.contiguous_format)
           if need_grad_rw and reduction_weight is not None else _empty(x))
    return gx, gw, grw


def grads_or_none(g: Tuple[torch.Tensor, torch.Tensor, torch.Tensor], need: List[bool]):
    return tuple(t if n else None for t, n in zip(g, need))


# ---------------------------------------------------------------------------
# the reference op's schema (cvmm.py:809): per-route forward, out_index = a
# one-element tensor holding -1 for "none"
# ---------------------------------------------------------------------------
@torch.library.custom_op(f"{NS}::cvmm_triton", mutates_args=())
def cvmm_triton(x: torch.Tensor, sel_index: torch.Tensor, sel: torch.Tensor, keys: torch.Tensor,
                out_dtype: torch.dtype, out_index: torch.Tensor, op_dtype: torch.dtype) -> torch.Tensor:
    # one-element out_index holding -1 = "none" (cvmm.py:845-846); with more
    # than one route a real out_index has more entries, so only a one-route
    # selection needs its value read (a host sync, as in the reference)
    R = sel.numel()
    sentinel = out_index.numel() == 1 and (R != 1 or int(out_index.item()) == -1)
    oi = None if sentinel else out_index
    s32 = sel.reshape(-1).to(torch.int32)
    off = N.host().expert_offsets(s32, keys.shape[0], N.stream_of(x.device))
    # products rounded once, straight to out_dtype (cvmm.py:832-833, :862-863)
    out = N.host().forward(x, keys, None, True, s32, sel_index, oi, off, None, None, N.dtype_id(op_dtype),
                           N.dtype_id(out_dtype), 0, N.stream_of(x.device))
    return out.view(*sel.shape, keys.shape[2])


@cvmm_triton.register_fake
def _(x, sel_index, sel, keys, out_dtype, out_index, op_dtype):
    return x.new_empty((*sel.shape, keys.shape[2]), dtype=out_dtype)


# ---------------------------------------------------------------------------
# router (its callers' softmax -> top-k -> renormalise -> sort, see
# api.cvmm_route_topk): weights fp32 [T, k], sel int64 [T, k], then the sort's
# sorted int32, perm, perm // k, offsets and inverse permutation
# ---------------------------------------------------------------------------
@torch.library.custom_op(f"{NS}::route_topk", mutates_args=())
def route_topk(logits: torch.Tensor, top_k: int, renormalize: bool) -> Tuple[torch.Tensor, torch.Tensor,
                                                                            torch.Tensor, torch.Tensor,
                                                                            torch.Tensor, torch.Tensor,
                                                                            torch.Tensor]:
    out = N.host().route_topk(logits, top_k, renormalize, N.stream_of(logits.device))
    return tuple(t.clone() for t in out)


@route_topk.register_fake
def _(logits, top_k, renormalize):
    T = logits.numel() // logits.shape[-1]
    E = logits.shape[-1]
    R = T * top_k
    return (logits.new_empty((T, top_k), dtype=torch.float32), logits.new_empty((T, top_k), dtype=torch.int64),
            logits.new_empty((R,), dtype=torch.int32), logits.new_empty((R,), dtype=torch.int64),
            logits.new_empty((R,), dtype=torch.int64), logits.new_empty((E,), dtype=torch.int64),
            logits.new_empty((R,), dtype=torch.int32))


@torch.library.custom_op(f"{NS}::route_topk_backward", mutates_args=())
def route_topk_backward(logits: torch.Tensor, sel: torch.Tensor, grad_weights: torch.Tensor, top_k: int,
                        renormalize: bool) -> torch.Tensor:
    return N.host().route_topk_backward(logits, sel, grad_weights, top_k, renormalize, N.stream_of(logits.device))


@route_topk_backward.register_fake
def _(logits, sel, grad_weights, top_k, renormalize):
    return torch.empty_like(logits, memory_format=torch.contiguous_format)


def _route_setup(ctx, inputs, output):
    logits, top_k, renormalize = inputs
    ctx.save_for_backward(logits, output[1])
    ctx.top_k, ctx.renormalize = top_k, renormalize


def _route_backward(ctx, grad_w, *_):
    logits, sel = ctx.saved_tensors
    if grad_w is None:
        return None, None, None
    return route_topk_backward(logits, sel, grad_w.contiguous(), ctx.top_k, ctx.renormalize), None, None


route_topk.register_autograd(_route_backward, setup_context=_route_setup)
