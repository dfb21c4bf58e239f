"""Right-padded variable-length sigmoid attention: custom ops, autograd, API.

Mirrors the reference's operator interface (MSDLLCpapers/triton-sigmoid,
src/triton_sigmoid/sigmoid_triton_padded.py):
  * `myops::sigmoid_attn_padded_fwd` / `myops::sigmoid_attn_padded_bwd` keep
    the reference's qualified names and schemas (:517-528, :626-638);
  * autograd saves (Q, K, V, seq_lens_k, seq_lens_q, bias[, score_mod])
    (:780-846);
  * `sigmoid_attention_padded` keeps the signature, defaults and ValueError
    texts of :853-1010.  Only the first seq_lens_q[b] queries and
    seq_lens_k[b] keys of batch b are valid; padded query rows of the output
    (and of dQ) are zero, padded key rows of dK/dV are zero, and padded K/V
    rows are never read.  seq_lens are clamped to [0, T] on the device (the
    reference reads out of bounds for seq_lens > T).
"""

from __future__ import annotations

import math
from typing import Optional

import torch

from . import _capi


@torch.library.custom_op("myops::sigmoid_attn_padded_fwd", mutates_args=())
def sigmoid_attn_padded_fwd_op(
    Q: torch.Tensor,
    K: torch.Tensor,
    V: torch.Tensor,
    seq_lens_k: torch.Tensor,
    seq_lens_q: torch.Tensor,
    bias: torch.Tensor,
    score_mod: Optional[torch.Tensor],
    sm_scale: torch.Tensor,
    is_causal: bool,
) -> torch.Tensor:
    """Padded forward.  Replaces sigmoid_triton_padded.py:517-623."""
    return _capi.forward(Q, K, V, bias, score_mod, sm_scale, seq_lens_q, seq_lens_k, is_causal)


@sigmoid_attn_padded_fwd_op.register_fake
def _(Q, K, V, seq_lens_k, seq_lens_q, bias, score_mod, sm_scale, is_causal):
    return torch.empty_like(Q)


@torch.library.custom_op("myops::sigmoid_attn_padded_bwd", mutates_args=())
def sigmoid_attn_padded_bwd_op(
    Q: torch.Tensor,
    K: torch.Tensor,
    V: torch.Tensor,
    dO: torch.Tensor,
    seq_lens_k: torch.Tensor,
    seq_lens_q: torch.Tensor,
    bias: torch.Tensor,
    score_mod: Optional[torch.Tensor],
    sm_scale: torch.Tensor,
    is_causal: bool,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Padded backward.  Replaces sigmoid_triton_padded.py:626-772."""
    return _capi.backward(Q, K, V, dO, bias, score_mod, sm_scale, seq_lens_q, seq_lens_k, is_causal)


@sigmoid_attn_padded_bwd_op.register_fake
def _(Q, K, V, dO, seq_lens_k, seq_lens_q, bias, score_mod, sm_scale, is_causal):
    return torch.empty_like(Q), torch.empty_like(K), torch.empty_like(V)


def _padded_setup_context(ctx, inputs, output):
    """sigmoid_triton_padded.py:817-839 (O is recomputed, not saved)."""
    Q, K, V, seq_lens_k, seq_lens_q, bias, score_mod, sm_scale, is_causal = inputs
    ctx.has_score_mod = score_mod is not None
    saved = [Q, K, V, seq_lens_k, seq_lens_q, bias, sm_scale]
    if ctx.has_score_mod:
        saved.append(score_mod)
    ctx.save_for_backward(*saved)
    ctx.is_causal = is_causal


def _padded_backward(ctx, dO):
    """Returns (dQ, dK, dV, None x 6) like sigmoid_triton_padded.py:780-814."""
    saved = ctx.saved_tensors
    Q, K, V, seq_lens_k, seq_lens_q, bias, sm_scale = saved[:7]
    score_mod = saved[7] if ctx.has_score_mod else None
    dQ, dK, dV = sigmoid_attn_padded_bwd_op(
        Q, K, V, dO, seq_lens_k, seq_lens_q, bias, score_mod, sm_scale, ctx.is_causal
    )
    return dQ, dK, dV, None, None, None, None, None, None


sigmoid_attn_padded_fwd_op.register_autograd(_padded_backward, setup_context=_padded_setup_context)


class _PaddedEager(torch.autograd.Function):
    """Eager-mode path of sigmoid_attention_padded when the C++ autograd node
    (_capi.autograd_node) is not used: the same kernels, saved
    tensors and gradients as myops::sigmoid_attn_padded_fwd with its
    registered autograd, without the custom-op dispatch.  torch.compile
    traces the registered op."""

    @staticmethod
    def forward(ctx, Q, K, V, seq_lens_k, seq_lens_q, bias, score_mod, sm_scale, is_causal):
        out, ctx.problem = _capi.forward_eager(Q, K, V, bias, score_mod, sm_scale, seq_lens_q, seq_lens_k,
                                               is_causal)
        _padded_setup_context(ctx, (Q, K, V, seq_lens_k, seq_lens_q, bias, score_mod, sm_scale, is_causal), out)
        return out

    @staticmethod
    def backward(ctx, dO):
        saved = ctx.saved_tensors
        Q, K, V, seq_lens_k, seq_lens_q, bias, sm_scale = saved[:7]
        score_mod = saved[7] if ctx.has_score_mod else None
        dQ, dK, dV = _capi.backward_eager(ctx.problem, Q, K, V, dO, bias, score_mod, sm_scale, seq_lens_q,
                                          seq_lens_k, ctx.is_causal)
        return dQ, dK, dV, None, None, None, None, None, None


def sigmoid_attention_padded(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    seq_lens_k: Optional[torch.Tensor] = None,
    seq_lens_q: Optional[torch.Tensor] = None,
    is_causal: bool = False,
    scale: Optional[float] = None,
    sigmoid_bias: Optional[float] = None,
    score_mod: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Sigmoid attention for right-padded variable-length batches, with autograd.

    output = sigmoid(Q·Kᵀ·scale + sigmoid_bias + score_mod[k_idx]) · V

    Args:
        query: [B, T_q, H, D]; key, value: [B, T_k, H, D] (T_q may differ from T_k).
        seq_lens_k / seq_lens_q: optional [B] valid lengths (any integer dtype,
            converted to int32); None means every position is valid.
        is_causal: query i attends to keys j <= i (absolute indices).
        scale: default 1/sqrt(D).
        sigmoid_bias: default -log(seq_lens_k[b]) per batch element.
        score_mod: optional [B, T_k] per-key bias; receives no gradient.

    Returns:
        [B, T_q, H, D] output; rows at or past seq_lens_q[b] are zero.
    """
    if query.dim() != 4 or key.dim() != 4 or value.dim() != 4:
        raise ValueError("Expected query, key, and value to be 4D tensors")

    B, T_q, H, D = query.shape
    B_k, T_k, H_k, D_k = key.shape
    B_v, T_v, H_v, D_v = value.shape
    if B != B_k or B != B_v:
        raise ValueError(f"Batch size mismatch: Q={B}, K={B_k}, V={B_v}")
    if H != H_k or H != H_v:
        raise ValueError(f"Number of heads mismatch: Q={H}, K={H_k}, V={H_v}")
    if D != D_k or D != D_v:
        raise ValueError(f"Head dimension mismatch: Q={D}, K={D_k}, V={D_v}")
    if T_k != T_v:
        raise ValueError(f"Key and value sequence lengths must match, got K={T_k}, V={T_v}")

    if seq_lens_k is None:
        seq_lens_k = _capi.device_constant((B,), T_k, torch.int32, query.device)
    else:
        if seq_lens_k.shape != (B,):
            raise ValueError(f"seq_lens_k must have shape ({B},), got {seq_lens_k.shape}")
        if seq_lens_k.dtype != torch.int32:
            seq_lens_k = seq_lens_k.to(torch.int32)
        seq_lens_k = seq_lens_k.contiguous()

    if seq_lens_q is None:
        seq_lens_q = _capi.device_constant((B,), T_q, torch.int32, query.device)
    else:
        if seq_lens_q.shape != (B,):
            raise ValueError(f"seq_lens_q must have shape ({B},), got {seq_lens_q.shape}")
        if seq_lens_q.dtype != torch.int32:
            seq_lens_q = seq_lens_q.to(torch.int32)
        seq_lens_q = seq_lens_q.contiguous()

    if score_mod is not None:
        if score_mod.shape != (B, T_k):
            raise ValueError(f"score_mod must have shape ({B}, {T_k}), got {score_mod.shape}")
        score_mod = score_mod.contiguous()

    query, key, value = query.contiguous(), key.contiguous(), value.contiguous()
    if torch.compiler.is_compiling():
        # Heads and head_dim are static; sequence lengths stay dynamic so one
        # compiled graph serves every Lmax.
        for x in (query, key, value):
            torch._dynamo.mark_static(x, -2)
            torch._dynamo.mark_static(x, -1)

    # Default bias -log(seq_lens_k) with no epsilon (sigmoid_triton_padded.py:995-996).
    if sigmoid_bias is None:
        bias = -torch.log(seq_lens_k.to(device=query.device, dtype=torch.float32))
    else:
        bias = _capi.device_constant((B,), float(sigmoid_bias), torch.float32, query.device)

    if scale is None:
        scale = 1.0 / math.sqrt(D)
    scale_tensor = _capi.device_constant((), float(scale), torch.float32, query.device)
    if torch.compiler.is_compiling():
        return sigmoid_attn_padded_fwd_op(query, key, value, seq_lens_k, seq_lens_q, bias, score_mod, scale_tensor,
                                          is_causal)
    node = _capi.autograd_node()
    if node is not None:
        return _capi.attention_node(node, query, key, value, bias, score_mod, scale_tensor, seq_lens_q, seq_lens_k,
                                    is_causal)
    return _PaddedEager.apply(query, key, value, seq_lens_k, seq_lens_q, bias, score_mod, scale_tensor, is_causal)
