"""Dense (same-length) sigmoid attention: custom ops, autograd and public API.

Mirrors the reference's operator interface (MSDLLCpapers/triton-sigmoid,
src/triton_sigmoid/sigmoid_triton_dense.py):
  * `myops::sigmoid_attention_fwd` / `myops::sigmoid_attention_bwd` keep the
    reference's qualified names and schemas (:475-484, :565-575), registered
    with torch.library.custom_op plus fake (meta) kernels so torch.compile
    traces them without graph breaks;
  * autograd saves (Q, K, V, bias[, score_mod]) and recomputes P in the
    backward (:696-753);
  * `sigmoid_attention` keeps the signature, defaults and ValueError texts of
    :761-853.
The op bodies call the gfx950 kernels through the C ABI (`_capi`).
"""

from __future__ import annotations

import math
from typing import Optional

import torch

from . import _capi


@torch.library.custom_op("myops::sigmoid_attention_fwd", mutates_args=())
def sigmoid_attention_fwd_op(
    Q: torch.Tensor,
    K: torch.Tensor,
    V: torch.Tensor,
    bias: torch.Tensor,
    score_mod: Optional[torch.Tensor],
    sm_scale: torch.Tensor,
    is_causal: bool,
) -> torch.Tensor:
    """O[B,T,H,D] = sigmoid(Q·Kᵀ·sm_scale + bias[b] + score_mod[b,k]) · V.

    Replaces sigmoid_triton_dense.py:475-562 (op body and kernel launch)."""
    return _capi.forward(Q, K, V, bias, score_mod, sm_scale, None, None, is_causal)


@sigmoid_attention_fwd_op.register_fake
def _(Q, K, V, bias, score_mod, sm_scale, is_causal):
    return torch.empty_like(Q)


@torch.library.custom_op("myops::sigmoid_attention_bwd", mutates_args=())
def sigmoid_attention_bwd_op(
    Q: torch.Tensor,
    K: torch.Tensor,
    V: torch.Tensor,
    dO: torch.Tensor,
    bias: torch.Tensor,
    score_mod: Optional[torch.Tensor],
    sm_scale: torch.Tensor,
    is_causal: bool,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(dQ, dK, dV) by recomputation.  Replaces sigmoid_triton_dense.py:565-688."""
    return _capi.backward(Q, K, V, dO, bias, score_mod, sm_scale, None, None, is_causal)


@sigmoid_attention_bwd_op.register_fake
def _(Q, K, V, dO, bias, score_mod, sm_scale, is_causal):
    return torch.empty_like(Q), torch.empty_like(K), torch.empty_like(V)


def _dense_setup_context(ctx, inputs, output):
    """Saves what the recompute backward needs; O is not saved
    (sigmoid_triton_dense.py:727-746)."""
    Q, K, V, bias, score_mod, sm_scale, is_causal = inputs
    ctx.has_score_mod = score_mod is not None
    if ctx.has_score_mod:
        ctx.save_for_backward(Q, K, V, bias, sm_scale, score_mod)
    else:
        ctx.save_for_backward(Q, K, V, bias, sm_scale)
    ctx.is_causal = is_causal


def _dense_backward(ctx, dO):
    """Returns (dQ, dK, dV, None x 4) like sigmoid_triton_dense.py:696-724."""
    if ctx.has_score_mod:
        Q, K, V, bias, sm_scale, score_mod = ctx.saved_tensors
    else:
        Q, K, V, bias, sm_scale = ctx.saved_tensors
        score_mod = None
    dQ, dK, dV = sigmoid_attention_bwd_op(Q, K, V, dO, bias, score_mod, sm_scale, ctx.is_causal)
    return dQ, dK, dV, None, None, None, None


sigmoid_attention_fwd_op.register_autograd(_dense_backward, setup_context=_dense_setup_context)


class _DenseEager(torch.autograd.Function):
    """Eager-mode path of sigmoid_attention when the C++ autograd node
    (_capi.autograd_node) is not used: the same kernels, saved tensors and
    gradients as myops::sigmoid_attention_fwd with its registered autograd,
    without the custom-op dispatch (which costs more host time per call than
    a small problem's kernels take).  torch.compile traces the registered op."""

    @staticmethod
    def forward(ctx, Q, K, V, bias, score_mod, sm_scale, is_causal):
        out, ctx.problem = _capi.forward_eager(Q, K, V, bias, score_mod, sm_scale, None, None, is_causal)
        _dense_setup_context(ctx, (Q, K, V, bias, score_mod, sm_scale, is_causal), out)
        return out

    @staticmethod
    def backward(ctx, dO):
        if ctx.has_score_mod:
            Q, K, V, bias, sm_scale, score_mod = ctx.saved_tensors
        else:
            Q, K, V, bias, sm_scale = ctx.saved_tensors
            score_mod = None
        dQ, dK, dV = _capi.backward_eager(ctx.problem, Q, K, V, dO, bias, score_mod, sm_scale, None, None,
                                          ctx.is_causal)
        return dQ, dK, dV, None, None, None, None


def sigmoid_attention(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    is_causal: bool = False,
    scale: Optional[float] = None,
    sigmoid_bias: Optional[float] = None,
    score_mod: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Sigmoid attention for dense (same-length) sequences, with autograd.

    output = sigmoid(Q·Kᵀ·scale + sigmoid_bias + score_mod[k_idx]) · V

    Args:
        query, key, value: [B, T, H, D] tensors (float16, bfloat16 or float32)
            on a gfx950 GPU.
        is_causal: query i attends to keys j <= i.
        scale: score scale, default 1/sqrt(D).
        sigmoid_bias: scalar added to every score, default -log(T).
        score_mod: optional [B, T] per-key bias added after sigmoid_bias,
            broadcast over queries and heads; receives no gradient.

    Returns:
        [B, T, H, D] output in the input dtype.
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
    if T_q != T_k or T_q != T_v:
        raise ValueError(
            f"Dense attention requires same sequence length for Q, K, V, got {T_q}, {T_k}, {T_v}"
        )
    if score_mod is not None:
        if score_mod.shape != (B, T_k):
            raise ValueError(f"score_mod must have shape ({B}, {T_k}), got {score_mod.shape}")
        score_mod = score_mod.contiguous()

    query, key, value = query.contiguous(), key.contiguous(), value.contiguous()
    if torch.compiler.is_compiling():
        for x in (query, key, value):
            torch._dynamo.mark_static(x, -2)  # heads
            torch._dynamo.mark_static(x, -1)  # head_dim

    T = T_q
    # Default bias is -log(T) with no epsilon, as sigmoid_triton_dense.py:840-841.
    if sigmoid_bias is not None:
        bias_value = float(sigmoid_bias)
    else:
        bias_value = -math.log(float(T)) if T > 0 else 0.0  # T == 0: nothing is computed
    bias = _capi.device_constant((B,), bias_value, torch.float32, query.device)
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    scale_tensor = _capi.device_constant((), float(scale), torch.float32, query.device)
    if torch.compiler.is_compiling():
        return sigmoid_attention_fwd_op(query, key, value, bias, score_mod, scale_tensor, is_causal)
    node = _capi.autograd_node()
    if node is not None:
        return _capi.attention_node(node, query, key, value, bias, score_mod, scale_tensor, None, None, is_causal)
    return _DenseEager.apply(query, key, value, bias, score_mod, scale_tensor, is_causal)
