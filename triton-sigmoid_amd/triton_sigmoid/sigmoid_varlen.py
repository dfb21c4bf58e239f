"""Packed variable-length (THD) sigmoid attention: custom ops, autograd, API.

The reference's operator set has no packed layout; its benchmark builds one
for flash_attn_varlen_func (MSDLLCpapers/triton-sigmoid,
benchmarks/benchmark_sigmoid.py:116-134: q, k, v as [total_tokens, H, D] plus
int32 cu_seqlens = [0, cumsum(seq_lens)]).  This module accepts that layout
and computes exactly what `sigmoid_attention_padded` computes for the same
sequences (sigmoid_triton_padded.py:853-1010): sequence b is rows
cu_seqlens[b] .. cu_seqlens[b+1]-1, attends only within itself (top-left
causal when is_causal), and its default bias is -log(its key length) with no
epsilon (sigmoid_triton_padded.py:995-996).  No padding exists, so no padding
is read, computed or written.

Ops: `myops::sigmoid_attn_varlen_fwd` / `myops::sigmoid_attn_varlen_bwd`
(the padded ops' schemas with cu_seqlens in place of seq_lens and the two
max_seqlen integers), with register_fake and register_autograd so
torch.compile traces them without graph breaks.
"""

from __future__ import annotations

import math
from typing import Optional

import torch

from . import _capi


@torch.library.custom_op("myops::sigmoid_attn_varlen_fwd", mutates_args=())
def sigmoid_attn_varlen_fwd_op(
    Q: torch.Tensor,
    K: torch.Tensor,
    V: torch.Tensor,
    cu_seqlens_k: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    max_seqlen_k: int,
    max_seqlen_q: int,
    bias: torch.Tensor,
    score_mod: Optional[torch.Tensor],
    sm_scale: torch.Tensor,
    is_causal: bool,
) -> torch.Tensor:
    """Packed forward (the padded forward of sigmoid_triton_padded.py:517-623
    on packed rows)."""
    return _capi.forward_packed(Q, K, V, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, bias,
                                score_mod, sm_scale, is_causal)


@sigmoid_attn_varlen_fwd_op.register_fake
def _(Q, K, V, cu_seqlens_k, cu_seqlens_q, max_seqlen_k, max_seqlen_q, bias, score_mod, sm_scale, is_causal):
    return torch.empty_like(Q)


@torch.library.custom_op("myops::sigmoid_attn_varlen_bwd", mutates_args=())
def sigmoid_attn_varlen_bwd_op(
    Q: torch.Tensor,
    K: torch.Tensor,
    V: torch.Tensor,
    dO: torch.Tensor,
    cu_seqlens_k: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    max_seqlen_k: int,
    max_seqlen_q: int,
    bias: torch.Tensor,
    score_mod: Optional[torch.Tensor],
    sm_scale: torch.Tensor,
    is_causal: bool,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Packed backward (the padded backward of sigmoid_triton_padded.py:626-772
    on packed rows)."""
    return _capi.backward_packed(Q, K, V, dO, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, bias,
                                 score_mod, sm_scale, is_causal)


@sigmoid_attn_varlen_bwd_op.register_fake
def _(Q, K, V, dO, cu_seqlens_k, cu_seqlens_q, max_seqlen_k, max_seqlen_q, bias, score_mod, sm_scale,
      is_causal):
    return torch.empty_like(Q), torch.empty_like(K), torch.empty_like(V)


def _varlen_setup_context(ctx, inputs, output):
    """Saves what the padded op saves (sigmoid_triton_padded.py:817-839), with
    cu_seqlens for seq_lens; O is recomputed, not saved."""
    Q, K, V, cu_seqlens_k, cu_seqlens_q, max_seqlen_k, max_seqlen_q, bias, score_mod, sm_scale, is_causal = inputs
    ctx.has_score_mod = score_mod is not None
    saved = [Q, K, V, cu_seqlens_k, cu_seqlens_q, bias, sm_scale]
    if ctx.has_score_mod:
        saved.append(score_mod)
    ctx.save_for_backward(*saved)
    ctx.max_seqlen_k, ctx.max_seqlen_q = max_seqlen_k, max_seqlen_q
    ctx.is_causal = is_causal


def _varlen_backward(ctx, dO):
    """Returns (dQ, dK, dV, None x 8)."""
    saved = ctx.saved_tensors
    Q, K, V, cu_seqlens_k, cu_seqlens_q, bias, sm_scale = saved[:7]
    score_mod = saved[7] if ctx.has_score_mod else None
    dQ, dK, dV = sigmoid_attn_varlen_bwd_op(
        Q, K, V, dO, cu_seqlens_k, cu_seqlens_q, ctx.max_seqlen_k, ctx.max_seqlen_q, bias, score_mod,
        sm_scale, ctx.is_causal
    )
    return dQ, dK, dV, None, None, None, None, None, None, None, None


sigmoid_attn_varlen_fwd_op.register_autograd(_varlen_backward, setup_context=_varlen_setup_context)


class _VarlenEager(torch.autograd.Function):
    """Eager-mode path of sigmoid_attention_varlen when the C++ autograd node
    (_capi.autograd_node) is not used: the same kernels, saved
    tensors and gradients as myops::sigmoid_attn_varlen_fwd with its
    registered autograd, without the custom-op dispatch.  torch.compile
    traces the registered op."""

    @staticmethod
    def forward(ctx, Q, K, V, cu_seqlens_k, cu_seqlens_q, max_seqlen_k, max_seqlen_q, bias, score_mod, sm_scale,
                is_causal):
        out = _capi.forward_packed(Q, K, V, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k, bias,
                                   score_mod, sm_scale, is_causal)
        _varlen_setup_context(ctx, (Q, K, V, cu_seqlens_k, cu_seqlens_q, max_seqlen_k, max_seqlen_q, bias,
                                    score_mod, sm_scale, is_causal), out)
        return out

    @staticmethod
    def backward(ctx, dO):
        saved = ctx.saved_tensors
        Q, K, V, cu_seqlens_k, cu_seqlens_q, bias, sm_scale = saved[:7]
        score_mod = saved[7] if ctx.has_score_mod else None
        dQ, dK, dV = _capi.backward_packed(Q, K, V, dO, cu_seqlens_q, cu_seqlens_k, ctx.max_seqlen_q,
                                           ctx.max_seqlen_k, bias, score_mod, sm_scale, ctx.is_causal)
        return dQ, dK, dV, None, None, None, None, None, None, None, None


def _check_cu(name: str, cu: torch.Tensor) -> torch.Tensor:
    if cu.dim() != 1 or cu.numel() < 1:
        raise ValueError(f"{name} must have shape (B + 1,), got {cu.shape}")
    if cu.dtype != torch.int32:
        cu = cu.to(torch.int32)
    return cu.contiguous()


def sigmoid_attention_varlen(
    query: torch.Tensor,
    key: torch.Tensor,
    value: torch.Tensor,
    cu_seqlens_q: torch.Tensor,
    cu_seqlens_k: torch.Tensor,
    max_seqlen_q: Optional[int] = None,
    max_seqlen_k: Optional[int] = None,
    is_causal: bool = False,
    scale: Optional[float] = None,
    sigmoid_bias: Optional[float] = None,
    score_mod: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Sigmoid attention over packed variable-length sequences, with autograd.

    output = sigmoid(Q·Kᵀ·scale + sigmoid_bias + score_mod[k_idx]) · V within
    each sequence.

    Args:
        query: [total_q, H, D]; key, value: [total_k, H, D].
        cu_seqlens_q / cu_seqlens_k: [B + 1] non-decreasing offsets (any integer
            dtype, converted to int32) with cu[0] = 0 and cu[B] = total rows;
            sequence b is rows cu[b] .. cu[b+1]-1.
        max_seqlen_q / max_seqlen_k: the longest query / key sequence (at
            least every length: a sequence longer than it is cut to its
            first max_seqlen rows, as flash_attn_varlen_func's contract has
            it).  None reads it from cu_seqlens (one device to host copy).
        is_causal: query i of a sequence attends to its keys j <= i.
        scale: default 1/sqrt(D).
        sigmoid_bias: default -log(key length of each sequence).
        score_mod: optional [total_k] per-key bias (packed like the keys);
            receives no gradient.

    Returns:
        [total_q, H, D] output, equal row for row to what
        `sigmoid_attention_padded` returns for the same sequences.

    Rows outside every sequence -- before cu[0], past cu[B] when cu does not
    cover all rows, and past max_seqlen of a longer sequence -- are zeros in
    the output and in dQ / dK / dV (they take no part in the attention), so
    no gradient row is left uninitialised.
    """
    if query.dim() != 3 or key.dim() != 3 or value.dim() != 3:
        raise ValueError("Expected query, key, and value to be 3D tensors (total_tokens, H, D)")
    _, H, D = query.shape
    N_k, H_k, D_k = key.shape
    N_v, H_v, D_v = value.shape
    if H != H_k or H != H_v:
        raise ValueError(f"Number of heads mismatch: Q={H}, K={H_k}, V={H_v}")
    if D != D_k or D != D_v:
        raise ValueError(f"Head dimension mismatch: Q={D}, K={D_k}, V={D_v}")
    if N_k != N_v:
        raise ValueError(f"Key and value token counts must match, got K={N_k}, V={N_v}")
    cu_seqlens_q = _check_cu("cu_seqlens_q", cu_seqlens_q)
    cu_seqlens_k = _check_cu("cu_seqlens_k", cu_seqlens_k)
    if cu_seqlens_q.shape != cu_seqlens_k.shape:
        raise ValueError(f"cu_seqlens_q and cu_seqlens_k must have the same shape, got "
                         f"{cu_seqlens_q.shape} and {cu_seqlens_k.shape}")
    B = cu_seqlens_q.numel() - 1
    if score_mod is not None:
        if score_mod.shape != (N_k,):
            raise ValueError(f"score_mod must have shape ({N_k},), got {score_mod.shape}")
        score_mod = score_mod.contiguous()

    lens_k = (cu_seqlens_k[1:] - cu_seqlens_k[:-1]).to(device=query.device)
    if max_seqlen_q is None:
        max_seqlen_q = int((cu_seqlens_q[1:] - cu_seqlens_q[:-1]).max().item()) if B > 0 else 0
    if max_seqlen_k is None:
        max_seqlen_k = int(lens_k.max().item()) if B > 0 else 0
    if max_seqlen_q < 0 or max_seqlen_k < 0:
        raise ValueError(f"max_seqlen must be non-negative, got q={max_seqlen_q}, k={max_seqlen_k}")

    query, key, value = query.contiguous(), key.contiguous(), value.contiguous()
    if torch.compiler.is_compiling():
        for x in (query, key, value):
            torch._dynamo.mark_static(x, -2)
            torch._dynamo.mark_static(x, -1)

    if sigmoid_bias is None:
        bias = -torch.log(lens_k.to(torch.float32))
    else:
        bias = _capi.device_constant((B,), float(sigmoid_bias), torch.float32, query.device)
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    scale_tensor = _capi.device_constant((), float(scale), torch.float32, query.device)
    cu_seqlens_k, cu_seqlens_q = cu_seqlens_k.to(query.device), cu_seqlens_q.to(query.device)
    if torch.compiler.is_compiling():
        return sigmoid_attn_varlen_fwd_op(query, key, value, cu_seqlens_k, cu_seqlens_q, int(max_seqlen_k),
                                          int(max_seqlen_q), bias, score_mod, scale_tensor, is_causal)
    node = _capi.autograd_node()
    if node is not None:
        return _capi.attention_node_packed(node, query, key, value, cu_seqlens_q, cu_seqlens_k, max_seqlen_q,
                                           max_seqlen_k, bias, score_mod, scale_tensor, is_causal)
    return _VarlenEager.apply(query, key, value, cu_seqlens_k, cu_seqlens_q, int(max_seqlen_k), int(max_seqlen_q),
                              bias, score_mod, scale_tensor, is_causal)
