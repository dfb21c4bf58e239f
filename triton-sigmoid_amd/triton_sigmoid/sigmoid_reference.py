"""Eager PyTorch sigmoid attention (public `sigmoid_attention_ref`).

Same signature and semantics as the reference's `sigmoid_attention_ref`
(MSDLLCpapers/triton-sigmoid, src/triton_sigmoid/sigmoid_reference.py:16-152):
  * upcast=True: everything in fp32;
  * upcast=False: Q·Kᵀ in the input dtype, bias/score_mod/sigmoid in fp32,
    P cast back to the input dtype before P·V;
  * reorder_ops scales K instead of Q;
  * default bias is -log(valid_keys + 1e-6);
  * causal masks key > query (top-left aligned) with -inf before the sigmoid,
    padded keys get P = 0 after it, padded query rows are zeroed.
It materialises [B, H, Tq, Tk] scores and runs on any device; it is the
readable definition of the operator, not a fast path.
"""

from __future__ import annotations

import math
from typing import Optional

import torch


def sigmoid_attention_ref(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    seq_lens_k: Optional[torch.Tensor] = None,
    seq_lens_q: Optional[torch.Tensor] = None,
    scale: Optional[float] = None,
    sigmoid_bias: Optional[float] = None,
    upcast: bool = True,
    reorder_ops: bool = False,
    causal: bool = False,
    score_mod: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """Eager sigmoid attention on [B, T, H, D] tensors; returns [B, Tq, H, D]."""
    B, Lq, H, D = q.shape
    Lk = k.shape[1]
    dev = q.device
    out_dtype = q.dtype
    if scale is None:
        scale = 1.0 / math.sqrt(D)

    key_pad = None
    if seq_lens_k is not None:
        key_pad = torch.arange(Lk, device=dev)[None, :] >= seq_lens_k.to(dev)[:, None]  # [B, Lk]
    query_pad = None
    if seq_lens_q is not None:
        query_pad = torch.arange(Lq, device=dev)[None, :] >= seq_lens_q.to(dev)[:, None]  # [B, Lq]

    if sigmoid_bias is not None:
        bias = sigmoid_bias
    elif seq_lens_k is not None:
        bias = -torch.log(seq_lens_k.to(dev).float() + 1e-6).view(B, 1, 1, 1)
    else:
        bias = -math.log(float(Lk) + 1e-6)

    if upcast:
        q, k, v = q.float(), k.float(), v.float()
    qs, ks = (q, k * scale) if reorder_ops else (q * scale, k)
    logits = torch.einsum("bqhd,bkhd->bhqk", qs, ks)
    # Mixed mode: the product is in the input dtype; adding a tensor bias
    # (padded case) promotes to fp32, a Python-float bias keeps the input
    # dtype, exactly as torch type promotion does in the reference.
    logits = logits * 1.0 + bias
    if score_mod is not None:
        logits = logits + score_mod.view(B, 1, 1, Lk)
    if causal:
        above = torch.ones(Lq, Lk, dtype=torch.bool, device=dev).triu(1)
        logits = logits.masked_fill(above, float("-inf"))
    attn = torch.sigmoid(logits)
    if key_pad is not None:
        attn = attn.masked_fill(key_pad.view(B, 1, 1, Lk), 0.0)
    if not upcast:
        attn = attn.to(out_dtype)
    out = torch.einsum("bhqk,bkhd->bqhd", attn, v)
    if query_pad is not None:
        out = out.masked_fill(query_pad.view(B, Lq, 1, 1), 0.0)
    return out.to(out_dtype)
