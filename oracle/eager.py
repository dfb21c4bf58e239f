"""TEST INFRASTRUCTURE ONLY — eager PyTorch restatement of the reference's
`sigmoid_attention_ref` (MSDLLCpapers/triton-sigmoid,
src/triton_sigmoid/sigmoid_reference.py:16-152).

Used by tests/ as the reference-style error baseline (the reference's tests
compare the kernel's error against the error of the mixed-precision eager path,
tests/test_sigmoid_dense.py:77-114) and by bench.py's cpu_baseline leg, where
its fp32 forward + autograd backward is timed on the host cores.  The product
path never imports it.  `mixed_fwd_bwd` is the mixed-precision path with its
backward written out on contiguous operands, for GPU runs in bf16 / fp16.

Follows sigmoid_reference.py line by line in behaviour:
  padding masks from seq_lens (:59-70); bias = sigmoid_bias or
  -log(valid_keys + 1e-6) (:73-80); upcast=True: fp32 throughout (:82-114);
  upcast=False: Q·Kᵀ in the input dtype, `*1.0 + bias` promotion, sigmoid,
  P cast to the input dtype, P·V in the input dtype (:116-148); reorder_ops
  scales K instead of Q (:89-92); causal triu(1) -> -inf (:100-102); key mask
  after the sigmoid (:106-108); query rows zeroed (:112-114).
"""

from __future__ import annotations

import math
from typing import Optional

import torch


def sigmoid_attention_eager(q, k, v, seq_lens_k: Optional[torch.Tensor] = None,
                            seq_lens_q: Optional[torch.Tensor] = None,
                            scale: Optional[float] = None, sigmoid_bias: Optional[float] = None,
                            upcast: bool = True, reorder_ops: bool = False, causal: bool = False,
                            score_mod: Optional[torch.Tensor] = None) -> torch.Tensor:
    B, Lq, H, D = q.shape
    Lk = k.shape[1]
    dev = q.device
    dtype_og = q.dtype
    if scale is None:
        scale = 1.0 / math.sqrt(D)

    kmask = None
    if seq_lens_k is not None:
        kmask = torch.arange(Lk, device=dev).unsqueeze(0) >= seq_lens_k.to(dev).unsqueeze(1)
    qmask = None
    if seq_lens_q is not None:
        qmask = torch.arange(Lq, device=dev).unsqueeze(0) >= seq_lens_q.to(dev).unsqueeze(1)

    if sigmoid_bias is not None:
        bias = sigmoid_bias
    elif seq_lens_k is not None:
        bias = -torch.log(seq_lens_k.to(dev).float() + 1e-6).view(B, 1, 1, 1)
    else:
        bias = -math.log(float(Lk) + 1e-6)

    if upcast:
        q, k, v = q.float(), k.float(), v.float()
    if reorder_ops:
        logits = torch.einsum("bqhd,bkhd->bhqk", q, k * scale)
    else:
        logits = torch.einsum("bqhd,bkhd->bhqk", q * scale, k)
    logits = logits + bias if upcast else logits * 1.0 + bias
    if score_mod is not None:
        logits = logits + score_mod.view(B, 1, 1, Lk)
    if causal:
        tri = torch.triu(torch.ones(Lq, Lk, dtype=torch.bool, device=dev), diagonal=1)
        logits = logits.masked_fill(tri[None, None], float("-inf"))
    attn = torch.sigmoid(logits)
    if kmask is not None:
        attn = attn.masked_fill(kmask.view(B, 1, 1, Lk), 0.0)
    if not upcast:
        attn = attn.to(dtype_og)
    out = torch.einsum("bhqk,bkhd->bqhd", attn, v)
    if qmask is not None:
        out = out.masked_fill(qmask.view(B, Lq, 1, 1), 0.0)
    return out.to(dtype_og)


def fwd_bwd_fp32(q, k, v, dout, causal=False, scale=None, sigmoid_bias=None,
                 seq_lens_q=None, seq_lens_k=None, score_mod=None):
    """fp32 eager forward + autograd backward; returns (O, dQ, dK, dV)."""
    q = q.detach().float().requires_grad_(True)
    k = k.detach().float().requires_grad_(True)
    v = v.detach().float().requires_grad_(True)
    o = sigmoid_attention_eager(q, k, v, seq_lens_k=seq_lens_k, seq_lens_q=seq_lens_q, scale=scale,
                                sigmoid_bias=sigmoid_bias, upcast=True, causal=causal,
                                score_mod=score_mod)
    o.backward(dout.float())
    return o.detach(), q.grad, k.grad, v.grad


def mixed_fwd_bwd(q, k, v, dout, seq_lens_k=None, seq_lens_q=None, scale=None, sigmoid_bias=None,
                  causal=False, score_mod=None):
    """The mixed-precision eager path (upcast=False, reorder_ops=True) with its
    backward written out step by step; returns (O, dQ, dK, dV).

    Same values as autograd through sigmoid_attention_eager(upcast=False,
    reorder_ops=True) up to the summation order of each matrix product: every
    product runs in the input dtype on contiguous operands (torch.matmul, no
    einsum and no transposed views, in the forward or the backward), and the
    element-wise steps keep the dtypes torch's promotion gives the eager
    expressions (`logits * 1.0 + bias` stays in the input dtype for a float
    bias and becomes fp32 for a [B] bias tensor, sigmoid_reference.py:127).
    Used where the eager path must run on a GPU in bf16 / fp16."""
    B, Lq, H, D = q.shape
    Lk = k.shape[1]
    dev, dt = q.device, q.dtype
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    kmask = qmask = None
    if seq_lens_k is not None:
        kmask = (torch.arange(Lk, device=dev).unsqueeze(0) >= seq_lens_k.to(dev).unsqueeze(1)).view(B, 1, 1, Lk)
    if seq_lens_q is not None:
        qmask = (torch.arange(Lq, device=dev).unsqueeze(0) >= seq_lens_q.to(dev).unsqueeze(1)).view(B, Lq, 1, 1)
    if sigmoid_bias is not None:
        bias = sigmoid_bias
    elif seq_lens_k is not None:
        bias = -torch.log(seq_lens_k.to(dev).float() + 1e-6).view(B, 1, 1, 1)
    else:
        bias = -math.log(float(Lk) + 1e-6)
    with torch.no_grad():
        ks = k * scale                                         # reorder_ops: K scaled
        qh = q.permute(0, 2, 1, 3).contiguous()                # [B, H, Lq, D]
        ksT = ks.permute(0, 2, 3, 1).contiguous()              # [B, H, D, Lk]
        logits = torch.matmul(qh, ksT)                         # [B, H, Lq, Lk]
        lg = logits * 1.0 + bias
        if score_mod is not None:
            lg = lg + score_mod.view(B, 1, 1, Lk)
        tri = None
        if causal:
            tri = torch.triu(torch.ones(Lq, Lk, dtype=torch.bool, device=dev), diagonal=1)[None, None]
            lg = lg.masked_fill(tri, float("-inf"))
        attn = torch.sigmoid(lg)
        if kmask is not None:
            attn = attn.masked_fill(kmask, 0.0)
        attn_d = attn.to(dt)
        vh = v.permute(0, 2, 1, 3).contiguous()                # [B, H, Lk, D]
        out = torch.matmul(attn_d, vh).permute(0, 2, 1, 3)     # [B, Lq, H, D]
        if qmask is not None:
            out = out.masked_fill(qmask, 0.0)
        out = out.to(dt)

        g = dout.to(dt)
        if qmask is not None:
            g = g.masked_fill(qmask, 0.0)
        gh = g.permute(0, 2, 1, 3).contiguous()                # [B, H, Lq, D]
        d_attn = torch.matmul(gh, v.permute(0, 2, 3, 1).contiguous())        # dO·Vᵀ
        dvh = torch.matmul(attn_d.transpose(-1, -2).contiguous(), gh)        # Pᵀ·dO
        d_attn = d_attn.to(attn.dtype)
        if kmask is not None:
            d_attn = d_attn.masked_fill(kmask, 0.0)
        d_lg = torch.ops.aten.sigmoid_backward(d_attn, attn)
        if tri is not None:
            d_lg = d_lg.masked_fill(tri, 0.0)
        d_logits = d_lg.to(logits.dtype)
        dqh = torch.matmul(d_logits, ks.permute(0, 2, 1, 3).contiguous())    # dS·(K·scale)
        dksh = torch.matmul(d_logits.transpose(-1, -2).contiguous(), qh)     # dSᵀ·Q
        dq = dqh.permute(0, 2, 1, 3).contiguous()
        dk = (dksh.permute(0, 2, 1, 3) * scale).contiguous()
        dv = dvh.permute(0, 2, 1, 3).contiguous()
    return out, dq, dk, dv
