"""Fused sigmoid attention for AMD MI355X (gfx950), drop-in for triton-sigmoid.

    output = sigmoid(Q·Kᵀ·scale + bias + score_mod[k]) · V

Public API (same names and signatures as MSDLLCpapers/triton-sigmoid,
src/triton_sigmoid/__init__.py:68-78):
  * sigmoid_attention(query, key, value, is_causal, scale, sigmoid_bias, score_mod)
  * sigmoid_attention_padded(query, key, value, seq_lens_k, seq_lens_q,
                             is_causal, scale, sigmoid_bias, score_mod)
  * sigmoid_attention_ref(...)  eager PyTorch definition
plus one addition with no counterpart in the reference's API:
  * sigmoid_attention_varlen(query, key, value, cu_seqlens_q, cu_seqlens_k,
                             max_seqlen_q, max_seqlen_k, is_causal, scale,
                             sigmoid_bias, score_mod)
    for packed [total_tokens, H, D] sequences (the layout the reference's
    benchmark builds for flash_attn_varlen_func).

The kernel entry points run hand-written HIP kernels for gfx950 (MFMA,
LDS-staged tiles) through the C ABI in libsigattn.so, registered as
torch.library custom ops `myops::sigmoid_attention_fwd/bwd`,
`myops::sigmoid_attn_padded_fwd/bwd` and `myops::sigmoid_attn_varlen_fwd/bwd`.
Importing works anywhere (so graphs can be traced on the CPU); calling the
kernels needs a gfx950 GPU and raises RuntimeError otherwise.  There is no
CPU or eager fallback.
"""

__version__ = "0.1.2"

from .sigmoid_dense import sigmoid_attention
from .sigmoid_padded import sigmoid_attention_padded
from .sigmoid_reference import sigmoid_attention_ref
from .sigmoid_varlen import sigmoid_attention_varlen

__all__ = [
    "sigmoid_attention",
    "sigmoid_attention_padded",
    "sigmoid_attention_ref",
    "sigmoid_attention_varlen",
]
