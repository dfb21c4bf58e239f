"""TEST INFRASTRUCTURE ONLY — CPU oracle for fused sigmoid attention.

Importable only from tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, as the checker; never from the product (triton_sigmoid).
  sigmoid_oracle — numpy float64 restatement of the reference kernels' forward
                   and recompute backward (with I/O-dtype rounding of P and dS);
  eager          — eager PyTorch restatement of the reference's
                   sigmoid_attention_ref (fp32 and mixed precision).
"""
