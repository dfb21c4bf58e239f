// Portable kernels for the cases the MFMA kernels do not take: fp32 inputs,
// head dims 16 and 32, and rows that are not 16-byte aligned.  One thread owns
// one query row (forward, dQ) or one key row (dK/dV) and walks the other
// sequence through LDS tiles with fp32 FMAs.  Same semantics as the MFMA
// kernels and the reference kernels (sigmoid_triton_dense.py:23-467,
// sigmoid_triton_padded.py:24-509): P and dS are rounded to the I/O dtype
// before their second product, accumulation is fp32, masks are causal
// (key <= query, top-left) and seq_lens bounds, padded rows are written as 0.
#include "common.h"
#include "launch.h"

namespace sigattn {

template <typename T> __device__ __forceinline__ float ld(const void *base, int64_t i) {
  if constexpr (sizeof(T) == 4) return ((const float *)base)[i];
  else return Elem<T>::to_f32(((const uint16_t *)base)[i]);
}
template <typename T> __device__ __forceinline__ void st(void *base, int64_t i, float x) {
  if constexpr (sizeof(T) == 4) ((float *)base)[i] = x;
  else ((uint16_t *)base)[i] = Elem<T>::from_f32(x);
}

__device__ __forceinline__ float sigmoid_of(float s, float scale, float c) {
  // s*scale + c, then 1 / (1 + 2^(-x*log2 e))
  const float x = __builtin_fmaf(s, scale, c);
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(-x * kLog2e));
}

constexpr int GB = 64;  // rows per block (one per thread)
constexpr int GT = 32;  // tile length along the walked sequence

template <typename T, int D, bool CAUSAL>
__global__ __launch_bounds__(GB) void fwd_generic_kernel(const KParams p) {
  __shared__ float sK[GT][D + 1];
  __shared__ float sV[GT][D + 1];
  __shared__ float sC[GT];
  const int BH = p.B * p.H;
  const int bh = blockIdx.x % BH, qb = blockIdx.x / BH;
  const int b = bh / p.H, h = bh % p.H;
  const int Lq = p.len_q(b), Lk = p.len_k(b);
  const int q = qb * GB + threadIdx.x;
  const int64_t qbase = p.q_base(b, h);
  const int64_t kbase = p.k_base(b, h);
  const float scale = *p.scale, bias = p.bias[b];

  float qv[D], acc[D];
  const bool qok = q < Lq;
#pragma unroll
  for (int d = 0; d < D; ++d) {
    qv[d] = qok ? ld<T>(p.q, qbase + (int64_t)q * p.sq_t + d) : 0.0f;
    acc[d] = 0.0f;
  }
  int nend = Lk;
  if (CAUSAL) nend = min(nend, min(qb * GB + GB, Lq));
  if (qb * GB >= Lq) nend = 0;
  for (int n0 = 0; n0 < nend; n0 += GT) {
    for (int e = threadIdx.x; e < GT * D; e += GB) {
      const int r = e / D, d = e % D, key = n0 + r;
      const bool ok = key < Lk;
      sK[r][d] = ok ? ld<T>(p.k, kbase + (int64_t)key * p.sk_t + d) : 0.0f;
      sV[r][d] = ok ? ld<T>(p.v, kbase + (int64_t)key * p.sk_t + d) : 0.0f;
    }
    if (threadIdx.x < GT) {
      const int key = n0 + threadIdx.x;
      sC[threadIdx.x] = (p.score_mod && key < Lk) ? p.score_mod[p.mod_base(b) + key] : 0.0f;
    }
    __syncthreads();
    const int jn = min(GT, nend - n0);
    for (int j = 0; j < jn; ++j) {
      const int key = n0 + j;
      float s = 0.0f;
#pragma unroll
      for (int d = 0; d < D; ++d) s = __builtin_fmaf(qv[d], sK[j][d], s);
      float pr = sigmoid_of(s, scale, bias + sC[j]);
      if (CAUSAL && key > q) pr = 0.0f;
      pr = round_to<T>(pr);
#pragma unroll
      for (int d = 0; d < D; ++d) acc[d] = __builtin_fmaf(pr, sV[j][d], acc[d]);
    }
    __syncthreads();
  }
  if (q < p.q_rows_out(Lq)) {
#pragma unroll
    for (int d = 0; d < D; ++d) st<T>(p.out, qbase + (int64_t)q * p.sq_t + d, qok ? acc[d] : 0.0f);
  }
}

template <typename T, int D, bool CAUSAL>
__global__ __launch_bounds__(GB) void dq_generic_kernel(const KParams p) {
  __shared__ float sK[GT][D + 1];
  __shared__ float sV[GT][D + 1];
  __shared__ float sC[GT];
  const int BH = p.B * p.H;
  const int bh = blockIdx.x % BH, qb = blockIdx.x / BH;
  const int b = bh / p.H, h = bh % p.H;
  const int Lq = p.len_q(b), Lk = p.len_k(b);
  const int q = qb * GB + threadIdx.x;
  const int64_t qbase = p.q_base(b, h);
  const int64_t kbase = p.k_base(b, h);
  const float scale = *p.scale, bias = p.bias[b];

  float qv[D], dov[D], acc[D];
  const bool qok = q < Lq;
#pragma unroll
  for (int d = 0; d < D; ++d) {
    qv[d] = qok ? ld<T>(p.q, qbase + (int64_t)q * p.sq_t + d) : 0.0f;
    dov[d] = qok ? ld<T>(p.dout, qbase + (int64_t)q * p.sq_t + d) : 0.0f;
    acc[d] = 0.0f;
  }
  int nend = Lk;
  if (CAUSAL) nend = min(nend, min(qb * GB + GB, Lq));
  if (qb * GB >= Lq) nend = 0;
  for (int n0 = 0; n0 < nend; n0 += GT) {
    for (int e = threadIdx.x; e < GT * D; e += GB) {
      const int r = e / D, d = e % D, key = n0 + r;
      const bool ok = key < Lk;
      sK[r][d] = ok ? ld<T>(p.k, kbase + (int64_t)key * p.sk_t + d) : 0.0f;
      sV[r][d] = ok ? ld<T>(p.v, kbase + (int64_t)key * p.sk_t + d) : 0.0f;
    }
    if (threadIdx.x < GT) {
      const int key = n0 + threadIdx.x;
      sC[threadIdx.x] = (p.score_mod && key < Lk) ? p.score_mod[p.mod_base(b) + key] : 0.0f;
    }
    __syncthreads();
    const int jn = min(GT, nend - n0);
    for (int j = 0; j < jn; ++j) {
      const int key = n0 + j;
      float s = 0.0f, dp = 0.0f;
#pragma unroll
      for (int d = 0; d < D; ++d) {
        s = __builtin_fmaf(qv[d], sK[j][d], s);
        dp = __builtin_fmaf(dov[d], sV[j][d], dp);
      }
      const float pr = sigmoid_of(s, scale, bias + sC[j]);
      const float t = pr * dp;
      float ds = __builtin_fmaf(-pr, t, t);
      if (CAUSAL && key > q) ds = 0.0f;
      ds = round_to<T>(ds);
#pragma unroll
      for (int d = 0; d < D; ++d) acc[d] = __builtin_fmaf(ds, sK[j][d], acc[d]);
    }
    __syncthreads();
  }
  if (q < p.q_rows_out(Lq)) {
#pragma unroll
    for (int d = 0; d < D; ++d)
      st<T>(p.dq, qbase + (int64_t)q * p.sq_t + d, qok ? acc[d] * scale : 0.0f);
  }
}

template <typename T, int D, bool CAUSAL>
__global__ __launch_bounds__(GB) void dkdv_generic_kernel(const KParams p) {
  __shared__ float sQ[GT][D + 1];
  __shared__ float sO[GT][D + 1];
  const int BH = p.B * p.H;
  const int bh = blockIdx.x % BH, kb = blockIdx.x / BH;
  const int b = bh / p.H, h = bh % p.H;
  const int Lq = p.len_q(b), Lk = p.len_k(b);
  const int key = kb * GB + threadIdx.x;
  const int64_t qbase = p.q_base(b, h);
  const int64_t kbase = p.k_base(b, h);
  const float scale = *p.scale, bias = p.bias[b];
  const bool kok = key < Lk;
  const float c = bias + ((p.score_mod && kok) ? p.score_mod[p.mod_base(b) + key] : 0.0f);

  float kv[D], vv[D], dk[D], dv[D];
#pragma unroll
  for (int d = 0; d < D; ++d) {
    kv[d] = kok ? ld<T>(p.k, kbase + (int64_t)key * p.sk_t + d) : 0.0f;
    vv[d] = kok ? ld<T>(p.v, kbase + (int64_t)key * p.sk_t + d) : 0.0f;
    dk[d] = 0.0f;
    dv[d] = 0.0f;
  }
  const int mstart = CAUSAL ? (kb * GB) / GT * GT : 0;
  const int mend = (kb * GB >= Lk) ? 0 : Lq;
  for (int m0 = mstart; m0 < mend; m0 += GT) {
    for (int e = threadIdx.x; e < GT * D; e += GB) {
      const int r = e / D, d = e % D, q = m0 + r;
      const bool ok = q < Lq;
      sQ[r][d] = ok ? ld<T>(p.q, qbase + (int64_t)q * p.sq_t + d) : 0.0f;
      sO[r][d] = ok ? ld<T>(p.dout, qbase + (int64_t)q * p.sq_t + d) : 0.0f;
    }
    __syncthreads();
    const int jn = min(GT, mend - m0);
    for (int j = 0; j < jn; ++j) {
      const int q = m0 + j;
      float s = 0.0f, dp = 0.0f;
#pragma unroll
      for (int d = 0; d < D; ++d) {
        s = __builtin_fmaf(sQ[j][d], kv[d], s);
        dp = __builtin_fmaf(sO[j][d], vv[d], dp);
      }
      float pr = sigmoid_of(s, scale, c);
      const float t = pr * dp;
      float ds = __builtin_fmaf(-pr, t, t);
      if (CAUSAL && key > q) { pr = 0.0f; ds = 0.0f; }
      pr = round_to<T>(pr);
      ds = round_to<T>(ds);
#pragma unroll
      for (int d = 0; d < D; ++d) {
        dv[d] = __builtin_fmaf(pr, sO[j][d], dv[d]);
        dk[d] = __builtin_fmaf(ds, sQ[j][d], dk[d]);
      }
    }
    __syncthreads();
  }
  if (key < p.k_rows_out(Lk)) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      st<T>(p.dk, kbase + (int64_t)key * p.sk_t + d, kok ? dk[d] * scale : 0.0f);
      st<T>(p.dv, kbase + (int64_t)key * p.sk_t + d, kok ? dv[d] : 0.0f);
    }
  }
}

// ---- launchers ---------------------------------------------------------------

#define SIGATTN_GENERIC_LAUNCHER(NAME, KERNEL, ROWS)                                   \
  template <typename T, int D>                                                         \
  static void NAME##_t(const KParams &kp, bool causal, hipStream_t s) {                \
    KParams p = kp;                                                                    \
    p.nblk = ((ROWS) + GB - 1) / GB;                                                   \
    const dim3 grid((unsigned)(p.nblk * p.B * p.H));                                   \
    if (causal) KERNEL<T, D, true><<<grid, dim3(GB), 0, s>>>(p);                       \
    else KERNEL<T, D, false><<<grid, dim3(GB), 0, s>>>(p);                             \
  }                                                                                    \
  template <typename T>                                                                \
  static void NAME##_d(const KParams &p, int D, bool causal, hipStream_t s) {          \
    switch (D) {                                                                       \
      case 16: NAME##_t<T, 16>(p, causal, s); break;                                   \
      case 32: NAME##_t<T, 32>(p, causal, s); break;                                   \
      case 64: NAME##_t<T, 64>(p, causal, s); break;                                   \
      default: NAME##_t<T, 128>(p, causal, s); break;                                  \
    }                                                                                  \
  }                                                                                    \
  void NAME(const KParams &p, int dtype, int D, bool causal, hipStream_t s) {          \
    if (dtype == kF32) NAME##_d<float>(p, D, causal, s);                               \
    else if (dtype == kBF16) NAME##_d<__bf16>(p, D, causal, s);                        \
    else NAME##_d<_Float16>(p, D, causal, s);                                          \
  }

SIGATTN_GENERIC_LAUNCHER(launch_fwd_generic, fwd_generic_kernel, p.Tq)
SIGATTN_GENERIC_LAUNCHER(launch_bwd_dq_generic, dq_generic_kernel, p.Tq)
SIGATTN_GENERIC_LAUNCHER(launch_bwd_dkdv_generic, dkdv_generic_kernel, p.Tk)

#undef SIGATTN_GENERIC_LAUNCHER

// Rows of packed outputs that no sequence covers, for two axes in one launch
// (zero_gap_rows; the first nblk0 workgroups take ax0).
template <int ESIZE>
__global__ __launch_bounds__(256) void zero_gaps_kernel(const GapAxis ax0, const GapAxis ax1, int nblk0) {
  __shared__ unsigned long long lds[2];
  const bool second = (int)blockIdx.x >= nblk0;
  zero_gap_rows<ESIZE>(second ? ax1 : ax0, second ? (int)blockIdx.x - nblk0 : (int)blockIdx.x, lds);
}

void launch_zero_gaps(const GapAxis &a, const GapAxis &b, int esize, hipStream_t st) {
  const int64_t na = a.rows > 0 ? (a.rows + 63) / 64 : 0, nb = b.rows > 0 ? (b.rows + 63) / 64 : 0;
  if (na + nb == 0) return;
  const dim3 grid((unsigned)(na + nb));
  if (esize == 4) zero_gaps_kernel<4><<<grid, dim3(256), 0, st>>>(a, b, (int)na);
  else zero_gaps_kernel<2><<<grid, dim3(256), 0, st>>>(a, b, (int)na);
}

}  // namespace sigattn
