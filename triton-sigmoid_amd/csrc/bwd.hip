// Recompute backward on gfx950 MFMA: dQ kernel (query-stationary) and dK/dV
// kernel (key-stationary).  No atomics: every output element is owned by one
// lane, so results are bitwise deterministic.
//
// Semantics follow the reference's _bwd_dense_dq_kernel / _bwd_dense_dkdv_kernel
// (src/triton_sigmoid/sigmoid_triton_dense.py:162-307, :315-467) and the padded
// variants (src/triton_sigmoid/sigmoid_triton_padded.py:179-339, :342-509):
//   P = sigmoid(S*scale + bias (+ score_mod[key])) recomputed in fp32;
//   dP = dO·Vᵀ; dS = P(1-P)dP computed as fma(P, -P*dP, P*dP); masked dS = 0;
//   dQ = (dS rounded to the I/O dtype)·K · scale;
//   dV = (P rounded)ᵀ·dO;  dK = (dS rounded)ᵀ·Q · scale.
// Padded query rows get dQ = 0 and padded key rows dK = dV = 0; zero-filled
// rows past seq_lens contribute exactly 0, so only causal needs an element mask.
#include "common.h"
#include "launch.h"

namespace sigattn {

// ---------------------------------------------------------------------------
// dQ: workgroup = 4 waves x 32 queries; walks 64-key tiles of K and V staged
// row-major in LDS (Kᵀ operands come from ds_read_b64_tr_b16).
//   Sᵀ = K·Qᵀ, dPᵀ = V·dOᵀ (accumulators: lane = query column),
//   dQᵀ += Kᵀ·dSᵀ with dSᵀ taken from the accumulator registers.
// ---------------------------------------------------------------------------
template <typename T, int D, bool CAUSAL, bool SCOREMOD>
__global__ __launch_bounds__(256, 2) void bwd_dq_kernel(const KParams p) {
  constexpr int BM = 128, BN = 64;
  constexpr int NKS = D / 16, NDB = D / 32;

  __shared__ __attribute__((aligned(16))) uint16_t sK[BN * D];  // swizzled tiles
  __shared__ __attribute__((aligned(16))) uint16_t sV[BN * D];
  __shared__ __attribute__((aligned(16))) float sC[SCOREMOD ? BN : 4];

  const int BH = p.B * p.H;
  const int bh = blockIdx.x % BH;
  int qb = blockIdx.x / BH;
  if (CAUSAL) qb = p.nblk - 1 - qb;
  const int b = bh / p.H, h = bh % p.H;
  const int Lq = clamp_len(p.seq_q, b, p.Tq);
  const int Lk = clamp_len(p.seq_k, b, p.Tk);

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int l32 = lane & 31, hi = lane >> 5;
  const int q0 = qb * BM, qw = q0 + w * 32, my_q = qw + l32;

  const int64_t qoff = (int64_t)b * p.sq_b + (int64_t)h * p.sq_h;
  const int64_t koff = (int64_t)b * p.sk_b + (int64_t)h * p.sk_h;
  const uint16_t *Qb = (const uint16_t *)p.q + qoff;
  const uint16_t *dOb = (const uint16_t *)p.dout + qoff;
  const uint16_t *Kb = (const uint16_t *)p.k + koff;
  const uint16_t *Vb = (const uint16_t *)p.v + koff;
  uint16_t *dQb = (uint16_t *)p.dq + qoff;

  int nend = Lk;
  if (CAUSAL) nend = min(nend, min(q0 + BM, Lq));
  if (q0 >= Lq) nend = 0;
  const int ntiles = (nend + BN - 1) / BN;

  const float scale = *p.scale;
  const float bias = p.bias[b];
  const float nsl = -scale * kLog2e, nbl = -bias * kLog2e;

  u32x4 qf[NKS], of[NKS];
  {
    const bool ok = my_q < Lq;
    const uint16_t *qr = Qb + (int64_t)my_q * p.sq_t + 8 * hi;
    const uint16_t *orow = dOb + (int64_t)my_q * p.sq_t + 8 * hi;
#pragma unroll
    for (int s = 0; s < NKS; ++s) {
      qf[s] = ok ? *(const u32x4 *)(qr + 16 * s) : zero4();
      of[s] = ok ? *(const u32x4 *)(orow + 16 * s) : zero4();
    }
  }
  f32x16 acc[NDB];
#pragma unroll
  for (int d = 0; d < NDB; ++d) acc[d] = zero16();

  TileStager<BN, D> kst, vst;
  float creg = 0.0f;
  auto gload = [&](int n0) {
    kst.load(Kb, p.sk_t, n0, Lk, tid);
    vst.load(Vb, p.sk_t, n0, Lk, tid);
    if (SCOREMOD && tid < BN) {
      const int key = n0 + tid;
      creg = key < Lk ? -(bias + p.score_mod[(int64_t)b * p.Tk + key]) * kLog2e : 0.0f;
    }
  };

  if (ntiles > 0) gload(0);
  for (int it = 0; it < ntiles; ++it) {
    const int n0 = it * BN;
    __syncthreads();  // previous tile fully consumed
    kst.store(sK, tid);
    vst.store(sV, tid);
    if (SCOREMOD && tid < BN) sC[tid] = creg;
    __syncthreads();
    if (it + 1 < ntiles) gload(n0 + BN);

    if (!CAUSAL || n0 <= qw + 31) {
      uint32_t dsk[BN / 4];
#pragma unroll
      for (int kb = 0; kb < BN / 32; ++kb) {
        const int kbase = n0 + kb * 32;
        if (CAUSAL && kbase > qw + 31) {
#pragma unroll
          for (int i = 0; i < 8; ++i) dsk[kb * 8 + i] = 0u;
          continue;
        }
        f32x16 s = zero16(), dp = zero16();
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
          s = Elem<T>::mfma(read_row_operand<D>(sK, kb * 32 + l32, ks, hi), qf[ks], s);
          dp = Elem<T>::mfma(read_row_operand<D>(sV, kb * 32 + l32, ks, hi), of[ks], dp);
        }
        float c[16];
        if constexpr (SCOREMOD) {
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const float4 cv = *(const float4 *)&sC[kb * 32 + 8 * g + 4 * hi];
            c[4 * g + 0] = cv.x; c[4 * g + 1] = cv.y; c[4 * g + 2] = cv.z; c[4 * g + 3] = cv.w;
          }
        } else {
#pragma unroll
          for (int i = 0; i < 16; ++i) c[i] = nbl;
        }
        float ds[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float pr = sigmoid_from_neg_log2(__builtin_fmaf(s[i], nsl, c[i]));
          const float t = pr * dp[i];
          ds[i] = __builtin_fmaf(-pr, t, t);
        }
        if (CAUSAL && kbase + 31 > qw) {
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int key = kbase + 8 * (i / 4) + 4 * hi + (i % 4);
            if (key > my_q) ds[i] = 0.0f;
          }
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) dsk[kb * 8 + i] = Elem<T>::pack(ds[2 * i], ds[2 * i + 1]);
      }
      // dQᵀ[d, q] += Kᵀ[d, key] · dSᵀ[key, q]
#pragma unroll
      for (int ks = 0; ks < BN / 16; ++ks) {
        if (CAUSAL && n0 + ks * 16 > qw + 31) break;
        const u32x4 bop = (u32x4){dsk[4 * ks], dsk[4 * ks + 1], dsk[4 * ks + 2], dsk[4 * ks + 3]};
#pragma unroll
        for (int db = 0; db < NDB; ++db)
          acc[db] = Elem<T>::mfma(read_tr16_swz<D>(sK, db * 32, ks, lane), bop, acc[db]);
      }
    }
  }

  if (my_q < p.Tq) {
    uint16_t *row = dQb + (int64_t)my_q * p.sq_t;
    const bool valid = my_q < Lq;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d0 = db * 32 + 8 * g + 4 * hi;
        u32x2 o;
        o.x = valid ? Elem<T>::pack(acc[db][4 * g] * scale, acc[db][4 * g + 1] * scale) : 0u;
        o.y = valid ? Elem<T>::pack(acc[db][4 * g + 2] * scale, acc[db][4 * g + 3] * scale) : 0u;
        *(u32x2 *)(row + d0) = o;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// dK/dV: workgroup = 4 waves x 32 keys; walks 64-query tiles of Q and dO
// staged row-major in LDS (Qᵀ, dOᵀ operands come from ds_read_b64_tr_b16).
//   S = Q·Kᵀ, dP = dO·Vᵀ (accumulators: lane = key column),
//   dVᵀ += dOᵀ·P and dKᵀ += Qᵀ·dS with P, dS taken from the accumulators.
// ---------------------------------------------------------------------------
template <typename T, int D, bool CAUSAL, bool SCOREMOD>
__global__ __launch_bounds__(256, (D == 64 ? 2 : 1)) void bwd_dkdv_kernel(const KParams p) {
  constexpr int BN = 128, BMQ = 64;
  constexpr int NKS = D / 16, NDB = D / 32;

  __shared__ __attribute__((aligned(16))) uint16_t sQ[BMQ * D];  // swizzled tiles
  __shared__ __attribute__((aligned(16))) uint16_t sO[BMQ * D];

  const int BH = p.B * p.H;
  const int bh = blockIdx.x % BH;
  const int kblk = blockIdx.x / BH;  // causal: low key blocks carry the most work and come first
  const int b = bh / p.H, h = bh % p.H;
  const int Lq = clamp_len(p.seq_q, b, p.Tq);
  const int Lk = clamp_len(p.seq_k, b, p.Tk);

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int l32 = lane & 31, hi = lane >> 5;
  const int k0 = kblk * BN, kw = k0 + w * 32, my_k = kw + l32;

  const int64_t qoff = (int64_t)b * p.sq_b + (int64_t)h * p.sq_h;
  const int64_t koff = (int64_t)b * p.sk_b + (int64_t)h * p.sk_h;
  const uint16_t *Qb = (const uint16_t *)p.q + qoff;
  const uint16_t *dOb = (const uint16_t *)p.dout + qoff;
  const uint16_t *Kb = (const uint16_t *)p.k + koff;
  const uint16_t *Vb = (const uint16_t *)p.v + koff;
  uint16_t *dKb = (uint16_t *)p.dk + koff;
  uint16_t *dVb = (uint16_t *)p.dv + koff;

  const int mstart = CAUSAL ? (k0 / BMQ) * BMQ : 0;
  const int mend = (k0 >= Lk) ? mstart : Lq;
  const int ntiles = mend > mstart ? (mend - mstart + BMQ - 1) / BMQ : 0;

  const float scale = *p.scale;
  const float bias = p.bias[b];
  const float nsl = -scale * kLog2e;
  const bool kok = my_k < Lk;
  float nc = -bias * kLog2e;
  if (SCOREMOD) nc = kok ? -(bias + p.score_mod[(int64_t)b * p.Tk + my_k]) * kLog2e : 0.0f;

  u32x4 kf[NKS], vf[NKS];
  {
    const uint16_t *kr = Kb + (int64_t)my_k * p.sk_t + 8 * hi;
    const uint16_t *vr = Vb + (int64_t)my_k * p.sk_t + 8 * hi;
#pragma unroll
    for (int s = 0; s < NKS; ++s) {
      kf[s] = kok ? *(const u32x4 *)(kr + 16 * s) : zero4();
      vf[s] = kok ? *(const u32x4 *)(vr + 16 * s) : zero4();
    }
  }
  f32x16 dka[NDB], dva[NDB];
#pragma unroll
  for (int d = 0; d < NDB; ++d) { dka[d] = zero16(); dva[d] = zero16(); }

  TileStager<BMQ, D> qst, ost;
  if (ntiles > 0) {
    qst.load(Qb, p.sq_t, mstart, Lq, tid);
    ost.load(dOb, p.sq_t, mstart, Lq, tid);
  }
  for (int it = 0; it < ntiles; ++it) {
    const int m0 = mstart + it * BMQ;
    __syncthreads();
    qst.store(sQ, tid);
    ost.store(sO, tid);
    __syncthreads();
    if (it + 1 < ntiles) {
      qst.load(Qb, p.sq_t, m0 + BMQ, Lq, tid);
      ost.load(dOb, p.sq_t, m0 + BMQ, Lq, tid);
    }

    if (!CAUSAL || m0 + BMQ - 1 >= kw) {
      uint32_t pk[BMQ / 4], dsk[BMQ / 4];
#pragma unroll
      for (int qbk = 0; qbk < BMQ / 32; ++qbk) {
        const int qbase = m0 + qbk * 32;
        if (CAUSAL && qbase + 31 < kw) {
#pragma unroll
          for (int i = 0; i < 8; ++i) { pk[qbk * 8 + i] = 0u; dsk[qbk * 8 + i] = 0u; }
          continue;
        }
        f32x16 s = zero16(), dp = zero16();
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks) {
          s = Elem<T>::mfma(read_row_operand<D>(sQ, qbk * 32 + l32, ks, hi), kf[ks], s);
          dp = Elem<T>::mfma(read_row_operand<D>(sO, qbk * 32 + l32, ks, hi), vf[ks], dp);
        }
        float pv[16], ds[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          pv[i] = sigmoid_from_neg_log2(__builtin_fmaf(s[i], nsl, nc));
          const float t = pv[i] * dp[i];
          ds[i] = __builtin_fmaf(-pv[i], t, t);
        }
        if (CAUSAL && qbase < kw + 31) {
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int q = qbase + 8 * (i / 4) + 4 * hi + (i % 4);
            if (q < my_k) { pv[i] = 0.0f; ds[i] = 0.0f; }
          }
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          pk[qbk * 8 + i] = Elem<T>::pack(pv[2 * i], pv[2 * i + 1]);
          dsk[qbk * 8 + i] = Elem<T>::pack(ds[2 * i], ds[2 * i + 1]);
        }
      }
      // dVᵀ[d, key] += dOᵀ[d, q] · P[q, key];  dKᵀ[d, key] += Qᵀ[d, q] · dS[q, key]
#pragma unroll
      for (int ks = 0; ks < BMQ / 16; ++ks) {
        if (CAUSAL && m0 + ks * 16 + 15 < kw) continue;
        const u32x4 pb = (u32x4){pk[4 * ks], pk[4 * ks + 1], pk[4 * ks + 2], pk[4 * ks + 3]};
        const u32x4 db_ = (u32x4){dsk[4 * ks], dsk[4 * ks + 1], dsk[4 * ks + 2], dsk[4 * ks + 3]};
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
          dva[db] = Elem<T>::mfma(read_tr16_swz<D>(sO, db * 32, ks, lane), pb, dva[db]);
          dka[db] = Elem<T>::mfma(read_tr16_swz<D>(sQ, db * 32, ks, lane), db_, dka[db]);
        }
      }
    }
  }

  if (my_k < p.Tk) {
    uint16_t *kr = dKb + (int64_t)my_k * p.sk_t;
    uint16_t *vr = dVb + (int64_t)my_k * p.sk_t;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d0 = db * 32 + 8 * g + 4 * hi;
        u32x2 ok_, ov;
        ok_.x = kok ? Elem<T>::pack(dka[db][4 * g] * scale, dka[db][4 * g + 1] * scale) : 0u;
        ok_.y = kok ? Elem<T>::pack(dka[db][4 * g + 2] * scale, dka[db][4 * g + 3] * scale) : 0u;
        ov.x = kok ? Elem<T>::pack(dva[db][4 * g], dva[db][4 * g + 1]) : 0u;
        ov.y = kok ? Elem<T>::pack(dva[db][4 * g + 2], dva[db][4 * g + 3]) : 0u;
        *(u32x2 *)(kr + d0) = ok_;
        *(u32x2 *)(vr + d0) = ov;
      }
    }
  }
}

#define SIGATTN_BWD_LAUNCHER(NAME, KERNEL, ROWBLK, ROWS)                                    \
  template <typename T, int D>                                                              \
  static void NAME##_t(const KParams &kp, bool causal, bool sm, hipStream_t st) {           \
    KParams p = kp;                                                                         \
    p.nblk = ((ROWS) + (ROWBLK) - 1) / (ROWBLK);                                            \
    const dim3 grid((unsigned)(p.nblk * p.B * p.H)), block(256);                            \
    if (causal) {                                                                           \
      if (sm) KERNEL<T, D, true, true><<<grid, block, 0, st>>>(p);                          \
      else KERNEL<T, D, true, false><<<grid, block, 0, st>>>(p);                            \
    } else {                                                                                \
      if (sm) KERNEL<T, D, false, true><<<grid, block, 0, st>>>(p);                         \
      else KERNEL<T, D, false, false><<<grid, block, 0, st>>>(p);                           \
    }                                                                                       \
  }                                                                                         \
  void NAME(const KParams &p, int dtype, int D, bool causal, bool sm, hipStream_t st) {     \
    if (dtype == kBF16) {                                                                   \
      if (D == 128) NAME##_t<__bf16, 128>(p, causal, sm, st);                               \
      else NAME##_t<__bf16, 64>(p, causal, sm, st);                                         \
    } else {                                                                                \
      if (D == 128) NAME##_t<_Float16, 128>(p, causal, sm, st);                             \
      else NAME##_t<_Float16, 64>(p, causal, sm, st);                                       \
    }                                                                                       \
  }

SIGATTN_BWD_LAUNCHER(launch_bwd_dq_mfma, bwd_dq_kernel, 128, p.Tq)
SIGATTN_BWD_LAUNCHER(launch_bwd_dkdv_mfma, bwd_dkdv_kernel, 128, p.Tk)

#undef SIGATTN_BWD_LAUNCHER

}  // namespace sigattn
