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
// Padded query rows get dQ = 0 and padded key rows dK = dV = 0.
//
// Both kernels stream their tiles (K, V for dQ; Q, dO for dK/dV) into
// double-buffered swizzled LDS with direct global->LDS DMA one tile ahead,
// and keep the stationary rows as MFMA operands in registers.  The dK/dV
// kernel (one wave per SIMD, accumulators in AGPRs) runs each tile as
// scheduling regions that overlap the P / dS VALU work of one 32-query block
// with the MFMA chains of the next; the dQ kernel (two waves per SIMD) relies
// on the second wave for that overlap.  Rows past seq_lens are fetched as
// copies of the last valid row (in bounds) and masked on boundary tiles.
#include <type_traits>

#include "common.h"
#include "launch.h"

namespace sigattn {

// ---------------------------------------------------------------------------
// dQ: workgroup = 4 waves x 32 queries; walks 64-key tiles of K and V.
//   Sᵀ = K·Qᵀ, dPᵀ = V·dOᵀ (accumulators: lane = query column),
//   dQᵀ += Kᵀ·dSᵀ with dSᵀ taken from the accumulator registers and Kᵀ read
//   from the K tile with ds_read_b64_tr_b16.
// ---------------------------------------------------------------------------
template <typename T, int D, bool CAUSAL, bool SCOREMOD>
__global__ __launch_bounds__(256, 2) void bwd_dq_kernel(const KParams p) {
  constexpr int BM = 128, BN = 64;
  constexpr int NKS = D / 16, NDB = D / 32;

  __shared__ __attribute__((aligned(16))) uint16_t sK[2][BN * D];
  __shared__ __attribute__((aligned(16))) uint16_t sV[2][BN * D];
  __shared__ __attribute__((aligned(16))) float sC[SCOREMOD ? 2 * BN : 4];

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

  TileOffsets<D> to;
  to.init(lane);
  DmaPlan<BN, D, 4> dma;
  dma.init(w, lane);
  const int kv_stride_bytes = (int)(p.sk_t * 2);

  // dS of one 32-key block into eight packed words.
  auto ds_block = [&](const f32x16 &s, const f32x16 &dp, int st, int kl, int kbase, uint32_t *out,
                      bool mask) SIGATTN_INLINE {
    float c[16];
    if constexpr (SCOREMOD) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const float4 cv = *(const float4 *)&sC[st * BN + kl + 8 * g + 4 * hi];
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
    if (mask) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int key = kbase + 8 * (i / 4) + 4 * hi + (i % 4);
        if (key >= Lk || (CAUSAL && key > my_q)) ds[i] = 0.0f;
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) out[i] = Elem<T>::pack(ds[2 * i], ds[2 * i + 1]);
  };

  // dQᵀ[d, q] += Kᵀ[d, key] · dSᵀ[key, q] for the two 16-key steps of block kbi.
  auto dq_block = [&](int st, int kbi, const uint32_t *dsk) SIGATTN_INLINE {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const u32x4 bop = (u32x4){dsk[4 * j], dsk[4 * j + 1], dsk[4 * j + 2], dsk[4 * j + 3]};
#pragma unroll
      for (int db = 0; db < NDB; ++db)
        acc[db] = Elem<T>::mfma(ld_tr<D>(sK[st], to, 2 * kbi + j, db), bop, acc[db]);
    }
  };

  // Per 32-key block: Sᵀ/dPᵀ chains (16 MFMA), dS (VALU), dQ (8 MFMA).  The
  // blocks run one after the other (four 32x32 fp32 accumulators plus the Q
  // and dO operands would not fit next to the dQ accumulators); the second
  // wave on each SIMD supplies the MFMA/VALU overlap.
  auto tile_step = [&](int st, int n0, bool mask) SIGATTN_INLINE {
#pragma unroll
    for (int kbi = 0; kbi < 2; ++kbi) {
      f32x16 s = zero16(), dp = zero16();
      uint32_t dk[8];
#pragma unroll
      for (int ks = 0; ks < NKS; ++ks) {
        s = Elem<T>::mfma(ld_row<D>(sK[st], to, 32 * kbi, ks), qf[ks], s);
        dp = Elem<T>::mfma(ld_row<D>(sV[st], to, 32 * kbi, ks), of[ks], dp);
      }
      ds_block(s, dp, st, 32 * kbi, n0 + 32 * kbi, dk, mask);
      dq_block(st, kbi, dk);
    }
  };

  float creg = 0.0f;
  auto load_c = [&](int n0) SIGATTN_INLINE {
    if (SCOREMOD && tid < BN) {
      const int key = n0 + tid;
      creg = key < Lk ? -(bias + p.score_mod[(int64_t)b * p.Tk + key]) * kLog2e : 0.0f;
    }
  };
  auto issue = [&](int st, int n0) SIGATTN_INLINE {
    dma.issue(sK[st], Kb, kv_stride_bytes, n0, Lk);
    dma.issue(sV[st], Vb, kv_stride_bytes, n0, Lk);
  };
  auto iteration = [&](int it, auto stage_tag) SIGATTN_INLINE {
    constexpr int ST = decltype(stage_tag)::value;
    const int n0 = it * BN;
    wait_dma();
    if (SCOREMOD && tid < BN) sC[ST * BN + tid] = creg;
    __syncthreads();
    if (it + 1 < ntiles) {
      load_c(n0 + BN);
      issue(ST ^ 1, n0 + BN);
    }
    if (!CAUSAL || n0 <= qw + 31) {
      tile_step(ST, n0, (n0 + BN > Lk) || (CAUSAL && n0 + BN - 1 > qw));
    }
  };

  if (ntiles > 0) {
    load_c(0);
    issue(0, 0);
  }
  for (int it = 0; it < ntiles; it += 2) {
    iteration(it, std::integral_constant<int, 0>{});
    if (it + 1 < ntiles) iteration(it + 1, std::integral_constant<int, 1>{});
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
        o.x = Elem<T>::pack(acc[db][4 * g] * scale, acc[db][4 * g + 1] * scale);
        o.y = Elem<T>::pack(acc[db][4 * g + 2] * scale, acc[db][4 * g + 3] * scale);
        if (!valid) o = (u32x2){0u, 0u};
        *(u32x2 *)(row + d0) = o;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// dK/dV: workgroup = 4 waves x 32 keys; walks 64-query tiles of Q and dO,
// two 32-query blocks at a time.
//   S = Q·Kᵀ, dP = dO·Vᵀ (accumulators: lane = key column),
//   dVᵀ += dOᵀ·P and dKᵀ += Qᵀ·dS with P, dS taken from the accumulators and
//   Qᵀ, dOᵀ read from the tiles with ds_read_b64_tr_b16.
// ---------------------------------------------------------------------------
template <typename T, int D, bool CAUSAL, bool SCOREMOD>
__global__ __launch_bounds__(256, (D == 64 ? 2 : 1)) void bwd_dkdv_kernel(const KParams p) {
  constexpr int BN = 128, BMQ = 64;  // keys per workgroup, queries per LDS tile
  constexpr int NKS = D / 16, NDB = D / 32;

  __shared__ __attribute__((aligned(16))) uint16_t sQ[2][BMQ * D];
  __shared__ __attribute__((aligned(16))) uint16_t sO[2][BMQ * D];

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

  TileOffsets<D> to;
  to.init(lane);
  DmaPlan<BMQ, D, 4> dma;
  dma.init(w, lane);
  const int q_stride_bytes = (int)(p.sq_t * 2);

  // P and dS of one 32-query block (rows qbase.., this lane's key).
  auto pds_block = [&](const f32x16 &s, const f32x16 &dp, int qbase, uint32_t *pk, uint32_t *dsk,
                       bool mask) SIGATTN_INLINE {
    float pv[16], ds[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      pv[i] = sigmoid_from_neg_log2(__builtin_fmaf(s[i], nsl, nc));
      const float t = pv[i] * dp[i];
      ds[i] = __builtin_fmaf(-pv[i], t, t);
    }
    if (mask) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int q = qbase + 8 * (i / 4) + 4 * hi + (i % 4);
        if (q >= Lq || (CAUSAL && q < my_k)) { pv[i] = 0.0f; ds[i] = 0.0f; }
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      pk[i] = Elem<T>::pack(pv[2 * i], pv[2 * i + 1]);
      dsk[i] = Elem<T>::pack(ds[2 * i], ds[2 * i + 1]);
    }
  };

  // dVᵀ += dOᵀ·P and dKᵀ += Qᵀ·dS for the two 16-query steps of block qbk.
  auto grad_block = [&](int st, int qbk, const uint32_t *pk, const uint32_t *dsk) SIGATTN_INLINE {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const u32x4 pb = (u32x4){pk[4 * j], pk[4 * j + 1], pk[4 * j + 2], pk[4 * j + 3]};
      const u32x4 sb = (u32x4){dsk[4 * j], dsk[4 * j + 1], dsk[4 * j + 2], dsk[4 * j + 3]};
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
        dva[db] = Elem<T>::mfma(ld_tr<D>(sO[st], to, 2 * qbk + j, db), pb, dva[db]);
        dka[db] = Elem<T>::mfma(ld_tr<D>(sQ[st], to, 2 * qbk + j, db), sb, dka[db]);
      }
    }
  };

  // One pair of 32-query blocks (tile rows qo .. qo+63) in four regions:
  // A S0/dP0 chains; B S1/dP1 chains || P,dS of block 0;
  // C grads of block 0 || P,dS of block 1; D grads of block 1.
  auto pair_step = [&](int st, int m0, int qo, bool mask) SIGATTN_INLINE {
    f32x16 s0 = zero16(), d0 = zero16(), s1 = zero16(), d1 = zero16();
    uint32_t p0[8], g0[8], p1[8], g1[8];
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      s0 = Elem<T>::mfma(ld_row<D>(sQ[st], to, qo, ks), kf[ks], s0);
      d0 = Elem<T>::mfma(ld_row<D>(sO[st], to, qo, ks), vf[ks], d0);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      s1 = Elem<T>::mfma(ld_row<D>(sQ[st], to, qo + 32, ks), kf[ks], s1);
      d1 = Elem<T>::mfma(ld_row<D>(sO[st], to, qo + 32, ks), vf[ks], d1);
    }
    pds_block(s0, d0, m0 + qo, p0, g0, mask);
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
    for (int i = 0; i < 2 * NKS; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 7, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    grad_block(st, qo / 32, p0, g0);
    pds_block(s1, d1, m0 + qo + 32, p1, g1, mask);
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
    for (int i = 0; i < 4 * NDB; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 7, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    grad_block(st, qo / 32 + 1, p1, g1);
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
    for (int i = 0; i < 4 * NDB; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
  };

  // A 128-query tile = two pairs; each pair masks / skips on its own rows.
  auto tile_step = [&](int st, int m0) SIGATTN_INLINE {
#pragma unroll
    for (int qo = 0; qo < BMQ; qo += 64) {
      const int mq = m0 + qo;
      if (CAUSAL && mq + 63 < kw) continue;  // every query of the pair precedes this wave's keys
      pair_step(st, m0, qo, (mq + 64 > Lq) || (CAUSAL && mq < kw + 31));
    }
  };

  auto issue = [&](int st, int m0) SIGATTN_INLINE {
    dma.issue(sQ[st], Qb, q_stride_bytes, m0, Lq);
    dma.issue(sO[st], dOb, q_stride_bytes, m0, Lq);
  };
  auto iteration = [&](int it, auto stage_tag) SIGATTN_INLINE {
    constexpr int ST = decltype(stage_tag)::value;
    const int m0 = mstart + it * BMQ;
    wait_dma();
    __syncthreads();
    if (it + 1 < ntiles) issue(ST ^ 1, m0 + BMQ);
    if (!CAUSAL || m0 + BMQ - 1 >= kw) tile_step(ST, m0);
  };

  if (ntiles > 0) issue(0, mstart);
  for (int it = 0; it < ntiles; it += 2) {
    iteration(it, std::integral_constant<int, 0>{});
    if (it + 1 < ntiles) iteration(it + 1, std::integral_constant<int, 1>{});
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
        ok_.x = Elem<T>::pack(dka[db][4 * g] * scale, dka[db][4 * g + 1] * scale);
        ok_.y = Elem<T>::pack(dka[db][4 * g + 2] * scale, dka[db][4 * g + 3] * scale);
        ov.x = Elem<T>::pack(dva[db][4 * g], dva[db][4 * g + 1]);
        ov.y = Elem<T>::pack(dva[db][4 * g + 2], dva[db][4 * g + 3]);
        if (!kok) { ok_ = (u32x2){0u, 0u}; ov = (u32x2){0u, 0u}; }
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
