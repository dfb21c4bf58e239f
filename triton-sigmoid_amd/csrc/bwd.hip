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
__device__ __forceinline__ void bwd_dq_body(const KParams &p, const int wg) {
  constexpr int BM = 128, BN = 64;
  constexpr int NKS = D / 16, NDB = D / 32;

  __shared__ __attribute__((aligned(16))) uint16_t sK[2][BN * D];
  __shared__ __attribute__((aligned(16))) uint16_t sV[2][BN * D];
  __shared__ __attribute__((aligned(16))) float sC[SCOREMOD ? 2 * BN : 4];

  int b, h, qb;
  int ritem = 0, rchunk = 0;  // range split: the item and this workgroup's chunk of its keys
  if (!CAUSAL && p.rsplit > 1) {
    int bh;
    ritem = wg / p.rsplit, rchunk = wg % p.rsplit;
    dense_item(ritem, p.B * p.H, p.nblk, true, bh, qb);
    b = bh / p.H, h = bh % p.H;
  } else if (p.ragged() && p.B <= 64) {
    const auto lq = [&](int i) SIGATTN_INLINE { return p.len_q(i); };
    const auto lk = [&](int i) SIGATTN_INLINE { return p.len_k(i); };
    const WorkItem it = CAUSAL ? WorkOrder::by_level(wg, p.B, p.H, lq, BM, p.nblk, true, p.ncu,
                                                     D <= 64 ? 3 : 2)
                               : WorkOrder::by_stream(wg, p.B, p.H, lq, BM, p.nblk, lk);
    b = it.b, h = it.h, qb = it.blk;
  } else {
    const int BH = p.B * p.H;
    int bh;
    dense_item(wg, BH, p.nblk, !CAUSAL, bh, qb);
    if (CAUSAL) qb = p.nblk - 1 - qb;  // heaviest query blocks first
    b = bh / p.H, h = bh % p.H;
  }
  const int Lq = p.len_q(b);
  // Keys of this workgroup: under the range split, its chunk of the item's
  // key tiles, indexed from the chunk's first key.
  int key0 = 0, Lk = p.len_k(b);
  if (!CAUSAL && p.rsplit > 1) {
    const int ntk = (Lk + BN - 1) / BN;
    key0 = split_tile(rchunk, p.rsplit, ntk) * BN;
    Lk = min(Lk, split_tile(rchunk + 1, p.rsplit, ntk) * BN) - key0;
  }
  const bool half = p.half_head(D);  // head_dim 16 in this D = 32 kernel
  // Padding item: its zero rows as part of one contiguous span (see zero_row_span).
  if (qb * BM >= Lq && p.q_rows_contiguous(half ? 16 : D)) {
    zero_row_span((uint16_t *)p.dq + (int64_t)b * p.sq_b, p.sq_t, qb * BM, min(qb * BM + BM, p.Tq), h, p.H,
                  threadIdx.x, 256);
    return;
  }

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int l32 = lane & 31, hi = lane >> 5;
  const int q0 = qb * BM, qw = q0 + w * 32, my_q = qw + l32;

  const int64_t qoff = p.q_base(b, h);
  const int64_t koff = p.k_base(b, h) + (int64_t)key0 * p.sk_t;
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
      const bool in = ok && !(half && s > 0);
      qf[s] = in ? *(const u32x4 *)(qr + 16 * s) : zero4();
      of[s] = in ? *(const u32x4 *)(orow + 16 * s) : zero4();
    }
  }
  f32x16 acc[NDB];
#pragma unroll
  for (int d = 0; d < NDB; ++d) acc[d] = zero16();

  TileOffsets<D> to;
  to.init(lane);
  DmaPlan<BN, D, 4> dma;
  dma.init(w, lane, half);
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
      creg = key < Lk ? -(bias + p.score_mod[p.mod_base(b) + key0 + key]) * kLog2e : 0.0f;
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

  if (!CAUSAL && p.rsplit > 1 &&
      !split_combine<NDB, 4>([&](int i) SIGATTN_INLINE -> f32x16 & { return acc[i]; },
                             p.rs_part + (int64_t)ritem * p.rsplit * (BM * D), p.rs_cnt + ritem, rchunk,
                             p.rsplit, w, lane))
    return;

  if (my_q < p.q_rows_out(Lq)) {
    uint16_t *row = dQb + (int64_t)my_q * p.sq_t;
    const bool valid = my_q < Lq;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        if (half && g >= 2) break;  // columns 16..31: not in the tensor
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

template <typename T, int D, bool CAUSAL, bool SCOREMOD>
__global__ __launch_bounds__(256, 2) void bwd_dq_kernel(const KParams p) {
  __shared__ unsigned long long gap_lds[2];
  const int wg = gap_prologue<2>(p, gap_lds);  // packed layouts: leading gap-zeroing workgroups
  if (wg >= 0) bwd_dq_body<T, D, CAUSAL, SCOREMOD>(p, wg);
}

// ---------------------------------------------------------------------------
// dK/dV: workgroup = 4 waves x 32 keys (one wave per SIMD); the
// queries stream through a 4-stage ring of 64-query Q and dO tiles as a
// continuous sequence of 32-query blocks g.  Per block and wave:
//   S = Q·Kᵀ and dP = dO·Vᵀ (A: Q / dO rows from LDS, B: K / V rows held in
//   registers; accumulators: lane = key column, registers = query rows),
//   dVᵀ += dOᵀ·P and dKᵀ += Qᵀ·dS (A: dOᵀ / Qᵀ via ds_read_b64_tr_b16,
//   B: packed P / dS words straight from the accumulator layout).
// Region r runs, as one straight-line sequence, the S / dP MFMAs of block r,
// the gradient MFMAs of block r-2 and the P / dS VALU work of block r-1; every
// MFMA A operand is read from LDS eight MFMAs ahead through a rotating
// register queue, so no MFMA waits on a fresh LDS read.  Element masks
// (causal diagonal, seq_lens_q, pipeline fill) are applied to the packed
// words of the few blocks that need them.
// ---------------------------------------------------------------------------
template <typename T, int D, bool CAUSAL, bool SCOREMOD, bool DSOUT>
__device__ __forceinline__ void bwd_dkdv_body(const KParams &p, const int wg) {
  constexpr int BN = 128;                 // keys per workgroup (32 per wave)
  constexpr int BMQ = 64;                 // queries per LDS tile (two 32-query blocks)
  constexpr int NST = 4;                  // LDS ring stages
  constexpr int NKS = D / 16, NDB = D / 32;
  constexpr int NM = 2 * NKS + 4 * NDB;   // MFMAs per region
  constexpr int LA = D <= 64 ? 4 : 8;     // operand read-ahead, in MFMAs
  constexpr int NWIN = NM / 4;            // VALU windows (four MFMAs each) per region
  constexpr int PPW = 8 / NWIN;           // element pairs per window
  constexpr int BAR = NM - LA;            // MFMA position of the tile barrier in odd regions
  static_assert(NM % LA == 0 && BAR % 4 == 0, "region shape");
  // The region loop unrolls 8 regions (4 tiles); its compile-time stage
  // indices need 4 tiles to be a whole number of ring turns.
  static_assert(4 % NST == 0, "ring stages");

  __shared__ __attribute__((aligned(16))) uint16_t sQ[NST][BMQ * D];
  __shared__ __attribute__((aligned(16))) uint16_t sO[NST][BMQ * D];

  int b, h, kblk;
  int ritem = 0, rchunk = 0;  // range split: the item and this workgroup's chunk of its queries
  if (!CAUSAL && !DSOUT && p.rsplit > 1) {
    int bh;
    ritem = wg / p.rsplit, rchunk = wg % p.rsplit;
    dense_item(ritem, p.B * p.H, p.nblk, true, bh, kblk);
    b = bh / p.H, h = bh % p.H;
  } else if (p.ragged() && p.B <= 64) {
    const auto lq = [&](int i) SIGATTN_INLINE { return p.len_q(i); };
    const auto lk = [&](int i) SIGATTN_INLINE { return p.len_k(i); };
    const WorkItem it = CAUSAL ? WorkOrder::by_level(wg, p.B, p.H, lk, BN, p.nblk, false, p.ncu,
                                                     D <= 64 ? 2 : 1)
                               : WorkOrder::by_stream(wg, p.B, p.H, lk, BN, p.nblk, lq);
    b = it.b, h = it.h, kblk = it.blk;
  } else {
    const int BH = p.B * p.H;
    int bh;
    dense_item(wg, BH, p.nblk, !CAUSAL, bh, kblk);  // causal: low key blocks (the most work) first
    b = bh / p.H, h = bh % p.H;
  }
  const int Lq = p.len_q(b);
  const int Lk = p.len_k(b);
  const bool half = p.half_head(D);  // head_dim 16 in this D = 32 kernel
  // Padding item: its zero dK and dV rows as part of contiguous spans (see zero_row_span).
  if (kblk * BN >= Lk && p.k_rows_contiguous(half ? 16 : D)) {
    const int r1 = min(kblk * BN + BN, p.Tk);
    zero_row_span((uint16_t *)p.dk + (int64_t)b * p.sk_b, p.sk_t, kblk * BN, r1, h, p.H, threadIdx.x, 256);
    zero_row_span((uint16_t *)p.dv + (int64_t)b * p.sk_b, p.sk_t, kblk * BN, r1, h, p.H, threadIdx.x, 256);
    return;
  }

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, hi = lane >> 5;
  const int k0 = kblk * BN, kw = k0 + w * 32, my_k = kw + l32;

  const int64_t qoff = p.q_base(b, h);
  const int64_t koff = p.k_base(b, h);
  const uint16_t *Qb = (const uint16_t *)p.q + qoff;
  const uint16_t *dOb = (const uint16_t *)p.dout + qoff;
  const uint16_t *Kb = (const uint16_t *)p.k + koff;
  const uint16_t *Vb = (const uint16_t *)p.v + koff;
  uint16_t *dKb = (uint16_t *)p.dk + koff;
  uint16_t *dVb = (uint16_t *)p.dv + koff;

  // Causal: queries before the workgroup's first key see none of its keys.
  // Range split: this workgroup's chunk of the item's query tiles.
  int mstart = CAUSAL ? (k0 / BMQ) * BMQ : 0;
  int mend = (k0 >= Lk) ? mstart : Lq;
  if (!CAUSAL && !DSOUT && p.rsplit > 1 && k0 < Lk) {
    const int ntq = (Lq + BMQ - 1) / BMQ;
    mstart = split_tile(rchunk, p.rsplit, ntq) * BMQ;
    mend = min(Lq, split_tile(rchunk + 1, p.rsplit, ntq) * BMQ);
  }
  const int ntiles = mend > mstart ? (mend - mstart + BMQ - 1) / BMQ : 0;
  const int NB = 2 * ntiles;

  const float scale = *p.scale;
  const float bias = p.bias[b];
  const float nsl = -scale * kLog2e;
  const bool kok = my_k < Lk;
  float nc = -bias * kLog2e;
  if (SCOREMOD) nc = kok ? -(bias + p.score_mod[p.mod_base(b) + my_k]) * kLog2e : 0.0f;

  u32x4 kf[NKS], vf[NKS];
  {
    const uint16_t *kr = Kb + (int64_t)my_k * p.sk_t + 8 * hi;
    const uint16_t *vr = Vb + (int64_t)my_k * p.sk_t + 8 * hi;
#pragma unroll
    for (int s = 0; s < NKS; ++s) {
      const bool in = kok && !(half && s > 0);
      kf[s] = in ? *(const u32x4 *)(kr + 16 * s) : zero4();
      vf[s] = in ? *(const u32x4 *)(vr + 16 * s) : zero4();
    }
  }
  // Consume the K / V loads before the loop, so the compiler's wait for them
  // is not placed at the loop head, where it would also wait for tile copies.
#pragma unroll
  for (int s = 0; s < NKS; ++s) asm volatile("" ::"v"(kf[s]), "v"(vf[s]));

  f32x16 dka[NDB], dva[NDB];
#pragma unroll
  for (int d = 0; d < NDB; ++d) { dka[d] = zero16(); dva[d] = zero16(); }

  TileOffsets<D> to;
  to.init(lane);
  DmaPlan<BMQ, D, 4> dma;
  dma.init(w, lane, half);
  const int q_stride_bytes = (int)(p.sq_t * 2);
  auto issue = [&](int st, int t) SIGATTN_INLINE {
    dma.issue(sQ[st], Qb + (int64_t)mstart * p.sq_t, q_stride_bytes, t * BMQ, mend - mstart);
    dma.issue(sO[st], dOb + (int64_t)mstart * p.sq_t, q_stride_bytes, t * BMQ, mend - mstart);
  };

  f32x16 sacc[2], pacc[2];       // S and dP accumulators, by block parity
  uint32_t pw[2][8], dw[2][8];   // packed P and dS words, by block parity
  u32x4 opq[LA];                 // A operands of the next LA MFMAs (slot = position % LA)
  float ex[PPW][2];              // exp2 terms of the next element pairs

  // A operand of MFMA m of the region whose blocks (S/dP block, gradient
  // block) sit at tile rows kl in ring stages stc / stg.
  auto read_op = [&](int m, int stc, int stg, int kl) SIGATTN_INLINE {
    if (m < 2 * NKS) {
      return (m % 2 == 0) ? ld_row<D>(sQ[stc], to, kl, m / 2) : ld_row<D>(sO[stc], to, kl, m / 2);
    } else {
      const int i = m - 2 * NKS, j = i / (2 * NDB), dbi = (i / 2) % NDB;
      return (i % 2 == 0) ? ld_tr<D>(sO[stg], to, kl / 16 + j, dbi)
                          : ld_tr<D>(sQ[stg], to, kl / 16 + j, dbi);
    }
  };

  // Zeroes the P and dS entries of block g whose query lies before the
  // block range (pipeline fill; as unsigned such queries may also wrap to
  // huge values), at or past seq_lens_q, or (causal) before the lane's key.
  auto mask_words = [&](int slot, int g) SIGATTN_INLINE {
    int qbase = mstart + 32 * g;
    asm volatile("" : "+s"(qbase));  // keeps this rare fix-up in its own branch
    const unsigned lo = CAUSAL ? (unsigned)max(my_k, mstart) : (unsigned)mstart;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int i = 2 * e;
      const unsigned q0 = (unsigned)(qbase + 8 * (i / 4) + 4 * hi + (i % 4));
      const bool ok0 = q0 >= lo && q0 < (unsigned)Lq;
      const bool ok1 = q0 + 1u >= lo && q0 + 1u < (unsigned)Lq;
      const uint32_t m = (ok0 ? 0x0000ffffu : 0u) | (ok1 ? 0xffff0000u : 0u);
      pw[slot][e] &= m;
      dw[slot][e] &= m;
    }
  };
  auto needs_mask = [&](int g) SIGATTN_INLINE {
    const int qb0 = mstart + 32 * g;
    return g < 0 || qb0 + 32 > Lq || (CAUSAL && qb0 < kw + 31);
  };

  // Two-pass backward: the masked dS words of block g (slot `slot`) become
  // this wave's tile (query block mstart/32 + g, key block kw/32) of the dS
  // workspace (DsLayout).  Tiles of queries past seq_lens_q, of keys past
  // seq_lens_k, or (causal) wholly above the diagonal are not stored; the dQ
  // pass reads none of them.
  const int kbw = kw / 32;
  uint16_t *ds_bh = nullptr;
  if constexpr (DSOUT)
    ds_bh = p.ds + ((int64_t)b * p.H + h) * DsLayout::per_bh(p.ds_nqb, p.ds_nkb, CAUSAL) *
                       DsLayout::kTileElems;
  // Every region issues exactly two store instructions, so the tile
  // barrier can wait for its copies with a fixed vmcnt while the stores are
  // still in flight: a skipped tile is a store through a buffer resource of
  // zero bytes, which the hardware drops.
  auto store_ds = [&](int slot, int g) SIGATTN_INLINE {
    const int qb = mstart / 32 + g;
    const bool ok = g >= 0 && 32 * qb < Lq && kw < Lk && (!CAUSAL || qb >= kbw);
    // Buffer over this wave's tile (or over nothing).
    const uint16_t *tp = ds_bh + (ok ? DsLayout::tile(qb, kbw, p.ds_nqb, CAUSAL) : 0) * DsLayout::kTileElems;
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc((void *)tp, (short)0, ok ? 2048 : 0, kBufferWord3);
    const int off = 16 * lane;
    __builtin_amdgcn_raw_buffer_store_b128((u32x4){dw[slot][0], dw[slot][1], dw[slot][2], dw[slot][3]}, rs,
                                           off, 0, kStoreNT);
    __builtin_amdgcn_raw_buffer_store_b128((u32x4){dw[slot][4], dw[slot][5], dw[slot][6], dw[slot][7]}, rs,
                                           off + 1024, 0, kStoreNT);
  };

  // One region (U = r mod 8, so every slot and ring stage is static).
  auto region = [&](int r, auto u_tag) SIGATTN_INLINE {
    constexpr int U = decltype(u_tag)::value;
    constexpr int SL = U % 2;                     // parity of blocks r and r-2
    constexpr int KL = 32 * (U % 2);              // tile rows of blocks r and r-2
    constexpr int KLn = 32 * ((U + 1) % 2);       // tile rows of blocks r+1 and r-1
    constexpr int STC = (U / 2) % NST;            // stage of block r
    constexpr int STG = ((U + 6) / 2) % NST;      // stage of block r-2
    constexpr int STCn = ((U + 1) / 2) % NST;     // stage of block r+1
    constexpr int STGn = ((U + 7) / 2) % NST;     // stage of block r-1
#pragma unroll
    for (int win = 0; win < NWIN; ++win) {
      if ((U % 2) == 1 && win * 4 == BAR) {
        // Publish tile (r+1)/2 before the first read of it (the read-ahead of
        // block r+1), then start the copy of the tile after it into the stage
        // of the tile three back, whose last reads were two regions ago.
        const int t1 = (r + 1) / 2;
        if (t1 < ntiles) {
          if constexpr (DSOUT) {
            // Tile t1's copies are older than the dS stores issued since
            // (two per region; region 1 follows only region 0's), which may
            // stay in flight.
            if (r == 1) wait_vm<2>();
            else wait_vm<4>();
          } else {
            wait_dma();
          }
          asm volatile("" ::: "memory");
          __builtin_amdgcn_s_barrier();
          asm volatile("" ::: "memory");
          if (t1 + 1 < ntiles) issue((t1 + 1) % NST, t1 + 1);
        }
      }
      // dS of block r-2 (its words stay intact until the next region's
      // VALU work), stored where the next vmcnt(0) is furthest away: at the
      // start of even regions, after the tile barrier in odd ones.
      if constexpr (DSOUT) {
        if (((U % 2) == 0 && win == 0) || ((U % 2) == 1 && win * 4 == BAR)) store_ds(SL, r - 2);
      }
      // One wait for the window's four operands instead of one per MFMA.
      asm volatile("" ::"v"(opq[(win * 4) % LA]), "v"(opq[(win * 4 + 1) % LA]),
                   "v"(opq[(win * 4 + 2) % LA]), "v"(opq[(win * 4 + 3) % LA]));
#pragma unroll
      for (int mm = 0; mm < 4; ++mm) {
        const int m = win * 4 + mm;
        const u32x4 a = opq[m % LA];
        if (m < 2 * NKS) {
          if (m % 2 == 0) sacc[SL] = Elem<T>::mfma(a, kf[m / 2], m == 0 ? zero16() : sacc[SL]);
          else pacc[SL] = Elem<T>::mfma(a, vf[m / 2], m == 1 ? zero16() : pacc[SL]);
        } else {
          const int i = m - 2 * NKS, j = i / (2 * NDB), dbi = (i / 2) % NDB;
          if (i % 2 == 0) {
            const u32x4 bp = (u32x4){pw[SL][4 * j], pw[SL][4 * j + 1], pw[SL][4 * j + 2], pw[SL][4 * j + 3]};
            dva[dbi] = Elem<T>::mfma(a, bp, dva[dbi]);
          } else {
            const u32x4 bd = (u32x4){dw[SL][4 * j], dw[SL][4 * j + 1], dw[SL][4 * j + 2], dw[SL][4 * j + 3]};
            dka[dbi] = Elem<T>::mfma(a, bd, dka[dbi]);
          }
        }
        // Refill the slot with the operand of MFMA m + LA (next region when
        // it wraps: S/dP block r+1, gradient block r-1).
        if (m + LA < NM) opq[m % LA] = read_op(m + LA, STC, STG, KL);
        else opq[m % LA] = read_op(m + LA - NM, STCn, STGn, KLn);
      }
      // VALU: P / dS of block r-1 (parity 1-SL).  Stage B (reciprocal, dS,
      // packing) for this window's pairs, stage A (exp2) for the next
      // window's pairs -- or, in the last window, the first pairs of block r.
      float nx[PPW][2];
#pragma unroll
      for (int pp = 0; pp < PPW; ++pp) {
        const bool last = win + 1 == NWIN;
        const int e = last ? pp : (win + 1) * PPW + pp;
        const f32x16 &sv = last ? sacc[SL] : sacc[1 - SL];
        nx[pp][0] = __builtin_amdgcn_exp2f(__builtin_fmaf(acc_read(sv[2 * e]), nsl, nc));
        nx[pp][1] = __builtin_amdgcn_exp2f(__builtin_fmaf(acc_read(sv[2 * e + 1]), nsl, nc));
      }
#pragma unroll
      for (int pp = 0; pp < PPW; ++pp) {
        const int e = win * PPW + pp;
        // Written stage by stage for both elements, so each transcendental
        // result is not consumed by the very next instruction.
        float pr[2], t[2], ds[2];
#pragma unroll
        for (int x = 0; x < 2; ++x) pr[x] = __builtin_amdgcn_rcpf(1.0f + ex[pp][x]);
#pragma unroll
        for (int x = 0; x < 2; ++x) t[x] = pr[x] * acc_read(pacc[1 - SL][2 * e + x]);
#pragma unroll
        for (int x = 0; x < 2; ++x) ds[x] = __builtin_fmaf(-pr[x], t[x], t[x]);
        pw[1 - SL][e] = Elem<T>::pack(pr[0], pr[1]);
        dw[1 - SL][e] = Elem<T>::pack(ds[0], ds[1]);
        asm volatile("" : "+v"(pw[1 - SL][e]), "+v"(dw[1 - SL][e]));
      }
#pragma unroll
      for (int pp = 0; pp < PPW; ++pp) { ex[pp][0] = nx[pp][0]; ex[pp][1] = nx[pp][1]; }
#pragma unroll
      for (int mm = 0; mm < 4; ++mm) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
        __builtin_amdgcn_sched_group_barrier(0x402, 4 * PPW, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
    if (r == 0 || needs_mask(r - 1)) mask_words(1 - SL, r - 1);
  };

  // Pipeline fill: blocks -2 and -1 contribute P = dS = 0; their gradient
  // operands come from ring stage 3, zeroed here (tile 3 arrives only after
  // region 3), so 0 * operand stays 0.
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    sacc[x] = zero16();
    pacc[x] = zero16();
#pragma unroll
    for (int e = 0; e < 8; ++e) { pw[x][e] = 0u; dw[x][e] = 0u; }
  }
#pragma unroll
  for (int pp = 0; pp < PPW; ++pp) { ex[pp][0] = 0.0f; ex[pp][1] = 0.0f; }
  for (int i = tid; i < BMQ * D / 8; i += 256) {
    *(u32x4 *)&sQ[NST - 1][8 * i] = zero4();
    *(u32x4 *)&sO[NST - 1][8 * i] = zero4();
  }
  if (ntiles > 0) {
    issue(0, 0);
    wait_dma();
  }
  __syncthreads();
  if (ntiles > 1) issue(1, 1);
#pragma unroll
  for (int m = 0; m < LA; ++m) opq[m] = read_op(m, 0, NST - 1, 0);

  for (int r0 = 0; r0 < NB + 2; r0 += 8) {
    region(r0 + 0, std::integral_constant<int, 0>{});
    if (r0 + 1 < NB + 2) region(r0 + 1, std::integral_constant<int, 1>{});
    if (r0 + 2 < NB + 2) region(r0 + 2, std::integral_constant<int, 2>{});
    if (r0 + 3 < NB + 2) region(r0 + 3, std::integral_constant<int, 3>{});
    if (r0 + 4 < NB + 2) region(r0 + 4, std::integral_constant<int, 4>{});
    if (r0 + 5 < NB + 2) region(r0 + 5, std::integral_constant<int, 5>{});
    if (r0 + 6 < NB + 2) region(r0 + 6, std::integral_constant<int, 6>{});
    if (r0 + 7 < NB + 2) region(r0 + 7, std::integral_constant<int, 7>{});
  }

  if (!CAUSAL && !DSOUT && p.rsplit > 1 &&
      !split_combine<2 * NDB, 4>(
          [&](int i) SIGATTN_INLINE -> f32x16 & { return i < NDB ? dka[i] : dva[i - NDB]; },
          p.rs_part + (int64_t)ritem * p.rsplit * (2 * BN * D), p.rs_cnt + ritem, rchunk, p.rsplit, w, lane))
    return;

  if (my_k < p.k_rows_out(Lk)) {
    uint16_t *kr = dKb + (int64_t)my_k * p.sk_t;
    uint16_t *vr = dVb + (int64_t)my_k * p.sk_t;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        if (half && g >= 2) break;  // columns 16..31: not in the tensor
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

template <typename T, int D, bool CAUSAL, bool SCOREMOD, bool DSOUT>
__global__ __launch_bounds__(256, (D <= 64 ? 2 : 1)) void bwd_dkdv_kernel(const KParams p) {
  bwd_dkdv_body<T, D, CAUSAL, SCOREMOD, DSOUT>(p, blockIdx.x);
}

// The recompute backward's two kernels in one launch (dense problems at
// D <= 64 whose two grids together need at most one workgroup per CU): the
// first ndq workgroups run dQ items, the rest dK/dV items, so the two halves
// share the GPU instead of each leaving half of it idle.  The bodies are the
// kernels' own, so results are bit-identical to the two launches.  The two
// bodies' LDS adds up (96 KB at D = 64), so one workgroup fits per CU.
template <typename T, int D, bool CAUSAL, bool SCOREMOD>
__global__ __launch_bounds__(256, 1) void bwd_fused_kernel(const KParams pq, const KParams pk, int ndq) {
  if ((int)blockIdx.x < ndq) bwd_dq_body<T, D, CAUSAL, SCOREMOD>(pq, blockIdx.x);
  else bwd_dkdv_body<T, D, CAUSAL, SCOREMOD, false>(pk, (int)blockIdx.x - ndq);
}

// ---------------------------------------------------------------------------
// dK/dV at D = 128 by wave pairs: workgroup = 8 waves, 128 keys.  Waves w and
// w + 4 own the same 32 keys and share SIMD w (waves are dealt to the four
// SIMDs round-robin), so each SIMD runs one wave of each role:
//   role A (waves 0-3): S = Q·Kᵀ (K rows in registers), P = sigmoid(S),
//     dVᵀ += dOᵀ·P, and every Q / dO tile copy;
//   role B (waves 4-7): dP = dO·Vᵀ (V rows in registers), dS = P·(1-P)·dP,
//     dKᵀ += Qᵀ·dS, and the dS tiles of the two-pass backward.
// The copies and the stores sit in different waves because a wave's memory
// operations complete in issue order: a copy wait behind dS stores would
// also wait for their acknowledgement (measured 3-7 % of the kernel).
// A hands P to B through LDS in fp32, so dS is computed from exactly the
// values bwd_dkdv_kernel uses and dK, dV are bit for bit the same.  Either
// role needs about half that kernel's registers (every accumulator stays in
// VGPRs), and with two waves per SIMD one wave's sigmoid work issues while
// the other wave's MFMAs run.
// The queries stream as in bwd_dkdv_kernel: 64-query tiles of Q and dO in a
// 4-stage ring, processed as 32-query blocks g.  Region r runs
//   A: S of block r, P of block r-1 (packed for the dV product and stored to
//      LDS for B), dV of block r-2;
//   B: dS of block r-2 (P from LDS, dP from its accumulator), dP of block r,
//      dK of block r-2.
// Every region has one barrier, placed before the operand read-ahead reaches
// the next region's first MFMAs: it publishes the tile of the next region
// (A waits for its copies just before) and the P that A stored before it,
// which B reads in the next region (the two P buffers alternate by block
// parity).
// ---------------------------------------------------------------------------
// Dense causal grids in dense_item's XCD-grouped order too: paired key
// blocks make every workgroup's work equal, so grouping costs no balance, and
// each XCD then reads the Q and dO rows of two (batch, head) pairs at a time
// instead of eight.  Measured at B=4 L=4096 H=16 D=128 causal: HBM fetch
// 757 -> 278 MB per launch (the algorithmic 268 MB), 0.661 -> 0.647 ms.
#ifndef SIGATTN_DKDV_GROUPED
#define SIGATTN_DKDV_GROUPED 1
#endif
constexpr bool kDkdvGrouped = SIGATTN_DKDV_GROUPED != 0;

template <typename T, bool CAUSAL, bool SCOREMOD, bool DSOUT>
__global__ __launch_bounds__(512, 1) void bwd_dkdv_pair_kernel(const KParams p) {
  constexpr int D = 128;
  constexpr int BN = 128;                 // keys per workgroup (32 per wave pair)
  constexpr int BMQ = 64;                 // queries per LDS tile (two 32-query blocks)
  constexpr int NST = 4;                  // LDS ring stages
  constexpr int NKS = D / 16, NDB = D / 32;
  constexpr int NM = NKS + 2 * NDB;       // MFMAs per region and wave
  constexpr int LA = 4;                   // operand read-ahead, in MFMAs
  constexpr int BAR = NM - LA;            // MFMA position of the region's barrier
  using Dma = DmaPlan<BMQ, D, 4>;
  constexpr int NCP = 2 * Dma::NI;        // copy instructions per tile and A wave
  static_assert(NM % LA == 0 && BAR >= 8, "region shape");
  // The region loop unrolls 8 regions (4 tiles); its compile-time stage
  // indices need 4 tiles to be a whole number of ring turns.
  static_assert(4 % NST == 0, "ring stages");

  __shared__ __attribute__((aligned(16))) uint16_t sQ[NST][BMQ * D];
  __shared__ __attribute__((aligned(16))) uint16_t sO[NST][BMQ * D];
  // P of block g, for pair w: sP[g & 1][w], lane l's elements 4c..4c+3 at 256 c + 4 l.
  __shared__ __attribute__((aligned(16))) float sP[2][4][1024];

  // Work: ragged batches take one key block per workgroup in WorkOrder's
  // order.  Dense problems take key blocks j and nblk-1-j in sequence
  // (grid = ceil(nblk/2) per (batch, head)): under the causal mask the two
  // together cost the same for every j, so all workgroups are equal, and
  // the grid has half as many workgroup starts.  A dense non-causal grid
  // that would not fill the GPU paired runs one key block per workgroup
  // (grid = nblk per (batch, head)).
  int b, h, kblk0, nitems;
  if (p.ragged() && p.B <= 64) {
    const auto lq = [&](int i) SIGATTN_INLINE { return p.len_q(i); };
    const auto lk = [&](int i) SIGATTN_INLINE { return p.len_k(i); };
    const WorkItem it = CAUSAL ? WorkOrder::by_level(blockIdx.x, p.B, p.H, lk, BN, p.nblk, false, p.ncu, 1)
                               : WorkOrder::by_stream(blockIdx.x, p.B, p.H, lk, BN, p.nblk, lq);
    b = it.b, h = it.h, kblk0 = it.blk, nitems = 1;
  } else {
    const int BH = p.B * p.H;
    int bh;
    dense_item(blockIdx.x, BH, (int)(gridDim.x / BH), !CAUSAL || kDkdvGrouped, bh, kblk0);
    const bool paired = (int)(gridDim.x / BH) < p.nblk;
    nitems = paired && p.nblk - 1 - kblk0 > kblk0 ? 2 : 1;
    b = bh / p.H, h = bh % p.H;
  }
  for (int item = 0; item < nitems; ++item) {
    const int kblk = item == 0 ? kblk0 : p.nblk - 1 - kblk0;
    // The previous key block's last reads of the ring and of the P buffers
    // precede this block's fills.
    if (item > 0) __syncthreads();
    const int Lq = p.len_q(b);
    const int Lk = p.len_k(b);
    // Padding item (ragged batches, one key block per workgroup): its zero
    // dK and dV rows as part of contiguous spans (see zero_row_span).
    if (nitems == 1 && kblk * BN >= Lk && p.k_rows_contiguous(D)) {
      const int r1 = min(kblk * BN + BN, p.Tk);
      zero_row_span((uint16_t *)p.dk + (int64_t)b * p.sk_b, p.sk_t, kblk * BN, r1, h, p.H, threadIdx.x, 512);
      zero_row_span((uint16_t *)p.dv + (int64_t)b * p.sk_b, p.sk_t, kblk * BN, r1, h, p.H, threadIdx.x, 512);
      return;
    }

    const int tid = threadIdx.x, lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int pair = wv & 3;
    const bool role_a = wv < 4;
    const int l32 = lane & 31, hi = lane >> 5;
    const int k0 = kblk * BN, kw = k0 + pair * 32, my_k = kw + l32;

    const int64_t qoff = p.q_base(b, h);
    const int64_t koff = p.k_base(b, h);
    const uint16_t *Qb = (const uint16_t *)p.q + qoff;
    const uint16_t *dOb = (const uint16_t *)p.dout + qoff;

    // Causal: queries before the workgroup's first key see none of its keys.
    const int mstart = CAUSAL ? (k0 / BMQ) * BMQ : 0;
    const int mend = (k0 >= Lk) ? mstart : Lq;
    const int ntiles = mend > mstart ? (mend - mstart + BMQ - 1) / BMQ : 0;
    const int NB = 2 * ntiles;

    const float scale = *p.scale;
    const bool kok = my_k < Lk;

    TileOffsets<D> to;
    to.init(lane);
    Dma dma;
    dma.init(pair, lane);
    const int q_stride_bytes = (int)(p.sq_t * 2);
    auto issue = [&](int st, int t) SIGATTN_INLINE {
      dma.issue(sQ[st], Qb + (int64_t)mstart * p.sq_t, q_stride_bytes, t * BMQ, mend - mstart);
      dma.issue(sO[st], dOb + (int64_t)mstart * p.sq_t, q_stride_bytes, t * BMQ, mend - mstart);
    };

    // Zeroes the packed words of block g whose query lies before the block
    // range (pipeline fill; as unsigned such queries may also wrap to huge
    // values), at or past seq_lens_q, or (causal) before the lane's key.
    auto mask_words = [&](uint32_t(&wds)[8], int g) SIGATTN_INLINE {
      int qbase = mstart + 32 * g;
      asm volatile("" : "+s"(qbase));  // keeps this rare fix-up in its own branch
      const unsigned lo = CAUSAL ? (unsigned)max(my_k, mstart) : (unsigned)mstart;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int i = 2 * e;
        const unsigned q0 = (unsigned)(qbase + 8 * (i / 4) + 4 * hi + (i % 4));
        const bool ok0 = q0 >= lo && q0 < (unsigned)Lq;
        const bool ok1 = q0 + 1u >= lo && q0 + 1u < (unsigned)Lq;
        wds[e] &= (ok0 ? 0x0000ffffu : 0u) | (ok1 ? 0xffff0000u : 0u);
      }
    };
    auto needs_mask = [&](int g) SIGATTN_INLINE {
      const int qb0 = mstart + 32 * g;
      return g < 0 || qb0 + 32 > Lq || (CAUSAL && qb0 < kw + 31);
    };

    // Pipeline fill: the gradient products of blocks -2 and -1 read ring stage
    // NST-1 (zeroed here; tile NST-1 arrives only in region 2) against zero
    // words, and B's first dS reads the zeroed P buffer 0.
    for (int i = tid; i < BMQ * D / 8; i += 512) {
      *(u32x4 *)&sQ[NST - 1][8 * i] = zero4();
      *(u32x4 *)&sO[NST - 1][8 * i] = zero4();
    }
    for (int i = tid; i < 2 * 4 * 1024 / 4; i += 512) *(u32x4 *)(&sP[0][0][0] + 4 * i) = zero4();
    if (role_a && ntiles > 0) {
      issue(0, 0);
      if (ntiles > 1) {
        issue(1, 1);
        wait_vm<NCP>();
      } else {
        wait_dma();
      }
    }
    __syncthreads();

    const int kmax = p.k_rows_out(Lk);
    if (role_a) {
      // ---------------- role A: S, P, dV ----------------
      const float bias = p.bias[b];
      const float nsl = -scale * kLog2e;
      float nc = -bias * kLog2e;
      if (SCOREMOD) nc = kok ? -(bias + p.score_mod[p.mod_base(b) + my_k]) * kLog2e : 0.0f;
      u32x4 kf[NKS];
      {
        const uint16_t *kr = (const uint16_t *)p.k + koff + (int64_t)my_k * p.sk_t + 8 * hi;
#pragma unroll
        for (int s = 0; s < NKS; ++s) kf[s] = kok ? *(const u32x4 *)(kr + 16 * s) : zero4();
      }
#pragma unroll
      for (int s = 0; s < NKS; ++s) asm volatile("" ::"v"(kf[s]));

      f32x16 dva[NDB], sacc[2];
      uint32_t pw[2][8];
#pragma unroll
      for (int d = 0; d < NDB; ++d) dva[d] = zero16();
#pragma unroll
      for (int x = 0; x < 2; ++x) {
        sacc[x] = zero16();
#pragma unroll
        for (int e = 0; e < 8; ++e) pw[x][e] = 0u;
      }
      float *xb0 = &sP[0][pair][4 * lane];
      float *xb1 = &sP[1][pair][4 * lane];

      // A operand of MFMA m of the region whose blocks (S block, dV block) sit
      // at tile rows kl in ring stages stc / stg.
      auto read_op = [&](int m, int stc, int stg, int kl) SIGATTN_INLINE {
        if (m % 2 == 0) return ld_row<D>(sQ[stc], to, kl, m / 2);
        const int i = m / 2;
        return ld_tr<D>(sO[stg], to, kl / 16 + i / NDB, i % NDB);
      };
      u32x4 opq[LA];
#pragma unroll
      for (int m = 0; m < LA; ++m) opq[m] = read_op(m, 0, NST - 1, 0);

      auto region = [&](int r, auto u_tag) SIGATTN_INLINE {
        constexpr int U = decltype(u_tag)::value;
        constexpr int SL = U % 2;                  // parity of blocks r and r-2
        constexpr int KL = 32 * (U % 2), KLn = 32 * ((U + 1) % 2);
        constexpr int STC = (U / 2) % NST, STG = ((U + 6) / 2) % NST;
        constexpr int STCn = ((U + 1) / 2) % NST, STGn = ((U + 7) / 2) % NST;
        float *xb = SL ? xb0 : xb1;                // P buffer of block r-1
        float keep[2];
#pragma unroll
        for (int m = 0; m < NM; ++m) {
          if (m == BAR) {
            if constexpr (U % 2 == 1) {
              // The next region starts tile t: wait for this wave's copies
              // of it (tile t+1's may stay in flight).
              const int t = (r + 1) / 2;
              if (t < ntiles) {
                if (t + 1 < ntiles) wait_vm<NCP>();
                else wait_dma();
              }
            }
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            if constexpr (U % 2 == 0) {
              // Every wave has finished region r-1, the last to read the
              // stage of tile r/2 - 2: refill it with tile r/2 + 2.
              const int t = r / 2 + 2;
              if (t < ntiles) issue((U / 2 + 2) % NST, t);
            }
          }
          asm volatile("" ::"v"(opq[m % LA]));
          const u32x4 a = opq[m % LA];
          if (m % 2 == 0) {
            sacc[SL] = Elem<T>::mfma(a, kf[m / 2], m == 0 ? zero16() : sacc[SL]);
          } else {
            const int i = m / 2, j = i / NDB, dbi = i % NDB;
            const u32x4 bp = (u32x4){pw[SL][4 * j], pw[SL][4 * j + 1], pw[SL][4 * j + 2], pw[SL][4 * j + 3]};
            dva[dbi] = Elem<T>::mfma(a, bp, dva[dbi]);
          }
          if (m + LA < NM) opq[m % LA] = read_op(m + LA, STC, STG, KL);
          else opq[m % LA] = read_op(m + LA - NM, STCn, STGn, KLn);
          // P of block r-1: element pair m at MFMA position m, stored to LDS
          // four elements at a time.
          if (m < 8) {
            float pr[2];
#pragma unroll
            for (int x = 0; x < 2; ++x) {
              const float ex = __builtin_amdgcn_exp2f(__builtin_fmaf(sacc[1 - SL][2 * m + x], nsl, nc));
              pr[x] = __builtin_amdgcn_rcpf(1.0f + ex);
            }
            pw[1 - SL][m] = Elem<T>::pack(pr[0], pr[1]);
            if (m % 2 == 0) {
              keep[0] = pr[0];
              keep[1] = pr[1];
            } else {
              *(float4 *)(xb + 256 * (m / 2)) = make_float4(keep[0], keep[1], pr[0], pr[1]);
            }
          }
        }
        if (r == 0 || needs_mask(r - 1)) mask_words(pw[1 - SL], r - 1);
      };

      for (int r0 = 0; r0 < NB + 2; r0 += 8) {
        region(r0 + 0, std::integral_constant<int, 0>{});
        if (r0 + 1 < NB + 2) region(r0 + 1, std::integral_constant<int, 1>{});
        if (r0 + 2 < NB + 2) region(r0 + 2, std::integral_constant<int, 2>{});
        if (r0 + 3 < NB + 2) region(r0 + 3, std::integral_constant<int, 3>{});
        if (r0 + 4 < NB + 2) region(r0 + 4, std::integral_constant<int, 4>{});
        if (r0 + 5 < NB + 2) region(r0 + 5, std::integral_constant<int, 5>{});
        if (r0 + 6 < NB + 2) region(r0 + 6, std::integral_constant<int, 6>{});
        if (r0 + 7 < NB + 2) region(r0 + 7, std::integral_constant<int, 7>{});
      }

      if (my_k < kmax) {
        uint16_t *vr = (uint16_t *)p.dv + koff + (int64_t)my_k * p.sk_t;
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int d0 = db * 32 + 8 * g + 4 * hi;
            u32x2 ov;
            ov.x = Elem<T>::pack(dva[db][4 * g], dva[db][4 * g + 1]);
            ov.y = Elem<T>::pack(dva[db][4 * g + 2], dva[db][4 * g + 3]);
            if (!kok) ov = (u32x2){0u, 0u};
            *(u32x2 *)(vr + d0) = ov;
          }
        }
      }
    } else {
      // ---------------- role B: dP, dS, dK, tile copies ----------------
      u32x4 vf[NKS];
      {
        const uint16_t *vr = (const uint16_t *)p.v + koff + (int64_t)my_k * p.sk_t + 8 * hi;
#pragma unroll
        for (int s = 0; s < NKS; ++s) vf[s] = kok ? *(const u32x4 *)(vr + 16 * s) : zero4();
      }
#pragma unroll
      for (int s = 0; s < NKS; ++s) asm volatile("" ::"v"(vf[s]));

      f32x16 dka[NDB], pacc[2];
      uint32_t dw[8];
#pragma unroll
      for (int d = 0; d < NDB; ++d) dka[d] = zero16();
      pacc[0] = zero16();
      pacc[1] = zero16();
      const float *xb0 = &sP[0][pair][4 * lane];
      const float *xb1 = &sP[1][pair][4 * lane];

      // Two-pass backward: this wave's dS tile of block g (DsLayout), skipped
      // (a store through an empty buffer resource, which the hardware drops)
      // past seq_lens_q / seq_lens_k or wholly above the causal diagonal.
      const int kbw = kw / 32;
      uint16_t *ds_bh = nullptr;
      if constexpr (DSOUT)
        ds_bh = p.ds + ((int64_t)b * p.H + h) * DsLayout::per_bh(p.ds_nqb, p.ds_nkb, CAUSAL) *
                           DsLayout::kTileElems;
      auto store_ds = [&](int g) SIGATTN_INLINE {
        const int qb = mstart / 32 + g;
        const bool ok = g >= 0 && 32 * qb < Lq && kw < Lk && (!CAUSAL || qb >= kbw);
        const uint16_t *tp = ds_bh + (ok ? DsLayout::tile(qb, kbw, p.ds_nqb, CAUSAL) : 0) * DsLayout::kTileElems;
        const __amdgpu_buffer_rsrc_t rs =
            __builtin_amdgcn_make_buffer_rsrc((void *)tp, (short)0, ok ? 2048 : 0, kBufferWord3);
        const int off = 16 * lane;
        __builtin_amdgcn_raw_buffer_store_b128((u32x4){dw[0], dw[1], dw[2], dw[3]}, rs, off, 0, kStoreNT);
        __builtin_amdgcn_raw_buffer_store_b128((u32x4){dw[4], dw[5], dw[6], dw[7]}, rs, off + 1024, 0, kStoreNT);
      };

      auto read_op = [&](int m, int stc, int stg, int kl) SIGATTN_INLINE {
        if (m % 2 == 0) return ld_row<D>(sO[stc], to, kl, m / 2);
        const int i = m / 2;
        return ld_tr<D>(sQ[stg], to, kl / 16 + i / NDB, i % NDB);
      };
      u32x4 opq[LA];
#pragma unroll
      for (int m = 0; m < LA; ++m) opq[m] = read_op(m, 0, NST - 1, 0);

      auto region = [&](int r, auto u_tag) SIGATTN_INLINE {
        constexpr int U = decltype(u_tag)::value;
        constexpr int SL = U % 2;
        constexpr int KL = 32 * (U % 2), KLn = 32 * ((U + 1) % 2);
        constexpr int STC = (U / 2) % NST, STG = ((U + 6) / 2) % NST;
        constexpr int STCn = ((U + 1) / 2) % NST, STGn = ((U + 7) / 2) % NST;
        // dS of block r-2: P from A (stored in region r-1), dP from the
        // accumulator block r-2 left in pacc[SL].
        {
          const float *xb = SL ? xb1 : xb0;
          float4 pv[4];
#pragma unroll
          for (int c = 0; c < 4; ++c) pv[c] = *(const float4 *)(xb + 256 * c);
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float pr0 = (e % 2 == 0) ? pv[e / 2].x : pv[e / 2].z;
            const float pr1 = (e % 2 == 0) ? pv[e / 2].y : pv[e / 2].w;
            const float t0 = pr0 * pacc[SL][2 * e], t1 = pr1 * pacc[SL][2 * e + 1];
            dw[e] = Elem<T>::pack(__builtin_fmaf(-pr0, t0, t0), __builtin_fmaf(-pr1, t1, t1));
          }
          if (r < 2 || needs_mask(r - 2)) mask_words(dw, r - 2);
          if constexpr (DSOUT) store_ds(r - 2);
        }
#pragma unroll
        for (int m = 0; m < NM; ++m) {
          if (m == BAR) {
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
          }
          asm volatile("" ::"v"(opq[m % LA]));
          const u32x4 a = opq[m % LA];
          if (m % 2 == 0) {
            pacc[SL] = Elem<T>::mfma(a, vf[m / 2], m == 0 ? zero16() : pacc[SL]);
          } else {
            const int i = m / 2, j = i / NDB, dbi = i % NDB;
            const u32x4 bd = (u32x4){dw[4 * j], dw[4 * j + 1], dw[4 * j + 2], dw[4 * j + 3]};
            dka[dbi] = Elem<T>::mfma(a, bd, dka[dbi]);
          }
          if (m + LA < NM) opq[m % LA] = read_op(m + LA, STC, STG, KL);
          else opq[m % LA] = read_op(m + LA - NM, STCn, STGn, KLn);
        }
      };

      for (int r0 = 0; r0 < NB + 2; r0 += 8) {
        region(r0 + 0, std::integral_constant<int, 0>{});
        if (r0 + 1 < NB + 2) region(r0 + 1, std::integral_constant<int, 1>{});
        if (r0 + 2 < NB + 2) region(r0 + 2, std::integral_constant<int, 2>{});
        if (r0 + 3 < NB + 2) region(r0 + 3, std::integral_constant<int, 3>{});
        if (r0 + 4 < NB + 2) region(r0 + 4, std::integral_constant<int, 4>{});
        if (r0 + 5 < NB + 2) region(r0 + 5, std::integral_constant<int, 5>{});
        if (r0 + 6 < NB + 2) region(r0 + 6, std::integral_constant<int, 6>{});
        if (r0 + 7 < NB + 2) region(r0 + 7, std::integral_constant<int, 7>{});
      }

      if (my_k < kmax) {
        uint16_t *kr = (uint16_t *)p.dk + koff + (int64_t)my_k * p.sk_t;
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const int d0 = db * 32 + 8 * g + 4 * hi;
            u32x2 ok_;
            ok_.x = Elem<T>::pack(dka[db][4 * g] * scale, dka[db][4 * g + 1] * scale);
            ok_.y = Elem<T>::pack(dka[db][4 * g + 2] * scale, dka[db][4 * g + 3] * scale);
            if (!kok) ok_ = (u32x2){0u, 0u};
            *(u32x2 *)(kr + d0) = ok_;
          }
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// dQ of the two-pass backward: dQ = dS · K · scale from the dS tiles the dK/dV
// kernel stored (DsLayout), with no recomputation of S, P or dP.
// Workgroup = NW waves x 64 queries (two 32-query column blocks per wave);
// keys stream in stages of KB 32-key blocks through an NST-stage LDS ring:
// the K rows (shared by the waves) and each wave's own dS tiles (its two
// query blocks x KB key blocks), all by direct global->LDS copies issued
// NST-1 stages ahead, so about (NST-1) x (32 KB x KB dS + K) per CU is in
// flight against HBM latency.
//   dQᵀ[d, q] += Kᵀ[d, key] · dSᵀ[key, q]
// A = Kᵀ via ds_read_b64_tr_b16 from the row-major K rows; B = dSᵀ via
// ds_read_b64_tr_b16 from the dS tile, which the copy lays out key-major
// (64 bytes per key: its four 16-byte pieces (g-pair c, query half h) at
// slot 2c + h), so lane (query n, k-slot h) receives keys 16ks + 4h + {0..3}
// and 16ks + 8 + 4h + {0..3} -- the same key order as the Kᵀ read.
// Per 32 keys a wave reads 4 KB of dS and runs 16 MFMAs: the kernel is bound
// by HBM bandwidth.
// ---------------------------------------------------------------------------
#ifndef SIGATTN_DQDS_NT
#define SIGATTN_DQDS_NT 1
#endif
constexpr bool kDqDsNT = SIGATTN_DQDS_NT != 0;

// Waves per SIMD of the kernel's resident workgroups (its register budget).
template <int D, int NW, int KB, int NST> constexpr int dq_ds_waves_per_simd() {
  const int occ = 163840 / (NST * (32 * KB * D + NW * 2 * KB * DsLayout::kTileElems) * 2);
  return occ * NW / 4 > 1 ? occ * NW / 4 : 1;
}

template <typename T, int D, bool CAUSAL, int NW, int KB, int NST>
__global__ __launch_bounds__(64 * NW, (dq_ds_waves_per_simd<D, NW, KB, NST>())) void bwd_dq_ds_kernel(
    const KParams p) {
  constexpr int BM = 64 * NW, BN = 32 * KB;
  constexpr int NDB = D / 32;
  constexpr int TE = DsLayout::kTileElems;
  constexpr int KI = BN * D / 8 / 64 / NW;  // K-row copy instructions per wave and stage
  constexpr int NI = KI + 4 * KB;           // copy instructions per wave and stage
  constexpr int PF = NST - 1;               // stages in flight ahead of the one computed
  // Resident workgroups per CU, by the LDS ring's size (160 KB per CU).
  constexpr int OCC = 163840 / (NST * (BN * D + NW * 2 * KB * TE) * 2);
  static_assert(KI >= 1 && (NST - 2) * NI < 64 && OCC >= 1, "stage shape");

  __shared__ __attribute__((aligned(16))) uint16_t sK[NST][BN * D];
  __shared__ __attribute__((aligned(16))) uint16_t sS[NST][NW * 2 * KB * TE];

  const int wg = gap_prologue<2>(p, sK);  // packed layouts: leading gap-zeroing workgroups
  if (wg < 0) return;
  int b, h, qblk;
  if (p.ragged() && p.B <= 64) {
    const auto lq = [&](int i) SIGATTN_INLINE { return p.len_q(i); };
    const auto lk = [&](int i) SIGATTN_INLINE { return p.len_k(i); };
    const WorkItem it = CAUSAL ? WorkOrder::by_level(wg, p.B, p.H, lq, BM, p.nblk, true, p.ncu, OCC)
                               : WorkOrder::by_stream(wg, p.B, p.H, lq, BM, p.nblk, lk);
    b = it.b, h = it.h, qblk = it.blk;
  } else {
    const int BH = p.B * p.H;
    int bh;
    dense_item(wg, BH, p.nblk, !CAUSAL, bh, qblk);
    if (CAUSAL) qblk = p.nblk - 1 - qblk;  // heaviest query blocks first
    b = bh / p.H, h = bh % p.H;
  }
  const int Lq = p.len_q(b);
  const int Lk = p.len_k(b);
  // Padding item: its zero rows as part of one contiguous span (see zero_row_span).
  if (qblk * BM >= Lq && p.q_rows_contiguous(D)) {
    zero_row_span((uint16_t *)p.dq + (int64_t)b * p.sq_b, p.sq_t, qblk * BM, min(qblk * BM + BM, p.Tq), h,
                  p.H, threadIdx.x, 64 * NW);
    return;
  }

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, hi = lane >> 5;
  const int q0 = qblk * BM;
  const int qbw = q0 / 32 + 2 * w;  // the wave's two query blocks: qbw, qbw + 1
  const int nqb_valid = (Lq + 31) / 32, nkb_valid = (Lk + 31) / 32;

  const int64_t qoff = p.q_base(b, h);
  const int64_t koff = p.k_base(b, h);
  const uint16_t *Kb = (const uint16_t *)p.k + koff;
  uint16_t *dQb = (uint16_t *)p.dq + qoff;
  const uint16_t *ds_bh = p.ds + ((int64_t)b * p.H + h) * DsLayout::per_bh(p.ds_nqb, p.ds_nkb, CAUSAL) * TE;

  int nend = Lk;
  if (CAUSAL) nend = min(nend, min(q0 + BM, Lq));
  if (q0 >= Lq) nend = 0;
  const int ntiles = (nend + BN - 1) / BN;

  // Tile (query block qb, key block kb) was stored by the dK/dV pass.
  auto tile_ok = [&](int qb, int kb) SIGATTN_INLINE {
    return qb < nqb_valid && kb < nkb_valid && (!CAUSAL || kb <= qb);
  };

  TileOffsets<D> to;
  to.init(lane);
  DmaPlan<BN, D, NW> dma;
  dma.init(w, lane);
  const int kv_stride_bytes = (int)(p.sk_t * 2);

  // Copy of a dS tile: instruction i fills keys 16i .. 16i+15 (1 KB); lane
  // j lands at key 16i + j/4, slot j%4 = (g-pair c, half h) and fetches
  // piece c of the stored lane 32h + key (at 1024 c + 16 (32h + key)).
  uint32_t soff[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int key = 16 * i + lane / 4, s = lane % 4;
    soff[i] = (uint32_t)((s >> 1) * 1024 + 16 * ((s & 1) * 32 + key));
  }
  // dSᵀ operand read: lane (group g16, s = 4e + m) reads key 16ks + 4h + e
  // (+8 for the second half), queries 4M .. 4M+3 with M = 4(g16 & 1) + m.
  int boff;
  {
    const int g16 = lane >> 4, s = lane & 15, e = s >> 2, m = s & 3, hh = g16 >> 1;
    boff = 32 * (4 * hh + e) + 8 * (2 * (g16 & 1) + (m & 1)) + 4 * (m >> 1);
  }
  auto ld_ds = [&](const uint16_t *tile, int ks) SIGATTN_INLINE {
    typedef short s16x4 __attribute__((ext_vector_type(4)));
    const uint16_t *base = tile + 512 * ks + boff;
    const s16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4 *)base);
    const s16x4 c = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) s16x4 *)(base + 256));
    const u32x2 lo = __builtin_bit_cast(u32x2, a);
    const u32x2 hv = __builtin_bit_cast(u32x2, c);
    return (u32x4){lo.x, lo.y, hv.x, hv.y};
  };
  // LDS slot of the wave's tile (column block cb, key block kl of the stage).
  auto ds_slot = [&](int st, int cb, int kl) SIGATTN_INLINE {
    return &sS[st][((4 * w + 2 * cb) * KB + 2 * kl) * TE / 2];
  };

  auto issue = [&](int st, int u) SIGATTN_INLINE {
    dma.issue(sK[st], Kb, kv_stride_bytes, u * BN, Lk);
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
#pragma unroll
      for (int kl = 0; kl < KB; ++kl) {
        const int qb = qbw + cb, kb = KB * u + kl;
        // Tiles the dK/dV pass did not store are replaced by tile 0 of this
        // (batch, head) (in bounds; their products are skipped).
        const int64_t ti = tile_ok(qb, kb) ? DsLayout::tile(qb, kb, p.ds_nqb, CAUSAL) : 0;
        const uint16_t *src = ds_bh + ti * TE;
#pragma unroll
        for (int i = 0; i < 2; ++i) {
          uint16_t *dst = ds_slot(st, cb, kl) + 512 * i;
          const uint32_t m0 = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)dst);
          // dS is read once: non-temporal loads keep it from displacing the
          // K rows the other workgroups of this (batch, head) re-read.
          if constexpr (kDqDsNT)
            asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1 nt"
                         :
                         : "v"(soff[i]), "s"(src), "{m0}"(m0)
                         : "memory");
          else
            asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
                         :
                         : "v"(soff[i]), "s"(src), "{m0}"(m0)
                         : "memory");
        }
      }
    }
  };

  f32x16 acc[2][NDB];
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int d = 0; d < NDB; ++d) acc[c][d] = zero16();

  // Every MFMA runs on every stage: a tile the dK/dV pass did not store
  // enters as a zero operand (the K rows are finite, so it adds exactly 0).
  // Branching around the products instead makes the compiler copy all the
  // accumulators at every join.
  auto compute = [&](int st, int u) SIGATTN_INLINE {
#pragma unroll
    for (int kl = 0; kl < KB; ++kl) {
      const int kb = KB * u + kl;
      const bool ok0 = tile_ok(qbw, kb), ok1 = tile_ok(qbw + 1, kb);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int ks = 2 * kl + j;
        u32x4 b0 = ld_ds(ds_slot(st, 0, kl), j);
        u32x4 b1 = ld_ds(ds_slot(st, 1, kl), j);
        b0 = ok0 ? b0 : zero4();
        b1 = ok1 ? b1 : zero4();
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
          const u32x4 a = ld_tr<D>(sK[st], to, ks, db);
          acc[0][db] = Elem<T>::mfma(a, b0, acc[0][db]);
          acc[1][db] = Elem<T>::mfma(a, b1, acc[1][db]);
        }
      }
    }
  };

#pragma unroll
  for (int u = 0; u < PF; ++u)
    if (u < ntiles) issue(u, u);
  for (int u = 0; u < ntiles; ++u) {
    // Wait for this wave's copies of stage u (the later stages' copies may
    // stay in flight), then for every wave's.
    wait_vm_steps<NI, PF - 1>(min(ntiles - 1 - u, PF - 1));
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    // The stage the copy fills last held stage u-1, which every wave has
    // finished reading (they all passed the barrier above after computing it).
    if (u + PF < ntiles) issue((u + PF) % NST, u + PF);
    compute(u % NST, u);
  }

  const float scale = *p.scale;
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const int my_q = q0 + 64 * w + 32 * c + l32;
    if (my_q < p.q_rows_out(Lq)) {
      uint16_t *row = dQb + (int64_t)my_q * p.sq_t;
      const bool valid = my_q < Lq;
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int d0 = db * 32 + 8 * g + 4 * hi;
          u32x2 o;
          o.x = Elem<T>::pack(acc[c][db][4 * g] * scale, acc[c][db][4 * g + 1] * scale);
          o.y = Elem<T>::pack(acc[c][db][4 * g + 2] * scale, acc[c][db][4 * g + 3] * scale);
          if (!valid) o = (u32x2){0u, 0u};
          *(u32x2 *)(row + d0) = o;
        }
      }
    }
  }
}

template <int ROWBLK, typename Launch>
static void launch_rows(const KParams &kp, int rows, Launch &&launch) {
  KParams p = kp;
  p.nblk = (rows + ROWBLK - 1) / ROWBLK;
  launch(p, dim3((unsigned)(p.nblk * p.B * p.H)));
}

template <typename T, int D>
static void bwd_dq_t(const KParams &kp, bool causal, bool sm, hipStream_t st) {
  launch_rows<128>(kp, kp.Tq, [&](const KParams &p, dim3 grid) {
    // Range split (dense non-causal): rsplit workgroups per item.
    if (!causal && p.rsplit > 1) grid.x *= (unsigned)p.rsplit;
    grid.x += (unsigned)(p.ngap[0] + p.ngap[1]);
    if (causal) {
      if (sm) bwd_dq_kernel<T, D, true, true><<<grid, 256, 0, st>>>(p);
      else bwd_dq_kernel<T, D, true, false><<<grid, 256, 0, st>>>(p);
    } else {
      if (sm) bwd_dq_kernel<T, D, false, true><<<grid, 256, 0, st>>>(p);
      else bwd_dq_kernel<T, D, false, false><<<grid, 256, 0, st>>>(p);
    }
  });
}

template <typename T, int D, bool DSOUT>
static void bwd_dkdv_t(const KParams &kp, bool causal, bool sm, hipStream_t st) {
  launch_rows<128>(kp, kp.Tk, [&](const KParams &p, dim3 grid) {
    if constexpr (D == 128) {
      // Dense problems: two key blocks per workgroup (see the kernel), or
      // one when a non-causal grid of pairs would not fill the GPU.
      if (!(p.ragged() && p.B <= 64)) {
        const int64_t paired = (int64_t)((p.nblk + 1) / 2) * p.B * p.H;
        const bool one_block = !causal && paired < device_compute_units();
        grid = dim3((unsigned)(one_block ? (int64_t)p.nblk * p.B * p.H : paired));
      }
      if (causal) {
        if (sm) bwd_dkdv_pair_kernel<T, true, true, DSOUT><<<grid, 512, 0, st>>>(p);
        else bwd_dkdv_pair_kernel<T, true, false, DSOUT><<<grid, 512, 0, st>>>(p);
      } else {
        if (sm) bwd_dkdv_pair_kernel<T, false, true, DSOUT><<<grid, 512, 0, st>>>(p);
        else bwd_dkdv_pair_kernel<T, false, false, DSOUT><<<grid, 512, 0, st>>>(p);
      }
      return;
    }
    // Range split (dense non-causal recompute backward): rsplit workgroups per item.
    if (!causal && !DSOUT && p.rsplit > 1) grid.x *= (unsigned)p.rsplit;
    if (causal) {
      if (sm) bwd_dkdv_kernel<T, D, true, true, DSOUT><<<grid, 256, 0, st>>>(p);
      else bwd_dkdv_kernel<T, D, true, false, DSOUT><<<grid, 256, 0, st>>>(p);
    } else {
      if (sm) bwd_dkdv_kernel<T, D, false, true, DSOUT><<<grid, 256, 0, st>>>(p);
      else bwd_dkdv_kernel<T, D, false, false, DSOUT><<<grid, 256, 0, st>>>(p);
    }
  });
}

// Waves and ring stages of the D = 128 dQ-from-dS kernel.  Measured at
// B=4 L=4096 H=16 D=128 (causal / non-causal, one run): 8 waves with 4 stages
// (160 KB) 0.254 / 0.414 ms, with 3 stages 0.256 / 0.424 ms, with 2 stages
// 0.284 / 0.478 ms; 4 waves (two workgroups per CU) with 3 or 4 stages
// 0.265 / 0.44-0.45 ms.
#ifndef SIGATTN_DQDS_NW_128
#define SIGATTN_DQDS_NW_128 8
#endif
#ifndef SIGATTN_DQDS_NST_128
#define SIGATTN_DQDS_NST_128 4
#endif

// Grids of the D = 128 kernel with fewer 8-wave workgroups than the GPU has
// compute units (small problems, and long ones whose heads run in groups
// under the workspace cap) take 4-wave workgroups of 256 query rows with a
// 3-stage ring (72 KB, two per CU) instead, twice the workgroups on twice
// the CUs.
#ifndef SIGATTN_DQDS_SMALL_GRID
#define SIGATTN_DQDS_SMALL_GRID 1
#endif

template <typename T, int D>
static void bwd_dq_ds_t(const KParams &kp, bool causal, hipStream_t st) {
  constexpr int NW128 = SIGATTN_DQDS_NW_128, NST128 = SIGATTN_DQDS_NST_128;
  if constexpr (D == 128) {
    const int64_t wide = (int64_t)((kp.Tq + 64 * NW128 - 1) / (64 * NW128)) * kp.B * kp.H;
    if (SIGATTN_DQDS_SMALL_GRID && NW128 == 8 && wide < kp.ncu) {
      launch_rows<256>(kp, kp.Tq, [&](const KParams &p, dim3 grid) {
        grid.x += (unsigned)(p.ngap[0] + p.ngap[1]);
        if (causal) bwd_dq_ds_kernel<T, D, true, 4, 1, 3><<<grid, 256, 0, st>>>(p);
        else bwd_dq_ds_kernel<T, D, false, 4, 1, 3><<<grid, 256, 0, st>>>(p);
      });
      return;
    }
  }
  launch_rows<(D == 128 ? 64 * NW128 : 256)>(kp, kp.Tq, [&](const KParams &p, dim3 grid) {
    // D = 128: 8 waves (512 query rows: each K row read serves twice the dS
    // of a 4-wave workgroup; two waves per SIMD), one 32-key block per stage
    // in a 4-stage ring.  D = 64: 4 waves (the K rows of a 32-key stage do not
    // divide over 8 waves' copies), 6-stage ring.
    grid.x += (unsigned)(p.ngap[0] + p.ngap[1]);
    if constexpr (D == 128) {
      if (causal) bwd_dq_ds_kernel<T, D, true, NW128, 1, NST128><<<grid, 64 * NW128, 0, st>>>(p);
      else bwd_dq_ds_kernel<T, D, false, NW128, 1, NST128><<<grid, 64 * NW128, 0, st>>>(p);
    } else {
      if (causal) bwd_dq_ds_kernel<T, D, true, 4, 1, 6><<<grid, 256, 0, st>>>(p);
      else bwd_dq_ds_kernel<T, D, false, 4, 1, 6><<<grid, 256, 0, st>>>(p);
    }
  });
}

// dtype in {kF16, kBF16}, D in {32, 64, 128} (the two-pass backward's
// dQ-from-dS kernel: 64 and 128 only).
template <bool WITH32 = true, class F>
static void by_type(int dtype, int D, F &&f) {
  const auto d = [&](auto *t) {
    if (D == 128) f(t, std::integral_constant<int, 128>{});
    else if (!WITH32 || D == 64) f(t, std::integral_constant<int, 64>{});
    else if constexpr (WITH32) f(t, std::integral_constant<int, 32>{});
  };
  if (dtype == kBF16) d((__bf16 *)nullptr);
  else d((_Float16 *)nullptr);
}

int bwd_dq_rows_per_workgroup() { return 128; }
int bwd_dkdv_rows_per_workgroup() { return 128; }
// Resident workgroups per CU of the recompute kernels at D = 64 (dQ: 32 KB of
// LDS and at most 168 VGPRs; dK/dV: 64 KB and 128 + 128 registers); D = 32
// the same.
int bwd_dq_workgroups_per_cu(int D) { return D <= 64 ? 3 : 2; }
int bwd_dkdv_workgroups_per_cu(int D) { return D <= 64 ? 2 : 1; }

void launch_bwd_dq_mfma(const KParams &p, int dtype, int D, bool causal, bool sm, hipStream_t st) {
  by_type(dtype, D, [&](auto *t, auto d) {
    bwd_dq_t<std::remove_pointer_t<decltype(t)>, decltype(d)::value>(p, causal, sm, st);
  });
}

void launch_bwd_dkdv_mfma(const KParams &p, int dtype, int D, bool causal, bool sm, bool dsout,
                          hipStream_t st) {
  by_type(dtype, D, [&](auto *t, auto d) {
    using T = std::remove_pointer_t<decltype(t)>;
    if (dsout) bwd_dkdv_t<T, decltype(d)::value, true>(p, causal, sm, st);
    else bwd_dkdv_t<T, decltype(d)::value, false>(p, causal, sm, st);
  });
}

void launch_bwd_fused_mfma(const KParams &kp, int dtype, int D, bool causal, bool sm, hipStream_t st) {
  by_type(dtype, D, [&](auto *t, auto d) {
    using T = std::remove_pointer_t<decltype(t)>;
    constexpr int DD = decltype(d)::value;
    if constexpr (DD <= 64) {
      KParams pq = kp, pk = kp;
      pq.nblk = (kp.Tq + 127) / 128;
      pk.nblk = (kp.Tk + 127) / 128;
      pq.rsplit = pk.rsplit = 1;
      pq.ngap[0] = pq.ngap[1] = pk.ngap[0] = pk.ngap[1] = 0;  // dense problems only: no packed gap rows
      const int ndq = pq.nblk * kp.B * kp.H;
      const dim3 grid((unsigned)(ndq + pk.nblk * kp.B * kp.H));
      if (causal) {
        if (sm) bwd_fused_kernel<T, DD, true, true><<<grid, 256, 0, st>>>(pq, pk, ndq);
        else bwd_fused_kernel<T, DD, true, false><<<grid, 256, 0, st>>>(pq, pk, ndq);
      } else {
        if (sm) bwd_fused_kernel<T, DD, false, true><<<grid, 256, 0, st>>>(pq, pk, ndq);
        else bwd_fused_kernel<T, DD, false, false><<<grid, 256, 0, st>>>(pq, pk, ndq);
      }
    }
  });
}

void launch_bwd_dq_ds_mfma(const KParams &p, int dtype, int D, bool causal, hipStream_t st) {
  by_type<false>(dtype, D, [&](auto *t, auto d) {
    bwd_dq_ds_t<std::remove_pointer_t<decltype(t)>, decltype(d)::value>(p, causal, st);
  });
}

}  // namespace sigattn
