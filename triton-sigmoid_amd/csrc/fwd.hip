// Forward kernel: O = sigmoid(Q·Kᵀ·scale + bias + score_mod) · V on gfx950 MFMA.
//
// Semantics follow the reference's _fwd_dense_kernel
// (src/triton_sigmoid/sigmoid_triton_dense.py:23-154) and _fwd_padded_kernel
// (src/triton_sigmoid/sigmoid_triton_padded.py:24-171):
//   S = Q·Kᵀ in fp32; S = S*scale + bias[b] (+ score_mod[b, key]);
//   causal keeps key <= query; P = sigmoid(S) in fp32; P is rounded to the
//   I/O dtype; O += P·V in fp32; O is stored in the I/O dtype; query rows at or
//   past seq_lens_q are zero; keys at or past seq_lens_k get P = 0.
//
// Structure: one workgroup = 256 queries of one (batch, head), split over its
// waves (NCB 32-row MFMA column blocks per wave; with NCB = 2 every K or Vᵀ
// operand read from LDS feeds two MFMAs).
//   * K and V stream through a 4-stage ring of 64-key swizzled LDS tiles
//     filled by direct global->LDS copies one tile ahead;
//   * keys are processed as a continuous sequence of 32-key blocks g with a
//     three-deep software pipeline: region r issues the Sᵀ(r) = K·Qᵀ MFMA
//     chains and the Oᵀ += Vᵀ·Pᵀ(r-2) MFMAs while the VALU computes
//     P(r-1) = sigmoid(Sᵀ(r-1)); every MFMA A operand is read from LDS
//     several MFMAs ahead through a rotating register queue;
//   * Pᵀ goes from the Sᵀ accumulators straight to the B operand of the next
//     product; Vᵀ comes from the row-major V tile via ds_read_b64_tr_b16;
//   * every region runs one straight-line sequence; element masks (causal
//     diagonal, seq_lens_k, pipeline fill) are applied afterwards to the
//     packed P words of the few blocks that need them;
//   * causal: tiles past the workgroup's last query are never loaded, and
//     the heaviest query blocks are launched first.
#include <type_traits>

#include "common.h"
#include "launch.h"

namespace sigattn {

// LDS ring stages of the D = 64 forward: three (48 KB) let three workgroups
// share a CU, four (64 KB) two.  D = 32 keeps four (32 KB).
#ifndef SIGATTN_FWD_D64_STAGES
#define SIGATTN_FWD_D64_STAGES 3
#endif

template <int D> constexpr int fwd_stages() { return D == 64 ? SIGATTN_FWD_D64_STAGES : 4; }

// Dense causal grids pair query blocks (j, nblk-1-j) in one workgroup, in
// the XCD-grouped order (every workgroup equal; K / V of a (batch, head) read
// by its workgroups while they sit in one L2).  Off: measured 2-3 % slower
// at B=4 L=4096 H=16 D=128 and 26 % at B=2 L=1024 H=8 D=64 (half the
// workgroups) than one block per workgroup, heaviest first.
#ifndef SIGATTN_FWD_CAUSAL_PAIRS
#define SIGATTN_FWD_CAUSAL_PAIRS 0
#endif
constexpr bool kFwdCausalPairs = SIGATTN_FWD_CAUSAL_PAIRS != 0;
// Dense causal order at D = 128 (one workgroup per CU): heaviest query
// blocks first within groups of this many (batch, head) pairs.  Measured at
// B=4 L=4096 H=16 (A/B in one run): HBM fetch per launch 452 MB with the
// plain order (every XCD cycling through 8 pairs), 269 MB with groups of 16
// (2 pairs per XCD at a time) at the same time (0.2818 / 0.2820 ms), 202 MB
// with groups of 8 but 11 % slower (the heaviest-first order then holds only
// within each group).  0 = the plain order.
#ifndef SIGATTN_FWD_BH_GROUP
#define SIGATTN_FWD_BH_GROUP 16
#endif
constexpr int kFwdBhGroup = SIGATTN_FWD_BH_GROUP;
// Resident workgroups per CU: D = 128 one (128 KB of LDS); D = 64 three (or
// two with four stages); D = 32 four (32 KB, at most 128 registers per wave).
template <int D> constexpr int fwd_occupancy() {
  return D == 64 ? (fwd_stages<D>() == 3 ? 3 : 2) : (D == 32 ? 4 : 1);
}

template <typename T, int D, int NWV, int NCB, bool CAUSAL, bool SCOREMOD>
__global__ __launch_bounds__(64 * NWV, fwd_occupancy<D>()) void fwd_mfma_kernel(const KParams p) {
  // NWV waves per workgroup (8: two per SIMD), NCB 32-query column blocks each.
  constexpr int QW = 32 * NCB;          // queries per wave
  constexpr int BM = NWV * QW;          // queries per workgroup
  constexpr int BN = 64;                // keys per LDS tile (two 32-key blocks)
  // LDS ring stages: D = 64 uses three (48 KB), so three workgroups share a CU.
  constexpr int NST = fwd_stages<D>();
  constexpr int NKS = D / 16;           // MFMA k-steps over the head dim
  constexpr int NDB = D / 32;           // 32-row blocks of Oᵀ
  constexpr int NSTEP = NKS + 2 * NDB;  // steps (NCB MFMAs sharing an A operand) per region
  // Operand read-ahead, in steps.  D = 128: a whole region (16) without
  // score_mod, 8 with it (16 would spill there); measured 2-3 % (8 vs 4) and
  // another 1-2.5 % (16 vs 8) at the headline shapes.  D = 64: 4 (three waves
  // per SIMD, 168 registers each); D = 32: 4, a whole region (2 with
  // score_mod, which spills at four waves per SIMD otherwise).
  constexpr int LA = D == 128 ? (SCOREMOD ? 8 : 16) : (D == 32 && SCOREMOD ? 2 : 4);
  constexpr int NWD = 8 * NCB;          // packed P words per block
  constexpr int BAR = NSTEP - LA;       // step of the tile barrier in odd regions
  static_assert(NSTEP % LA == 0, "region shape");

  __shared__ __attribute__((aligned(16))) uint16_t sK[NST][BN * D];
  __shared__ __attribute__((aligned(16))) uint16_t sV[NST][BN * D];
  __shared__ __attribute__((aligned(16))) float sC[SCOREMOD ? NST * BN : 4];

  const int wg = gap_prologue<2>(p, sK);  // packed layouts: leading gap-zeroing workgroups
  if (wg < 0) return;
  int b, h, qb0, nitems = 1;
  int ritem = 0, rchunk = 0;  // range split: the item and this workgroup's chunk of its keys
  if (!CAUSAL && p.rsplit > 1) {
    // Small dense grids: the rsplit workgroups of an item take adjacent ids.
    int bh;
    ritem = wg / p.rsplit, rchunk = wg % p.rsplit;
    dense_item(ritem, p.B * p.H, p.nblk, true, bh, qb0);
    b = bh / p.H, h = bh % p.H;
  } else if (p.ragged() && p.B <= 64) {
    const auto lq = [&](int i) SIGATTN_INLINE { return p.len_q(i); };
    const auto lk = [&](int i) SIGATTN_INLINE { return p.len_k(i); };
    const WorkItem it = CAUSAL ? WorkOrder::by_level(wg, p.B, p.H, lq, BM, p.nblk, true, p.ncu,
                                                     fwd_occupancy<D>())
                               : WorkOrder::by_stream(wg, p.B, p.H, lq, BM, p.nblk, lk);
    b = it.b, h = it.h, qb0 = it.blk;
  } else {
    const int BH = p.B * p.H;
    int bh;
    if (CAUSAL && kFwdCausalPairs) {
      // Query blocks nblk-1-j and j in sequence (grid = ceil(nblk/2) per
      // (batch, head)): under the causal mask the two together stream
      // nblk+1 key blocks' worth for every j, so all workgroups are equal and
      // the XCD-grouped order (K and V of a (batch, head) read by its
      // workgroups while they sit in one L2) costs no balance.
      int j;
      dense_item(wg, BH, (p.nblk + 1) / 2, true, bh, j);
      qb0 = p.nblk - 1 - j;
      nitems = j < qb0 ? 2 : 1;
    } else if (CAUSAL && D == 128 && kFwdBhGroup > 0 && BH % kFwdBhGroup == 0) {
      // Heaviest query blocks first within groups of kFwdBhGroup (batch,
      // head) pairs, group after group: each XCD (id % 8) holds the K / V
      // rows of kFwdBhGroup / 8 pairs at a time.
      const int g = wg / (kFwdBhGroup * p.nblk), r = wg % (kFwdBhGroup * p.nblk);
      bh = g * kFwdBhGroup + r % kFwdBhGroup;
      qb0 = p.nblk - 1 - r / kFwdBhGroup;
    } else {
      dense_item(wg, BH, p.nblk, !CAUSAL, bh, qb0);
      if (CAUSAL) qb0 = p.nblk - 1 - qb0;  // heaviest query blocks first
    }
    b = bh / p.H, h = bh % p.H;
  }

#pragma clang loop unroll(disable)
  for (int item = 0; item < nitems; ++item) {
    const int qb = item == 0 ? qb0 : p.nblk - 1 - qb0;
    // The previous item's last LDS reads precede this item's tile fills.
    if (item > 0) __syncthreads();
    const int Lq = p.len_q(b);
    // Keys of this workgroup: under the range split, its chunk of the item's
    // key tiles, indexed from the chunk's first key.
    int key0 = 0, Lk = p.len_k(b);
    if (!CAUSAL && p.rsplit > 1) {
      const int ntk = (Lk + BN - 1) / BN;
      key0 = split_tile(rchunk, p.rsplit, ntk) * BN;
      Lk = min(Lk, split_tile(rchunk + 1, p.rsplit, ntk) * BN) - key0;
    }
    // Padding item (the row block lies wholly past seq_lens_q): its zero rows
    // as part of one contiguous span over all heads when the layout allows.
    const bool half = p.half_head(D);  // head_dim 16 in this D = 32 kernel
    if (qb * BM >= Lq && nitems == 1 && p.q_rows_contiguous(half ? 16 : D)) {
      zero_row_span((uint16_t *)p.out + (int64_t)b * p.sq_b, p.sq_t, qb * BM, min(qb * BM + BM, p.Tq), h, p.H,
                    threadIdx.x, 64 * NWV);
      return;
    }

    const int tid = threadIdx.x, lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31, hi = lane >> 5;
    const int q0 = qb * BM;
    // Query slot of the wave.  With eight waves, waves w and w+4 share a SIMD;
    // giving them complementary slots (w and 7-w) evens out the per-SIMD work of
    // causal diagonal workgroups once waves stop at their own last key block.
    const int slot = (NWV == 8 && w >= 4) ? 11 - w : w;
    const int qw = q0 + slot * QW;    // this wave's first query
    const int myq0 = qw + l32;        // this lane's query in column block 0 (block c: +32c)

    const int64_t qoff = p.q_base(b, h), koff = p.k_base(b, h) + (int64_t)key0 * p.sk_t;
    const uint16_t *Qb = (const uint16_t *)p.q + qoff;
    const uint16_t *Kb = (const uint16_t *)p.k + koff;
    const uint16_t *Vb = (const uint16_t *)p.v + koff;
    uint16_t *Ob = (uint16_t *)p.out + qoff;

    int nend = Lk;
    if (CAUSAL) nend = min(nend, min(q0 + BM, Lq));
    if (q0 >= Lq) nend = 0;
    const int ntiles = (nend + BN - 1) / BN;
    const int NB = 2 * ntiles;  // 32-key blocks of the workgroup

    const float scale = *p.scale;
    const float bias = p.bias[b];
    const float nsl = -scale * kLog2e;
    const float nbl = -bias * kLog2e;

    // This wave's query rows as B operands (k = d = 16s + 8h + j).
    u32x4 qf[NCB][NKS];
  #pragma unroll
    for (int c = 0; c < NCB; ++c) {
      const int q = myq0 + 32 * c;
      const bool ok = q < Lq;
      const uint16_t *qrow = Qb + (int64_t)q * p.sq_t + 8 * hi;
  #pragma unroll
      for (int s = 0; s < NKS; ++s)
        qf[c][s] = ok && !(half && s > 0) ? *(const u32x4 *)(qrow + 16 * s) : zero4();
    }
    // Consume the Q loads here, so the compiler's wait for them is not placed
    // at the head of the key loop, where it would also wait for the tile copies.
  #pragma unroll
    for (int c = 0; c < NCB; ++c)
  #pragma unroll
      for (int s = 0; s < NKS; ++s) asm volatile("" ::"v"(qf[c][s]));

    f32x16 acc[NCB][NDB];
  #pragma unroll
    for (int c = 0; c < NCB; ++c)
  #pragma unroll
      for (int d = 0; d < NDB; ++d) acc[c][d] = zero16();

    TileOffsets<D> to;
    to.init(lane);
    DmaPlan<BN, D, NWV> dma;
    dma.init(w, lane, half);
    const int kv_stride_bytes = (int)(p.sk_t * 2);

    float creg = 0.0f;
    auto load_c = [&](int n0) SIGATTN_INLINE {
      if (SCOREMOD && tid < BN) {
        const int key = n0 + tid;
        creg = key < Lk ? -(bias + p.score_mod[p.mod_base(b) + key0 + key]) * kLog2e : 0.0f;
      }
    };
    auto issue = [&](int st, int t) SIGATTN_INLINE {
      load_c(t * BN);
      dma.issue(sK[st], Kb, kv_stride_bytes, t * BN, Lk);
      dma.issue(sV[st], Vb, kv_stride_bytes, t * BN, Lk);
    };

    // A operand of step o of the region whose S block sits at tile rows kl of
    // stage stc and whose Oᵀ block sits at the same rows of stage stv: steps
    // 0..NKS-1 are K rows (k-step o), the rest Vᵀ operands (16-key step j,
    // 32-row block db).
    auto read_op = [&](int o, int stc, int stv, int kl) SIGATTN_INLINE {
      if (o < NKS) return ld_row<D>(sK[stc], to, kl, o);
      const int i = o - NKS, j = i / NDB, db = i % NDB;
      return ld_tr<D>(sV[stv], to, kl / 16 + j, db);
    };
    // Block g needs element masks when it crosses seq_lens_k or the diagonal of
    // this wave's first query.
    auto needs_mask = [&](int g) SIGATTN_INLINE {
      return (32 * g + 32 > Lk) || (CAUSAL && 32 * g + 31 > qw);
    };
    // Zeroes the P entries of block g whose key lies before 0 (pipeline fill),
    // at or past seq_lens_k, or after the lane's query.  Works on the packed
    // words, so garbage scores of such keys never matter.
    auto mask_words = [&](uint32_t (&pk)[NCB][8], int g) SIGATTN_INLINE {
      int kbase = 32 * g;
      asm volatile("" : "+s"(kbase));  // keeps this rare fix-up in its own branch
  #pragma unroll
      for (int cb = 0; cb < NCB; ++cb) {
        const unsigned lim = CAUSAL ? (unsigned)min(Lk, myq0 + 32 * cb + 1) : (unsigned)Lk;
  #pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int i = 2 * e;
          const unsigned k0 = (unsigned)(kbase + 8 * (i / 4) + 4 * hi + (i % 4));
          const uint32_t m = (k0 < lim ? 0x0000ffffu : 0u) | (k0 + 1u < lim ? 0xffff0000u : 0u);
          pk[cb][e] &= m;
        }
      }
    };

    f32x16 sbuf[2][NCB];        // Sᵀ accumulators, by block parity
    uint32_t pbuf[2][NCB][8];   // packed P words, by block parity
    u32x4 opq[LA];              // A operands of the next LA steps (slot = step % LA)
    float ea[2];                // exp2 terms of the next word (sigmoid stage A)

    // Region r (U = r mod 8, so every slot and ring stage is static):
    //   MFMA: Sᵀ(r) = K·Qᵀ and Oᵀ += Vᵀ·Pᵀ(r-2), one step = NCB MFMAs (one per
    //         column block) sharing an A operand read LA steps earlier;
    //   VALU: P(r-1) = sigmoid(Sᵀ(r-1)) as a two-stage pipeline over packed
    //         words (exp2 of the next word, then reciprocal and packing);
    //   LDS:  the operand LA steps ahead (wrapping into region r+1).
    // Block g lives in tile g/2 (rows 32*(g%2)) in ring stage (g/2)%4.  In odd
    // regions r = 2u-1, step BAR publishes tile u (its first read, the K rows of
    // block r+1, comes next) and starts the copy of tile u+1 into the stage of
    // tile u+1-NST.  With four stages that tile's last reads were issued two
    // regions earlier, so the barrier needs no wait for this wave's own LDS
    // reads; with three (D = 64) they were issued in this region, and every
    // wave waits for them before the barrier.
    auto region = [&](int r, auto u_tag) SIGATTN_INLINE {
      constexpr int U = decltype(u_tag)::value;
      constexpr int SL = U % 2;                    // parity of blocks r and r-2
      constexpr int KL = 32 * (U % 2), KLn = 32 * ((U + 1) % 2);
      constexpr int STC = (U / 2) % NST;           // stage of block r
      constexpr int STV = ((U + 2 * NST - 2) / 2) % NST;  // stage of block r-2
      constexpr int STCn = ((U + 1) / 2) % NST;    // stage of block r+1
      constexpr int STVn = ((U + 2 * NST - 1) / 2) % NST;  // stage of block r-1
      f32x16(&sc)[NCB] = sbuf[SL];
      const f32x16(&sp)[NCB] = sbuf[1 - SL];
      uint32_t(&pn)[NCB][8] = pbuf[1 - SL];
      const uint32_t(&pp)[NCB][8] = pbuf[SL];
      float c[16];   // exp2 offsets of block r-1 (per key row)
      float cn[2];   // ... of block r's first word
      if constexpr (SCOREMOD) {
  #pragma unroll
        for (int g = 0; g < 4; ++g) {
          const float4 cv = *(const float4 *)&sC[STVn * BN + KLn + 8 * g + 4 * hi];
          c[4 * g + 0] = cv.x; c[4 * g + 1] = cv.y; c[4 * g + 2] = cv.z; c[4 * g + 3] = cv.w;
        }
  #pragma unroll
        for (int i = 0; i < 2; ++i) cn[i] = sC[STC * BN + KL + 4 * hi + i];
      } else {
  #pragma unroll
        for (int i = 0; i < 16; ++i) c[i] = nbl;
        cn[0] = cn[1] = nbl;
      }
  #pragma unroll
      for (int step = 0; step < NSTEP; ++step) {
        if ((U % 2) == 1 && step == BAR) {
          const int u = (r + 1) / 2;
          if (u < ntiles) {
            wait_dma();
            if (SCOREMOD && tid < BN) sC[(u % NST) * BN + tid] = creg;
            // With three stages the copy below refills the stage this region's
            // Vᵀ operands came from: every wave's reads of it complete first.
            if constexpr (NST == 3) asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            asm volatile("" ::: "memory");
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            if (u + 1 < ntiles) issue((u + 1) % NST, u + 1);
          }
        }
        // One wait for this step's operand.
        asm volatile("" ::"v"(opq[step % LA]));
        const u32x4 a = opq[step % LA];
        if (step < NKS) {
  #pragma unroll
          for (int c2 = 0; c2 < NCB; ++c2) sc[c2] = Elem<T>::mfma(a, qf[c2][step], step == 0 ? zero16() : sc[c2]);
        } else {
          const int i = step - NKS, j = i / NDB, db = i % NDB;
  #pragma unroll
          for (int c2 = 0; c2 < NCB; ++c2) {
            const u32x4 bp = (u32x4){pp[c2][4 * j], pp[c2][4 * j + 1], pp[c2][4 * j + 2], pp[c2][4 * j + 3]};
            acc[c2][db] = Elem<T>::mfma(a, bp, acc[c2][db]);
          }
        }
        if (step + LA < NSTEP) opq[step % LA] = read_op(step + LA, STC, STV, KL);
        else opq[step % LA] = read_op(step + LA - NSTEP, STCn, STVn, KLn);
        // Sigmoid words of this step: stage B (reciprocal, packing) of word wd
        // from ea, then stage A (exp2) of the next word into ea -- in the last
        // word, of block r's first word (its Sᵀ chains are complete by then).
  #pragma unroll
        for (int wd = step * NWD / NSTEP; wd < (step + 1) * NWD / NSTEP; ++wd) {
          {
            const int cb = wd / 8, e = wd % 8;
            const float a0 = __builtin_amdgcn_rcpf(1.0f + ea[0]);
            const float a1 = __builtin_amdgcn_rcpf(1.0f + ea[1]);
            pn[cb][e] = Elem<T>::pack(a0, a1);
            asm volatile("" : "+v"(pn[cb][e]));
          }
          if (wd + 1 < NWD) {
            const int cb = (wd + 1) / 8, e = (wd + 1) % 8;
            ea[0] = __builtin_amdgcn_exp2f(__builtin_fmaf(sp[cb][2 * e], nsl, c[2 * e]));
            ea[1] = __builtin_amdgcn_exp2f(__builtin_fmaf(sp[cb][2 * e + 1], nsl, c[2 * e + 1]));
          } else {
            ea[0] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[0][0], nsl, cn[0]));
            ea[1] = __builtin_amdgcn_exp2f(__builtin_fmaf(sc[0][1], nsl, cn[1]));
          }
        }
  #pragma unroll
        for (int c2 = 0; c2 < NCB; ++c2) {
          __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
          __builtin_amdgcn_sched_group_barrier(0x402, 5 * NWD / NSTEP / NCB + 1, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      if (r == 0 || needs_mask(r - 1)) mask_words(pn, r - 1);
    };

    // Pipeline fill: Pᵀ(-2) = Pᵀ(-1) = 0 (the latter through its mask).  The
    // Vᵀ operands of blocks -2 and -1 come from ring stage NST-1, zeroed here
    // (tile NST-1 is copied into it from the barrier of region 2·NST-5 on,
    // after every read of blocks -2 and -1), so 0 * operand stays 0.
  #pragma unroll
    for (int x = 0; x < 2; ++x) {
  #pragma unroll
      for (int c2 = 0; c2 < NCB; ++c2) {
        sbuf[x][c2] = zero16();
  #pragma unroll
        for (int e = 0; e < 8; ++e) pbuf[x][c2][e] = 0u;
      }
    }
    ea[0] = ea[1] = 0.0f;
    for (int i = tid; i < BN * D / 8; i += 64 * NWV) *(u32x4 *)&sV[NST - 1][8 * i] = zero4();

    if (ntiles > 0) {
      issue(0, 0);
      wait_dma();
      if (SCOREMOD && tid < BN) sC[tid] = creg;
    }
    __syncthreads();
    if (ntiles > 1) issue(1, 1);
  #pragma unroll
    for (int o = 0; o < LA; ++o) opq[o] = read_op(o, 0, NST - 1, 0);

    // This wave computes only up to its own last visible key block (causal) and
    // not at all past seq_lens_q; afterwards it only takes part in the tile
    // barriers and copies, leaving its SIMD to the other wave there.
    int NBw = NB;
    if (CAUSAL) NBw = min(NBw, (qw + QW - 1) / 32 + 1);
    if (qw >= Lq) NBw = 0;
    const int RW = NBw > 0 ? NBw + 2 : 0;
    // One pass of the loop covers 2·NST regions (NST tiles), so region r0 + U
    // starts tile r0/2 + U/2 with r0/2 a multiple of NST: every stage index in
    // region() is a compile-time function of U.
    for (int r0 = 0; r0 < RW; r0 += 2 * NST) {
      Unroll<0, 2 * NST>::run([&](auto u) SIGATTN_INLINE {
        if (r0 + decltype(u)::value < RW) region(r0 + decltype(u)::value, u);
      });
    }
    // The rest of the workgroup's regions: the same barriers and copies.
    for (int r = RW | 1; r < NB + 2; r += 2) {
      const int u = (r + 1) / 2;
      if (u < ntiles) {
        wait_dma();
        if (SCOREMOD && tid < BN) sC[(u % NST) * BN + tid] = creg;
        if constexpr (NST == 3) asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        if (u + 1 < ntiles) issue((u + 1) % NST, u + 1);
      }
    }

    if (!CAUSAL && p.rsplit > 1 &&
        !split_combine<NCB * NDB, NWV>([&](int i) SIGATTN_INLINE -> f32x16 & { return acc[i / NDB][i % NDB]; },
                                       p.rs_part + (int64_t)ritem * p.rsplit * (BM * D), p.rs_cnt + ritem,
                                       rchunk, p.rsplit, w, lane))
      return;

    // Oᵀ accumulators -> O rows (4 consecutive d per 8-byte store).
  #pragma unroll
    for (int c = 0; c < NCB; ++c) {
      const int q = myq0 + 32 * c;
      if (q < p.q_rows_out(Lq)) {
        uint16_t *orow = Ob + (int64_t)q * p.sq_t;
        const bool valid = q < Lq;
  #pragma unroll
        for (int db = 0; db < NDB; ++db) {
  #pragma unroll
          for (int g = 0; g < 4; ++g) {
            if (half && g >= 2) break;  // columns 16..31: not in the tensor
            const int d0 = db * 32 + 8 * g + 4 * hi;
            u32x2 o;
            o.x = Elem<T>::pack(acc[c][db][4 * g + 0], acc[c][db][4 * g + 1]);
            o.y = Elem<T>::pack(acc[c][db][4 * g + 2], acc[c][db][4 * g + 3]);
            if (!valid) o = (u32x2){0u, 0u};
            *(u32x2 *)(orow + d0) = o;
          }
        }
      }
    }
  }
}

// Query column blocks per wave: 1 = eight waves of 32 queries (two per SIMD,
// so each SIMD interleaves two waves' VALU and LDS work); 2 = four waves of
// 64 queries (every K / Vᵀ operand read feeds two MFMAs).  Measured at the
// headline shape: 1 is 2-3% faster.
#ifndef SIGATTN_FWD_NCB
#define SIGATTN_FWD_NCB 1
#endif

template <typename T, int D, int NWV>
static void launch_fwd_w(const KParams &kp, bool causal, bool scoremod, hipStream_t st) {
  constexpr int NCB = SIGATTN_FWD_NCB, BM = NWV * 32 * NCB;
  KParams p = kp;
  p.nblk = (p.Tq + BM - 1) / BM;
  // Dense causal problems (the kernel's order when not ragged with B <= 64):
  // two query blocks per workgroup.
  const bool pairs = causal && kFwdCausalPairs && !(p.ragged() && p.B <= 64);
  if (causal || p.rsplit < 1) p.rsplit = 1;
  const dim3 grid((unsigned)((pairs ? (p.nblk + 1) / 2 : p.nblk) * p.B * p.H * p.rsplit + p.ngap[0] + p.ngap[1]));
  const dim3 block(64 * NWV);
  if (causal) {
    if (scoremod) fwd_mfma_kernel<T, D, NWV, NCB, true, true><<<grid, block, 0, st>>>(p);
    else fwd_mfma_kernel<T, D, NWV, NCB, true, false><<<grid, block, 0, st>>>(p);
  } else {
    if (scoremod) fwd_mfma_kernel<T, D, NWV, NCB, false, true><<<grid, block, 0, st>>>(p);
    else fwd_mfma_kernel<T, D, NWV, NCB, false, false><<<grid, block, 0, st>>>(p);
  }
}

// D = 128: one workgroup of eight waves per CU (128 KB of LDS).  D = 64: a
// 3-stage ring of 48 KB, so three workgroups of four waves share a CU (three
// waves per SIMD, at most 168 VGPRs each) in small work units, which balance
// better on small or ragged (padded) batches.  Measured against two
// workgroups per CU with a 4-stage ring: 10-20 % faster dense (c4, c5 shapes)
// and 5-13 % padded.
template <typename T, int D>
static void launch_fwd_t(const KParams &kp, bool causal, bool scoremod, hipStream_t st) {
  launch_fwd_w<T, D, (D <= 64 ? 4 : 8) / SIGATTN_FWD_NCB>(kp, causal, scoremod, st);
}

int fwd_rows_per_workgroup(int D) { return (D <= 64 ? 4 : 8) * 32; }
int fwd_workgroups_per_cu(int D) {
  return D == 32 ? fwd_occupancy<32>() : (D == 64 ? fwd_occupancy<64>() : fwd_occupancy<128>());
}

__global__ __launch_bounds__(256) void rs_clear_kernel(int *a, int na, int *b, int nb) {
  for (int i = blockIdx.x * 256 + threadIdx.x; i < na + nb; i += gridDim.x * 256) {
    if (i < na) a[i] = 0;
    else b[i - na] = 0;
  }
}
void launch_rs_clear(int *a, int na, int *b, int nb, hipStream_t st) {
  const int n = na + nb;
  if (n > 0) rs_clear_kernel<<<(unsigned)min((n + 255) / 256, 64), 256, 0, st>>>(a, na, b, nb);
}

void launch_fwd_mfma(const KParams &p, int dtype, int D, bool causal, bool scoremod,
                     hipStream_t st) {
  if (dtype == kBF16) {
    if (D == 128) launch_fwd_t<__bf16, 128>(p, causal, scoremod, st);
    else if (D == 64) launch_fwd_t<__bf16, 64>(p, causal, scoremod, st);
    else launch_fwd_t<__bf16, 32>(p, causal, scoremod, st);
  } else {
    if (D == 128) launch_fwd_t<_Float16, 128>(p, causal, scoremod, st);
    else if (D == 64) launch_fwd_t<_Float16, 64>(p, causal, scoremod, st);
    else launch_fwd_t<_Float16, 32>(p, causal, scoremod, st);
  }
}

}  // namespace sigattn
