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
// Structure: one workgroup = 4 waves (one per SIMD) = 256 queries of one
// (batch, head); each wave owns 64 query rows (two 32-row MFMA column blocks),
// so every K or Vᵀ operand read from LDS feeds two MFMAs.
//   * K and V stream through a 3-stage ring of 64-key swizzled LDS tiles
//     filled by direct global->LDS copies two 32-key blocks ahead of use;
//   * keys are processed as a continuous sequence of 32-key blocks g with a
//     three-deep software pipeline: region r issues the Sᵀ(r) = K·Qᵀ MFMA
//     chains and the Oᵀ += Vᵀ·Pᵀ(r-2) MFMAs while the VALU computes
//     P(r-1) = sigmoid(Sᵀ(r-1)) and the LDS reads fetch the operands of
//     region r+1, so matrix, vector and LDS work overlap inside one wave;
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

template <typename T, int D, bool CAUSAL, bool SCOREMOD>
__global__ __launch_bounds__(256, 1) void fwd_mfma_kernel(const KParams p) {
  constexpr int BM = 256;      // queries per workgroup (64 per wave)
  constexpr int BN = 64;       // keys per LDS tile (two 32-key blocks)
  constexpr int NST = 3;       // LDS ring stages
  constexpr int NKS = D / 16;  // MFMA k-steps over the head dim
  constexpr int NDB = D / 32;  // 32-row blocks of Oᵀ

  __shared__ __attribute__((aligned(16))) uint16_t sK[NST][BN * D];
  __shared__ __attribute__((aligned(16))) uint16_t sV[NST][BN * D];
  __shared__ __attribute__((aligned(16))) float sC[SCOREMOD ? NST * BN : 4];

  const int BH = p.B * p.H;
  const int bh = blockIdx.x % BH;
  int qb = blockIdx.x / BH;
  if (CAUSAL) qb = p.nblk - 1 - qb;  // heaviest query blocks first
  const int b = bh / p.H, h = bh % p.H;

  const int Lq = clamp_len(p.seq_q, b, p.Tq);
  const int Lk = clamp_len(p.seq_k, b, p.Tk);

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, hi = lane >> 5;
  const int q0 = qb * BM;
  const int qw = q0 + w * 64;       // this wave's first query
  const int myq0 = qw + l32;        // this lane's query in column block 0 (block 1: +32)

  const uint16_t *Qb = (const uint16_t *)p.q + (int64_t)b * p.sq_b + (int64_t)h * p.sq_h;
  const uint16_t *Kb = (const uint16_t *)p.k + (int64_t)b * p.sk_b + (int64_t)h * p.sk_h;
  const uint16_t *Vb = (const uint16_t *)p.v + (int64_t)b * p.sk_b + (int64_t)h * p.sk_h;
  uint16_t *Ob = (uint16_t *)p.out + (int64_t)b * p.sq_b + (int64_t)h * p.sq_h;

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
  u32x4 qf[2][NKS];
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const int q = myq0 + 32 * c;
    const bool ok = q < Lq;
    const uint16_t *qrow = Qb + (int64_t)q * p.sq_t + 8 * hi;
#pragma unroll
    for (int s = 0; s < NKS; ++s) qf[c][s] = ok ? *(const u32x4 *)(qrow + 16 * s) : zero4();
  }
  // Consume the Q loads here, so the compiler's wait for them is not placed
  // at the head of the key loop, where it would also wait for the tile copies.
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int s = 0; s < NKS; ++s) asm volatile("" ::"v"(qf[c][s]));

  f32x16 acc[2][NDB];
#pragma unroll
  for (int c = 0; c < 2; ++c)
#pragma unroll
    for (int d = 0; d < NDB; ++d) acc[c][d] = zero16();

  TileOffsets<D> to;
  to.init(lane);
  DmaPlan<BN, D, 4> dma;
  dma.init(w, lane);
  const int kv_stride_bytes = (int)(p.sk_t * 2);

  float creg = 0.0f;
  auto load_c = [&](int n0) SIGATTN_INLINE {
    if (SCOREMOD && tid < BN) {
      const int key = n0 + tid;
      creg = key < Lk ? -(bias + p.score_mod[(int64_t)b * p.Tk + key]) * kLog2e : 0.0f;
    }
  };
  auto issue = [&](int st, int t) SIGATTN_INLINE {
    dma.issue(sK[st], Kb, kv_stride_bytes, t * BN, Lk);
    dma.issue(sV[st], Vb, kv_stride_bytes, t * BN, Lk);
  };

  // Operand registers: ka = K rows of the block whose Sᵀ chains run next,
  // va = Vᵀ operands of the block whose Oᵀ update runs next.  Each region
  // consumes them and refills them for the following region, so no MFMA
  // waits on an LDS read issued in its own region.
  u32x4 ka[NKS], va[2 * NDB];
  auto fetch_k = [&](int st, int kl) SIGATTN_INLINE {
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) ka[ks] = ld_row<D>(sK[st], to, kl, ks);
  };
  // Block g needs element masks when it crosses seq_lens_k or the diagonal of
  // this wave's first query.
  auto needs_mask = [&](int g) SIGATTN_INLINE {
    return (32 * g + 32 > Lk) || (CAUSAL && 32 * g + 31 > qw);
  };

  f32x16 sbuf[2][2];
  uint32_t pbuf[2][2][8];
  float ea[16 / (NKS + 2 * NDB)][2];  // exp2 terms of the next words (stage A output)

  // One region: 16 steps, each two MFMAs that share an A operand, the
  // refill of that operand for the next region, and the sigmoid of
  // 16 / (steps) packed P words of the previous block, so the VALU work runs
  // in the shadow of the matrix core and every operand is read from LDS a
  // full region before it is used.  Every region runs this same sequence;
  // blocks that need element masks are fixed up afterwards (mask_words).
  constexpr int NSTEP = NKS + 2 * NDB;
  constexpr int WPS = 16 / NSTEP;  // packed P words per step
  auto body = [&](auto u_tag) SIGATTN_INLINE {
    constexpr int U = decltype(u_tag)::value;
    constexpr int SL = U % 2, KLn = 32 * ((U + 1) % 2);
    constexpr int STK = ((U + 1) / 2) % 3, STV = ((U + 5) / 2) % 3;
    f32x16(&sc)[2] = sbuf[SL];
    const f32x16(&sp)[2] = sbuf[1 - SL];
    uint32_t(&pn)[2][8] = pbuf[1 - SL];
    const uint32_t(&pp)[2][8] = pbuf[SL];
    float c[16];
    if constexpr (SCOREMOD) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const float4 cv = *(const float4 *)&sC[STV * BN + KLn + 8 * g + 4 * hi];
        c[4 * g + 0] = cv.x; c[4 * g + 1] = cv.y; c[4 * g + 2] = cv.z; c[4 * g + 3] = cv.w;
      }
    } else {
#pragma unroll
      for (int i = 0; i < 16; ++i) c[i] = nbl;
    }
    // c terms of the next block's first WPS words (its exp stage runs in this
    // region's last step).
    float cn[2 * WPS];
    if constexpr (SCOREMOD) {
      constexpr int STN = (U / 2) % 3, KL = 32 * (U % 2);
#pragma unroll
      for (int i = 0; i < 2 * WPS; ++i) cn[i] = sC[STN * BN + KL + 8 * (i / 4) + 4 * hi + (i % 4)];
    } else {
#pragma unroll
      for (int i = 0; i < 2 * WPS; ++i) cn[i] = nbl;
    }
    sc[0] = zero16();
    sc[1] = zero16();
    // The sigmoid runs as a two-stage pipeline over packed words: step k
    // takes the exp2 of the words of step k+1 (stage A, into ea) and the
    // reciprocal and packing of the words of step k (stage B), so no
    // transcendental result is used by the next instruction.
    auto stage_a = [&](const f32x16 (&src)[2], const float *cc, int wd, float (&out)[2]) SIGATTN_INLINE {
      const int cb = wd / 8, e = wd % 8;
      out[0] = __builtin_amdgcn_exp2f(__builtin_fmaf(src[cb][2 * e], nsl, cc[0]));
      out[1] = __builtin_amdgcn_exp2f(__builtin_fmaf(src[cb][2 * e + 1], nsl, cc[1]));
    };
    auto words = [&](int step) SIGATTN_INLINE {
      float nx[WPS][2];
#pragma unroll
      for (int w2 = 0; w2 < WPS; ++w2) {
        if (step + 1 < NSTEP) {
          const int wd = (step + 1) * WPS + w2, e = wd % 8;
          stage_a(sp, &c[2 * e], wd, nx[w2]);
        } else {
          stage_a(sc, &cn[2 * w2], w2, nx[w2]);
        }
      }
#pragma unroll
      for (int w2 = 0; w2 < WPS; ++w2) {
        const int wd = step * WPS + w2, cb = wd / 8, e = wd % 8;
        const float a0 = __builtin_amdgcn_rcpf(1.0f + ea[w2][0]);
        const float a1 = __builtin_amdgcn_rcpf(1.0f + ea[w2][1]);
        pn[cb][e] = Elem<T>::pack(a0, a1);
        // Pins the word's computation to this step: without it the compiler
        // may sink the whole sigmoid below the region's MFMAs.
        asm volatile("" : "+v"(pn[cb][e]));
      }
#pragma unroll
      for (int w2 = 0; w2 < WPS; ++w2) { ea[w2][0] = nx[w2][0]; ea[w2][1] = nx[w2][1]; }
    };
#pragma unroll
    for (int step = 0; step < NSTEP; ++step) {
      if (step < NKS) {
        const int ks = step;
        sc[0] = Elem<T>::mfma(ka[ks], qf[0][ks], sc[0]);
        sc[1] = Elem<T>::mfma(ka[ks], qf[1][ks], sc[1]);
        ka[ks] = ld_row<D>(sK[STK], to, KLn, ks);
      } else {
        const int i = step - NKS, j = i / NDB, db = i % NDB;
        const u32x4 b0 = (u32x4){pp[0][4 * j], pp[0][4 * j + 1], pp[0][4 * j + 2], pp[0][4 * j + 3]};
        const u32x4 b1 = (u32x4){pp[1][4 * j], pp[1][4 * j + 1], pp[1][4 * j + 2], pp[1][4 * j + 3]};
        acc[0][db] = Elem<T>::mfma(va[i], b0, acc[0][db]);
        acc[1][db] = Elem<T>::mfma(va[i], b1, acc[1][db]);
        va[i] = ld_tr<D>(sV[STV], to, KLn / 16 + j, db);
      }
      words(step);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x402, 4 * WPS, 0);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      __builtin_amdgcn_sched_group_barrier(0x402, 6 * WPS, 0);
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // Zeroes the P entries of block r-1 (first key kbase) whose key lies before
  // 0 (pipeline fill), at or past seq_lens_k, or after the lane's query.
  // Works on the packed words, so garbage scores of such keys never matter.
  auto mask_words = [&](uint32_t (&pk)[2][8], int kbase) SIGATTN_INLINE {
    // Keeps this rare fix-up in its own branch: without the opaque copy of
    // kbase the compiler hoists the mask arithmetic into every region.
    asm volatile("" : "+s"(kbase));
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
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

  // Region r: MFMA: Sᵀ(r) from ka and Oᵀ += Vᵀ·Pᵀ(r-2) from va;
  //           VALU: P(r-1) = sigmoid(Sᵀ(r-1));
  //           LDS:  ka <- K rows of block r+1, va <- Vᵀ of block r-1.
  // Block g lives in tile g/2 (rows 32*(g%2)) in ring stage (g/2)%3.  Odd
  // regions r = 2t+1 first publish tile t+1 (wait for its copy, barrier) --
  // after which no wave reads tile t-1 again -- and then start the copy of
  // tile t+2 into tile t-1's stage, two regions ahead of its use.  U = r mod 6
  // is a compile-time constant, so every register slot and LDS stage is
  // static.  Blocks past the workgroup's keys (pipeline drain) read stale or
  // zeroed tiles and are masked to P = 0; Oᵀ only ever takes blocks 0..NB-1.
  auto region = [&](int r, auto u_tag) SIGATTN_INLINE {
    constexpr int U = decltype(u_tag)::value;
    if ((U % 2) == 1 && (r + 1) / 2 < ntiles) {
      const int t1 = (r + 1) / 2;
      wait_dma();
      if (SCOREMOD && tid < BN) sC[(t1 % 3) * BN + tid] = creg;
      __syncthreads();
      if (t1 + 1 < ntiles) {
        load_c((t1 + 1) * BN);
        issue((t1 + 1) % 3, t1 + 1);
      }
    }
    body(u_tag);
    if (r == 0 || needs_mask(r - 1)) mask_words(pbuf[1 - (U % 2)], 32 * (r - 1));
  };

  // Pipeline fill: Pᵀ(-2) = 0 and Vᵀ(-2) = 0 for region 0; stage 2 of V is
  // zeroed so region 1's Vᵀ(-1) (read before tile 2 arrives) is finite and
  // the masked Pᵀ(-1) = 0 adds nothing.
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    sbuf[x][0] = zero16();
    sbuf[x][1] = zero16();
#pragma unroll
    for (int e = 0; e < 8; ++e) { pbuf[x][0][e] = 0u; pbuf[x][1][e] = 0u; }
  }
#pragma unroll
  for (int i = 0; i < 2 * NDB; ++i) va[i] = zero4();
#pragma unroll
  for (int w2 = 0; w2 < WPS; ++w2) { ea[w2][0] = 0.0f; ea[w2][1] = 0.0f; }
#pragma unroll
  for (int i = tid; i < BN * D / 8; i += 256) *(u32x4 *)&sV[2][8 * i] = zero4();

  if (ntiles > 0) {
    load_c(0);
    issue(0, 0);
    wait_dma();
    if (SCOREMOD && tid < BN) sC[tid] = creg;
  }
  __syncthreads();
  if (ntiles > 1) {
    load_c(BN);
    issue(1, 1);
  }
  fetch_k(0, 0);
  for (int r0 = 0; r0 < NB + 2; r0 += 6) {
    region(r0 + 0, std::integral_constant<int, 0>{});
    if (r0 + 1 < NB + 2) region(r0 + 1, std::integral_constant<int, 1>{});
    if (r0 + 2 < NB + 2) region(r0 + 2, std::integral_constant<int, 2>{});
    if (r0 + 3 < NB + 2) region(r0 + 3, std::integral_constant<int, 3>{});
    if (r0 + 4 < NB + 2) region(r0 + 4, std::integral_constant<int, 4>{});
    if (r0 + 5 < NB + 2) region(r0 + 5, std::integral_constant<int, 5>{});
  }

  // Oᵀ accumulators -> O rows (4 consecutive d per 8-byte store).
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    const int q = myq0 + 32 * c;
    if (q < p.Tq) {
      uint16_t *orow = Ob + (int64_t)q * p.sq_t;
      const bool valid = q < Lq;
#pragma unroll
      for (int db = 0; db < NDB; ++db) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
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

template <typename T, int D>
static void launch_fwd_t(const KParams &kp, bool causal, bool scoremod, hipStream_t st) {
  constexpr int BM = 256;
  KParams p = kp;
  p.nblk = (p.Tq + BM - 1) / BM;
  const dim3 grid((unsigned)(p.nblk * p.B * p.H));
  const dim3 block(256);
  if (causal) {
    if (scoremod) fwd_mfma_kernel<T, D, true, true><<<grid, block, 0, st>>>(p);
    else fwd_mfma_kernel<T, D, true, false><<<grid, block, 0, st>>>(p);
  } else {
    if (scoremod) fwd_mfma_kernel<T, D, false, true><<<grid, block, 0, st>>>(p);
    else fwd_mfma_kernel<T, D, false, false><<<grid, block, 0, st>>>(p);
  }
}

void launch_fwd_mfma(const KParams &p, int dtype, int D, bool causal, bool scoremod,
                     hipStream_t st) {
  if (dtype == kBF16) {
    if (D == 128) launch_fwd_t<__bf16, 128>(p, causal, scoremod, st);
    else launch_fwd_t<__bf16, 64>(p, causal, scoremod, st);
  } else {
    if (D == 128) launch_fwd_t<_Float16, 128>(p, causal, scoremod, st);
    else launch_fwd_t<_Float16, 64>(p, causal, scoremod, st);
  }
}

}  // namespace sigattn
