// fp32 inputs on the matrix cores.  gfx950's v_mfma_f32_32x32x2_f32 takes fp32
// operands and accumulates in fp32 -- the precision of the reference's fp32
// dots (tl.dot with allow_tf32=False, sigmoid_triton_dense.py:123,149,272,
// 289,299,426,443,446,456; sigmoid_triton_padded.py:138,166,297,321,331,461,
// 485,488,498), which run on the scalar FMA units there.  Same semantics as
// the 16-bit MFMA kernels and the portable ones: masks are causal (key <=
// query, top-left) and seq_lens bounds, padded rows are written as zeros,
// packed layouts write each sequence's rows only.
//
// The instruction: C[i][j] += A[i][0] B[0][j] + A[i][1] B[1][j]; lane l gives
// A[l % 32][l / 32] and B[l / 32][l % 32], one float each, and holds
// C[8g + 4(l / 32) + r][l % 32] in accumulator element 4g + r.  At 64 of the
// SIMD's cycles per instruction, a 32x32 block costs D instructions per
// product pair against a few hundred cycles of sigmoid arithmetic, so these
// kernels are plain: four waves of 32 stationary rows, streamed rows in a
// ring of 32-row tiles copied straight into LDS, one barrier per tile.  Where
// two or more waves share a SIMD, one wave's sigmoid arithmetic runs under
// another's MFMAs; the backward kernels also spread it over their dP chains
// (head_product_with), and at D = 128, one wave per SIMD, the dQ kernel runs
// tile t's arithmetic under tile t+1's chains.
//
// Products over the head dim (S, dP) reduce d = s (lanes 0-31) and
// d = D/2 + s (lanes 32-63) in step s, so four consecutive steps take one
// 16-byte piece of the lane's row.  Products over the streamed rows (O, dQ,
// dK, dV) reduce rows 8g + r (lanes 0-31) and 8g + 4 + r (lanes 32-63) in
// step (g, r) -- the rows whose S (or dS) value the lane holds in
// accumulator element 4g + r -- so P and dS feed them as B operands where
// they were computed, in fp32, with no data movement.
#include "common.h"
#include "launch.h"

namespace sigattn {
namespace {

constexpr int FB = 32;        // streamed rows per LDS tile
constexpr int FW = 4;         // waves per workgroup
constexpr int FBM = FW * 32;  // stationary rows per workgroup

__device__ __forceinline__ f32x16 mma(float a, float b, const f32x16 &c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

// The lane's stationary row, head-dim halves by lane half: v[s] = row[hi * D/2 + s]
// (zeros when !ok; for head_dim 16 in the D = 32 kernels the upper half is zero).
template <int D>
__device__ __forceinline__ void load_half_row(float (&v)[D / 2], const float *row, int hi, bool ok) {
#pragma unroll
  for (int t = 0; t < D / 8; ++t) {
    const f32x4 x = ok ? *(const f32x4 *)(row + hi * (D / 2) + 4 * t) : f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    v[4 * t] = x.x, v[4 * t + 1] = x.y, v[4 * t + 2] = x.z, v[4 * t + 3] = x.w;
  }
}

// acc += (rows l % 32 of tile t) · v over the head dim (S or dP).
template <int D>
__device__ __forceinline__ void head_product(f32x16 &acc, const float *t, const float (&v)[D / 2], int l32,
                                             int hi) {
#pragma unroll
  for (int c = 0; c < D / 8; ++c) {
    const f32x4 a = *(const f32x4 *)(t + F32Tile<D>::piece(l32, hi * (D / 8) + c));
    acc = mma(a.x, v[4 * c], acc);
    acc = mma(a.y, v[4 * c + 1], acc);
    acc = mma(a.z, v[4 * c + 2], acc);
    acc = mma(a.w, v[4 * c + 3], acc);
  }
}

// accᵀ[d][j] += sum over the tile's rows i of t[i][d] · w[i][j], where the
// lane holds w[8g + 4hi + r][l % 32] in element 4g + r (O, dQ, dK, dV).
template <int D>
__device__ __forceinline__ void row_product(f32x16 (&acc)[D / 32], const float *t, const float (&w)[16],
                                            const F32RowReads<D> &rr) {
#pragma unroll
  for (int g = 0; g < 4; ++g)
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int db = 0; db < D / 32; ++db) acc[db] = mma(t[rr.at(g, r, db)], w[4 * g + r], acc[db]);
}

// Stores row `row` of an output from accᵀ (columns 32db + 8g + 4hi + r in
// element 4g + r of block db), times `mul`; zeros when !valid.
template <int D>
__device__ __forceinline__ void store_row(float *row, const f32x16 (&acc)[D / 32], float mul, bool valid, int hi,
                                          bool half) {
#pragma unroll
  for (int db = 0; db < D / 32; ++db)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      if (half && g >= 2) break;  // columns 16..31: not in the tensor
      f32x4 o = {acc[db][4 * g] * mul, acc[db][4 * g + 1] * mul, acc[db][4 * g + 2] * mul,
                 acc[db][4 * g + 3] * mul};
      if (!valid) o = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      *(f32x4 *)(row + 32 * db + 8 * g + 4 * hi) = o;
    }
}

// Resident waves per SIMD (four-wave workgroups): registers bound them; the
// LDS ring (stages x 2 tiles x 32 rows x D floats: 64 KB at D = 128 with two
// stages, 96 KB with three) fits.
template <int D> constexpr int fwd_f32_occupancy() { return D == 128 ? 2 : (D == 64 ? 3 : 4); }
template <int D> constexpr int bwd_f32_occupancy() { return D == 128 ? 1 : (D == 64 ? 2 : 3); }

// Ring stages of the dQ kernel: three where one wave holds a SIMD (D = 128),
// so that tile t+1's chains run while tile t's sigmoid arithmetic issues,
// else two.
#ifndef SIGATTN_F32_DQ_PIPE
#define SIGATTN_F32_DQ_PIPE 1
#endif
template <int D> constexpr int dq_f32_stages() {
  return SIGATTN_F32_DQ_PIPE && bwd_f32_occupancy<D>() == 1 ? 3 : 2;
}

// head_product with elem(i), i = 0..15 (a tile's per-element sigmoid
// arithmetic), spread over the chain's pieces: a scheduling fence after each
// piece keeps that VALU work between the MFMAs -- left to itself the compiler
// places it after the last one, where a wave alone on its SIMD leaves the
// matrix core idle.  Piece c+1's operand is read before piece c's MFMAs.
template <int D, class Elem>
__device__ __forceinline__ void head_product_with(f32x16 &acc, const float *t, const float (&v)[D / 2], int l32,
                                                  int hi, Elem &&elem) {
  constexpr int NP = D / 8, EPP = 16 / NP;
  static_assert(NP * EPP == 16, "elements per piece");
  f32x4 a = *(const f32x4 *)(t + F32Tile<D>::piece(l32, hi * NP));
#pragma unroll
  for (int c = 0; c < NP; ++c) {
    f32x4 an = a;
    if (c + 1 < NP) an = *(const f32x4 *)(t + F32Tile<D>::piece(l32, hi * NP + c + 1));
    acc = mma(a.x, v[4 * c], acc);
    acc = mma(a.y, v[4 * c + 1], acc);
    acc = mma(a.z, v[4 * c + 2], acc);
    acc = mma(a.w, v[4 * c + 3], acc);
#pragma unroll
    for (int j = 0; j < EPP; ++j) elem(c * EPP + j);
    __builtin_amdgcn_sched_barrier(0);
    a = an;
  }
}

// Forward: O = sigmoid(Q·Kᵀ·scale + bias [+ score_mod]) · V, one workgroup
// per (batch, head, 128-query block); keys streamed.
template <int D, bool CAUSAL, bool SCOREMOD>
__global__ __launch_bounds__(64 * FW, fwd_f32_occupancy<D>()) void fwd_f32_kernel(const KParams p) {
  constexpr int NDB = D / 32;
  __shared__ __attribute__((aligned(16))) float sK[2][FB * D];
  __shared__ __attribute__((aligned(16))) float sV[2][FB * D];
  __shared__ float sC[SCOREMOD ? 2 : 1][FB];

  const int wg = gap_prologue<4>(p, sK);  // packed layouts: leading gap-zeroing workgroups
  if (wg < 0) return;
  const int BH = p.B * p.H;
  const int bh = wg % BH;
  int qb = wg / BH;
  if (CAUSAL) qb = p.nblk - 1 - qb;  // heaviest query blocks first
  const int b = bh / p.H, h = bh % p.H;
  const int Lq = p.len_q(b), Lk = p.len_k(b);
  const bool half = p.half_head(D);
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, hi = lane >> 5;
  const int q0 = qb * FBM, qw = q0 + 32 * w, myq = qw + l32;

  const int64_t qoff = p.q_base(b, h), koff = p.k_base(b, h);
  const float *Qb = (const float *)p.q + qoff;
  const float *Kb = (const float *)p.k + koff;
  const float *Vb = (const float *)p.v + koff;
  float *Ob = (float *)p.out + qoff;

  int nend = Lk;
  if (CAUSAL) nend = min(nend, min(q0 + FBM, Lq));
  if (q0 >= Lq) nend = 0;
  const int ntiles = (nend + FB - 1) / FB;
  // This wave's keys: causal waves stop after their own diagonal block.
  const int wend = qw >= Lq ? 0 : (CAUSAL ? min(nend, qw + 32) : nend);

  const float scale = *p.scale, bias = p.bias[b];
  const float nsl = -scale * kLog2e, nbl = -bias * kLog2e;

  float qv[D / 2];
  load_half_row<D>(qv, Qb + (int64_t)myq * p.sq_t, hi, myq < Lq && !(half && hi));
  f32x16 acc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) acc[db] = zero16();

  DmaPlan<FB, 2 * D, FW> dma;
  dma.init(w, lane, half);
  F32RowReads<D> rr;
  rr.init(l32, hi);
  const int stride_bytes = (int)(p.sk_t * 4);
  float creg = 0.0f;
  auto issue = [&](int st, int t) SIGATTN_INLINE {
    if (SCOREMOD && tid < FB) {
      const int key = t * FB + tid;
      creg = key < Lk ? -(bias + p.score_mod[p.mod_base(b) + key]) * kLog2e : 0.0f;
    }
    dma.issue((uint16_t *)sK[st], (const uint16_t *)Kb, stride_bytes, t * FB, Lk);
    dma.issue((uint16_t *)sV[st], (const uint16_t *)Vb, stride_bytes, t * FB, Lk);
  };

  if (ntiles > 0) issue(0, 0);
  for (int t = 0; t < ntiles; ++t) {
    const int st = t & 1;
    wait_dma();
    if (SCOREMOD && tid < FB) sC[st][tid] = creg;
    // Tile t has landed for every wave, and every wave is done with tile t-1,
    // whose stage the next copy refills.
    __syncthreads();
    if (t + 1 < ntiles) issue(st ^ 1, t + 1);
    const int k0 = t * FB;
    if (k0 >= wend) continue;
    f32x16 s = zero16();
    head_product<D>(s, sK[st], qv, l32, hi);
    const bool mask = k0 + FB > Lk || (CAUSAL && k0 + FB - 1 > qw);
    float pr[16];
#pragma unroll
    for (int g = 0; g < 4; ++g)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 4 * g + r, kr = 8 * g + 4 * hi + r;
        const float c = SCOREMOD ? sC[st][kr] : nbl;
        float x = sigmoid_from_neg_log2(__builtin_fmaf(s[i], nsl, c));
        if (mask && (k0 + kr >= Lk || (CAUSAL && k0 + kr > myq))) x = 0.0f;
        pr[i] = x;
      }
    row_product<D>(acc, sV[st], pr, rr);
  }

  if (myq < p.q_rows_out(Lq)) store_row<D>(Ob + (int64_t)myq * p.sq_t, acc, 1.0f, myq < Lq, hi, half);
}

// dQ = (dP ⊙ P ⊙ (1 - P)) · K · scale with dP = dO · Vᵀ, one workgroup per
// (batch, head, 128-query block); keys streamed.
template <int D, bool CAUSAL, bool SCOREMOD>
__global__ __launch_bounds__(64 * FW, bwd_f32_occupancy<D>()) void dq_f32_kernel(const KParams p) {
  constexpr int NDB = D / 32;
  constexpr int NS = dq_f32_stages<D>();
  __shared__ __attribute__((aligned(16))) float sK[NS][FB * D];
  __shared__ __attribute__((aligned(16))) float sV[NS][FB * D];
  __shared__ float sC[SCOREMOD ? NS : 1][FB];

  const int wg = gap_prologue<4>(p, sK);  // packed layouts: leading gap-zeroing workgroups
  if (wg < 0) return;
  const int BH = p.B * p.H;
  const int bh = wg % BH;
  int qb = wg / BH;
  if (CAUSAL) qb = p.nblk - 1 - qb;
  const int b = bh / p.H, h = bh % p.H;
  const int Lq = p.len_q(b), Lk = p.len_k(b);
  const bool half = p.half_head(D);
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, hi = lane >> 5;
  const int q0 = qb * FBM, qw = q0 + 32 * w, myq = qw + l32;

  const int64_t qoff = p.q_base(b, h), koff = p.k_base(b, h);
  const float *Qb = (const float *)p.q + qoff;
  const float *dOb = (const float *)p.dout + qoff;
  const float *Kb = (const float *)p.k + koff;
  const float *Vb = (const float *)p.v + koff;
  float *dQb = (float *)p.dq + qoff;

  int nend = Lk;
  if (CAUSAL) nend = min(nend, min(q0 + FBM, Lq));
  if (q0 >= Lq) nend = 0;
  const int ntiles = (nend + FB - 1) / FB;
  const int wend = qw >= Lq ? 0 : (CAUSAL ? min(nend, qw + 32) : nend);

  const float scale = *p.scale, bias = p.bias[b];
  const float nsl = -scale * kLog2e, nbl = -bias * kLog2e;

  float qv[D / 2], ov[D / 2];
  const bool ok = myq < Lq && !(half && hi);
  load_half_row<D>(qv, Qb + (int64_t)myq * p.sq_t, hi, ok);
  load_half_row<D>(ov, dOb + (int64_t)myq * p.sq_t, hi, ok);
  f32x16 acc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) acc[db] = zero16();

  DmaPlan<FB, 2 * D, FW> dma;
  dma.init(w, lane, half);
  F32RowReads<D> rr;
  rr.init(l32, hi);
  const int stride_bytes = (int)(p.sk_t * 4);
  float creg = 0.0f;
  auto issue = [&](int st, int t) SIGATTN_INLINE {
    if (SCOREMOD && tid < FB) {
      const int key = t * FB + tid;
      creg = key < Lk ? -(bias + p.score_mod[p.mod_base(b) + key]) * kLog2e : 0.0f;
    }
    dma.issue((uint16_t *)sK[st], (const uint16_t *)Kb, stride_bytes, t * FB, Lk);
    dma.issue((uint16_t *)sV[st], (const uint16_t *)Vb, stride_bytes, t * FB, Lk);
  };

  // Element i of a tile (its key 8(i/4) + 4hi + i%4, the lane's query).
  auto sigma = [&](int st, const f32x16 &s, int i) SIGATTN_INLINE {
    const float c = SCOREMOD ? sC[st][8 * (i / 4) + 4 * hi + i % 4] : nbl;
    return sigmoid_from_neg_log2(__builtin_fmaf(s[i], nsl, c));
  };
  auto dsig = [](float pr, float dp) SIGATTN_INLINE {
    const float u = pr * dp;
    return __builtin_fmaf(-pr, u, u);  // dP·P·(1 - P)
  };
  float ds[16];
  // Keys at or past seq_lens_k, or (causal) after the lane's query, get
  // dS = 0 (one branch per tile, after the arithmetic); then dQ += dS·K over
  // tile t's rows.
  auto rows = [&](int t) SIGATTN_INLINE {
    const int k0 = t * FB;
    if (k0 + FB > Lk || (CAUSAL && k0 + FB - 1 > qw)) {
      const int lim = (CAUSAL ? min(Lk, myq + 1) : Lk) - k0 - 4 * hi;  // key k0 + 4hi + e valid iff e < lim
#pragma unroll
      for (int i = 0; i < 16; ++i)
        if (8 * (i / 4) + i % 4 >= lim) ds[i] = 0.0f;
    }
    row_product<D>(acc, sK[t % NS], ds, rr);
  };
  const int tb = (wend + FB - 1) / FB;  // this wave's key tiles: 0 .. tb-1
  if constexpr (NS == 2) {
    if (ntiles > 0) issue(0, 0);
    for (int t = 0; t < ntiles; ++t) {
      const int st = t & 1;
      wait_dma();
      if (SCOREMOD && tid < FB) sC[st][tid] = creg;
      // Tile t has landed for every wave, and every wave is done with tile
      // t-1, whose stage the next copy refills.
      __syncthreads();
      if (t + 1 < ntiles) issue(st ^ 1, t + 1);
      if (t >= tb) continue;
      f32x16 s = zero16(), dp = zero16();
      float pr[16];
      head_product<D>(s, sK[st], qv, l32, hi);
      head_product_with<D>(dp, sV[st], ov, l32, hi, [&](int i) SIGATTN_INLINE { pr[i] = sigma(st, s, i); });
#pragma unroll
      for (int i = 0; i < 16; ++i) ds[i] = dsig(pr[i], dp[i]);
      rows(t);
    }
  } else {
    // Three stages: iteration t runs tile t+1's S and dP chains with tile t's
    // arithmetic (inputs from the previous iteration) spread over the dP
    // chain, then tile t's row products.  Tile t+2 is copied meanwhile into
    // the stage of tile t-1, which every wave has finished by the barrier of
    // iteration t.
    f32x16 s0 = zero16(), p0 = zero16(), s1 = zero16(), p1 = zero16();
    if (ntiles > 0) {
      issue(0, 0);
      wait_dma();
      if (SCOREMOD && tid < FB) sC[0][tid] = creg;
      __syncthreads();
      if (ntiles > 1) issue(1, 1);
      if (tb > 0) {
        head_product<D>(s0, sK[0], qv, l32, hi);
        head_product<D>(p0, sV[0], ov, l32, hi);
      }
    }
    auto step = [&](int t, const f32x16 &sc, const f32x16 &pc, f32x16 &sn, f32x16 &pn) SIGATTN_INLINE {
      if (t + 1 < ntiles) {
        wait_dma();
        if (SCOREMOD && tid < FB) sC[(t + 1) % NS][tid] = creg;
        __syncthreads();
        if (t + 2 < ntiles) issue((t + 2) % NS, t + 2);
      }
      if (t >= tb) return;
      const int st = t % NS;
      auto elem = [&](int i) SIGATTN_INLINE { ds[i] = dsig(sigma(st, sc, i), pc[i]); };
      if (t + 1 < tb) {
        const int st1 = (t + 1) % NS;
        sn = zero16();
        pn = zero16();
        head_product<D>(sn, sK[st1], qv, l32, hi);
        head_product_with<D>(pn, sV[st1], ov, l32, hi, elem);
      } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) elem(i);
      }
      rows(t);
    };
    for (int t = 0; t < ntiles; t += 2) {
      step(t, s0, p0, s1, p1);
      if (t + 1 < ntiles) step(t + 1, s1, p1, s0, p0);
    }
  }

  if (myq < p.q_rows_out(Lq)) store_row<D>(dQb + (int64_t)myq * p.sq_t, acc, scale, myq < Lq, hi, half);
}

// dV = Pᵀ · dO and dK = dSᵀ · Q · scale, one workgroup per (batch, head,
// 128-key block); queries streamed.
template <int D, bool CAUSAL, bool SCOREMOD>
__global__ __launch_bounds__(64 * FW, bwd_f32_occupancy<D>()) void dkdv_f32_kernel(const KParams p) {
  constexpr int NDB = D / 32;
  __shared__ __attribute__((aligned(16))) float sQ[2][FB * D];
  __shared__ __attribute__((aligned(16))) float sO[2][FB * D];

  const int BH = p.B * p.H;
  const int bh = blockIdx.x % BH, kb = blockIdx.x / BH;  // causal: low key blocks (the most work) first
  const int b = bh / p.H, h = bh % p.H;
  const int Lq = p.len_q(b), Lk = p.len_k(b);
  const bool half = p.half_head(D);
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, hi = lane >> 5;
  const int k0 = kb * FBM, kw = k0 + 32 * w, myk = kw + l32;

  const int64_t qoff = p.q_base(b, h), koff = p.k_base(b, h);
  const float *Qb = (const float *)p.q + qoff;
  const float *dOb = (const float *)p.dout + qoff;
  const float *Kb = (const float *)p.k + koff;
  const float *Vb = (const float *)p.v + koff;
  float *dKb = (float *)p.dk + koff;
  float *dVb = (float *)p.dv + koff;

  // Queries of the workgroup: causal ones before its first key see none of its keys.
  const int mstart = CAUSAL ? min((k0 / FB) * FB, Lq) : 0;
  const int mend = k0 >= Lk ? mstart : Lq;
  const int ntiles = (mend - mstart + FB - 1) / FB;

  const float scale = *p.scale, bias = p.bias[b];
  const float nsl = -scale * kLog2e;
  const bool kok = myk < Lk;
  float nc = -bias * kLog2e;
  if (SCOREMOD) nc = kok ? -(bias + p.score_mod[p.mod_base(b) + myk]) * kLog2e : 0.0f;

  float kv[D / 2], vv[D / 2];
  const bool ok = kok && !(half && hi);
  load_half_row<D>(kv, Kb + (int64_t)myk * p.sk_t, hi, ok);
  load_half_row<D>(vv, Vb + (int64_t)myk * p.sk_t, hi, ok);
  f32x16 dka[NDB], dva[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) dka[db] = dva[db] = zero16();

  DmaPlan<FB, 2 * D, FW> dma;
  dma.init(w, lane, half);
  F32RowReads<D> rr;
  rr.init(l32, hi);
  const int stride_bytes = (int)(p.sq_t * 4);
  const float *Qm = Qb + (int64_t)mstart * p.sq_t;
  const float *dOm = dOb + (int64_t)mstart * p.sq_t;
  auto issue = [&](int st, int t) SIGATTN_INLINE {
    dma.issue((uint16_t *)sQ[st], (const uint16_t *)Qm, stride_bytes, t * FB, mend - mstart);
    dma.issue((uint16_t *)sO[st], (const uint16_t *)dOm, stride_bytes, t * FB, mend - mstart);
  };

  // This wave's query tiles ta <= t < tb: none for keys past Lk; causal, none
  // whose queries all precede the wave's first key (tile t ends at query
  // mstart + 32t + 31).
  int ta = 0;
  if (CAUSAL) {
    const int dd = kw - mstart - FB + 1;
    ta = dd > 0 ? (dd + FB - 1) / FB : 0;
  }
  const int tb = kw >= Lk ? 0 : ntiles;
  if (ntiles > 0) issue(0, 0);
  for (int t = 0; t < ntiles; ++t) {
    const int st = t & 1;
    wait_dma();
    __syncthreads();
    if (t + 1 < ntiles) issue(st ^ 1, t + 1);
    if (t < ta || t >= tb) continue;
    const int m0 = mstart + t * FB;
    f32x16 s = zero16(), dp = zero16();
    float pr[16], ds[16];
    head_product<D>(s, sQ[st], kv, l32, hi);
    // P = sigmoid(S) between the dP chain's MFMAs.
    head_product_with<D>(dp, sO[st], vv, l32, hi, [&](int i) SIGATTN_INLINE {
      pr[i] = sigmoid_from_neg_log2(__builtin_fmaf(s[i], nsl, nc));
    });
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const float u = pr[i] * dp[i];
      ds[i] = __builtin_fmaf(-pr[i], u, u);
    }
    // Queries at or past seq_lens_q, or (causal) before the lane's key: one
    // branch per tile, after the arithmetic.
    if (m0 + FB > Lq || (CAUSAL && m0 < kw + 31)) {
      const int e_end = Lq - m0 - 4 * hi;               // query m0 + 4hi + e valid iff
      const int e_lo = CAUSAL ? myk - m0 - 4 * hi : 0;  // e_lo <= e < e_end
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int e = 8 * (i / 4) + i % 4;
        if (e >= e_end || e < e_lo) pr[i] = ds[i] = 0.0f;
      }
    }
    row_product<D>(dva, sO[st], pr, rr);
    row_product<D>(dka, sQ[st], ds, rr);
  }

  if (myk < p.k_rows_out(Lk)) {
    store_row<D>(dKb + (int64_t)myk * p.sk_t, dka, scale, kok, hi, half);
    store_row<D>(dVb + (int64_t)myk * p.sk_t, dva, 1.0f, kok, hi, half);
  }
}

template <int D> void fwd_t(const KParams &kp, bool causal, bool scoremod, hipStream_t st) {
  KParams p = kp;
  p.nblk = (p.Tq + FBM - 1) / FBM;
  const dim3 grid((unsigned)(p.nblk * p.B * p.H + p.ngap[0] + p.ngap[1])), block(64 * FW);
  if (causal) {
    if (scoremod) fwd_f32_kernel<D, true, true><<<grid, block, 0, st>>>(p);
    else fwd_f32_kernel<D, true, false><<<grid, block, 0, st>>>(p);
  } else {
    if (scoremod) fwd_f32_kernel<D, false, true><<<grid, block, 0, st>>>(p);
    else fwd_f32_kernel<D, false, false><<<grid, block, 0, st>>>(p);
  }
}

template <int D> void dq_t(const KParams &kp, bool causal, bool scoremod, hipStream_t st) {
  KParams p = kp;
  p.nblk = (p.Tq + FBM - 1) / FBM;
  const dim3 grid((unsigned)(p.nblk * p.B * p.H + p.ngap[0] + p.ngap[1])), block(64 * FW);
  if (causal) {
    if (scoremod) dq_f32_kernel<D, true, true><<<grid, block, 0, st>>>(p);
    else dq_f32_kernel<D, true, false><<<grid, block, 0, st>>>(p);
  } else {
    if (scoremod) dq_f32_kernel<D, false, true><<<grid, block, 0, st>>>(p);
    else dq_f32_kernel<D, false, false><<<grid, block, 0, st>>>(p);
  }
}

template <int D> void dkdv_t(const KParams &kp, bool causal, bool scoremod, hipStream_t st) {
  KParams p = kp;
  p.nblk = (p.Tk + FBM - 1) / FBM;
  const dim3 grid((unsigned)(p.nblk * p.B * p.H)), block(64 * FW);  // no gap rows here (the dQ launch's)
  if (causal) {
    if (scoremod) dkdv_f32_kernel<D, true, true><<<grid, block, 0, st>>>(p);
    else dkdv_f32_kernel<D, true, false><<<grid, block, 0, st>>>(p);
  } else {
    if (scoremod) dkdv_f32_kernel<D, false, true><<<grid, block, 0, st>>>(p);
    else dkdv_f32_kernel<D, false, false><<<grid, block, 0, st>>>(p);
  }
}

}  // namespace

void launch_fwd_f32(const KParams &p, int D, bool causal, bool scoremod, hipStream_t st) {
  if (D == 128) fwd_t<128>(p, causal, scoremod, st);
  else if (D == 64) fwd_t<64>(p, causal, scoremod, st);
  else fwd_t<32>(p, causal, scoremod, st);
}

void launch_bwd_dq_f32(const KParams &p, int D, bool causal, bool scoremod, hipStream_t st) {
  if (D == 128) dq_t<128>(p, causal, scoremod, st);
  else if (D == 64) dq_t<64>(p, causal, scoremod, st);
  else dq_t<32>(p, causal, scoremod, st);
}

void launch_bwd_dkdv_f32(const KParams &p, int D, bool causal, bool scoremod, hipStream_t st) {
  if (D == 128) dkdv_t<128>(p, causal, scoremod, st);
  else if (D == 64) dkdv_t<64>(p, causal, scoremod, st);
  else dkdv_t<32>(p, causal, scoremod, st);
}

}  // namespace sigattn
