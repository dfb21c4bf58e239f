// Forward kernel: O = sigmoid(Q·Kᵀ·scale + bias + score_mod) · V on gfx950 MFMA.
//
// Semantics follow the reference's _fwd_dense_kernel
// (src/triton_sigmoid/sigmoid_triton_dense.py:23-154) and _fwd_padded_kernel
// (src/triton_sigmoid/sigmoid_triton_padded.py:24-171):
//   S = Q·Kᵀ in fp32; S = S*scale + bias[b] (+ score_mod[b, key]);
//   causal keeps key <= query; P = sigmoid(S) in fp32; P is rounded to the
//   I/O dtype; O += P·V in fp32; O is stored in the I/O dtype; query rows at or
//   past seq_lens_q are zero; K/V rows at or past seq_lens_k are never read.
//
// Structure (one workgroup = 4 waves = 128 queries of one (batch, head)):
//   * each wave keeps its 32 query rows as MFMA operands in VGPRs;
//   * 64-key tiles of K and V are double-buffered row-major in LDS; the next
//     tile's global loads are issued before the current tile's MFMAs;
//   * Sᵀ = K·Qᵀ (32x32x16 MFMA), sigmoid on the fp32 accumulators, then
//     Oᵀ += Vᵀ·Pᵀ with Pᵀ taken straight from the Sᵀ accumulator registers and
//     Vᵀ read from the row-major V tile with ds_read_b64_tr_b16;
//   * causal: key tiles past the block's last query are never loaded, a wave
//     skips 32-key blocks entirely above its rows, the element mask runs only
//     on blocks that straddle the diagonal; the grid runs heaviest blocks first.
// Zero-filled K/V rows past seq_lens_k contribute exactly 0 (P·0), so only the
// causal condition needs an element mask.
#include "common.h"
#include "launch.h"

namespace sigattn {

template <typename T, int D, bool CAUSAL, bool SCOREMOD>
__global__ __launch_bounds__(256, 2) void fwd_mfma_kernel(const KParams p) {
  constexpr int BM = 128;      // queries per workgroup
  constexpr int BN = 64;       // keys per tile
  constexpr int NKS = D / 16;  // MFMA k-steps over the head dim
  constexpr int NDB = D / 32;  // 32-row blocks of Oᵀ

  // Swizzled (unpadded) K and V tiles, two stages each.
  __shared__ __attribute__((aligned(16))) uint16_t sK[2][BN * D];
  __shared__ __attribute__((aligned(16))) uint16_t sV[2][BN * D];
  __shared__ __attribute__((aligned(16))) float sC[SCOREMOD ? 2 * BN : 4];

  const int BH = p.B * p.H;
  const int id = blockIdx.x;
  const int bh = id % BH;
  int qb = id / BH;
  if (CAUSAL) qb = p.nblk - 1 - qb;  // heaviest query blocks first
  const int b = bh / p.H, h = bh % p.H;

  const int Lq = clamp_len(p.seq_q, b, p.Tq);
  const int Lk = clamp_len(p.seq_k, b, p.Tk);

  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int l32 = lane & 31, hi = lane >> 5;
  const int q0 = qb * BM;
  const int qw = q0 + w * 32;
  const int my_q = qw + l32;

  const uint16_t *Qb = (const uint16_t *)p.q + (int64_t)b * p.sq_b + (int64_t)h * p.sq_h;
  const uint16_t *Kb = (const uint16_t *)p.k + (int64_t)b * p.sk_b + (int64_t)h * p.sk_h;
  const uint16_t *Vb = (const uint16_t *)p.v + (int64_t)b * p.sk_b + (int64_t)h * p.sk_h;
  uint16_t *Ob = (uint16_t *)p.out + (int64_t)b * p.sq_b + (int64_t)h * p.sq_h;

  int nend = Lk;
  if (CAUSAL) nend = min(nend, min(q0 + BM, Lq));
  if (q0 >= Lq) nend = 0;
  const int ntiles = (nend + BN - 1) / BN;

  const float scale = *p.scale;
  const float bias = p.bias[b];
  const float nsl = -scale * kLog2e;
  const float nbl = -bias * kLog2e;

  // This wave's query rows as B operands (k = d = 16s + 8h + j).
  u32x4 qf[NKS];
  {
    const bool ok = my_q < Lq;
    const uint16_t *qrow = Qb + (int64_t)my_q * p.sq_t + 8 * hi;
#pragma unroll
    for (int s = 0; s < NKS; ++s) qf[s] = ok ? *(const u32x4 *)(qrow + 16 * s) : zero4();
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
  auto lstore = [&](int st) {
    kst.store(sK[st], tid);
    vst.store(sV[st], tid);
    if (SCOREMOD && tid < BN) sC[st * BN + tid] = creg;
  };

  if (ntiles > 0) {
    gload(0);
    lstore(0);
  }
  __syncthreads();

  for (int it = 0; it < ntiles; ++it) {
    const int st = it & 1;
    const int n0 = it * BN;
    const bool more = it + 1 < ntiles;
    if (more) gload(n0 + BN);

    if (!CAUSAL || n0 <= qw + 31) {
      uint32_t pk[BN / 4];  // this lane's BN/2 probabilities, packed in pairs
#pragma unroll
      for (int kb = 0; kb < BN / 32; ++kb) {
        const int kbase = n0 + kb * 32;
        if (CAUSAL && kbase > qw + 31) {
#pragma unroll
          for (int i = 0; i < 8; ++i) pk[kb * 8 + i] = 0u;
          continue;
        }
        f32x16 s = zero16();
#pragma unroll
        for (int ks = 0; ks < NKS; ++ks)
          s = Elem<T>::mfma(read_row_operand<D>(sK[st], kb * 32 + l32, ks, hi), qf[ks], s);

        float c[16];
        if constexpr (SCOREMOD) {
#pragma unroll
          for (int g = 0; g < 4; ++g) {
            const float4 cv = *(const float4 *)&sC[st * BN + kb * 32 + 8 * g + 4 * hi];
            c[4 * g + 0] = cv.x; c[4 * g + 1] = cv.y; c[4 * g + 2] = cv.z; c[4 * g + 3] = cv.w;
          }
        } else {
#pragma unroll
          for (int i = 0; i < 16; ++i) c[i] = nbl;
        }
        float pv[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) pv[i] = sigmoid_from_neg_log2(__builtin_fmaf(s[i], nsl, c[i]));
        if (CAUSAL && kbase + 31 > qw) {
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int key = kbase + 8 * (i / 4) + 4 * hi + (i % 4);
            if (key > my_q) pv[i] = 0.0f;
          }
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) pk[kb * 8 + i] = Elem<T>::pack(pv[2 * i], pv[2 * i + 1]);
      }

      // Oᵀ[d, q] += Vᵀ[d, key] · Pᵀ[key, q]
#pragma unroll
      for (int ks = 0; ks < BN / 16; ++ks) {
        if (CAUSAL && n0 + ks * 16 > qw + 31) break;
        const u32x4 bop = (u32x4){pk[4 * ks], pk[4 * ks + 1], pk[4 * ks + 2], pk[4 * ks + 3]};
#pragma unroll
        for (int db = 0; db < NDB; ++db)
          acc[db] = Elem<T>::mfma(read_tr16_swz<D>(sV[st], db * 32, ks, lane), bop, acc[db]);
      }
    }

    if (more) lstore(st ^ 1);
    __syncthreads();
  }

  // Oᵀ accumulators -> O rows (4 consecutive d per 8-byte store).
  if (my_q < p.Tq) {
    uint16_t *orow = Ob + (int64_t)my_q * p.sq_t;
    const bool valid = my_q < Lq;
#pragma unroll
    for (int db = 0; db < NDB; ++db) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d0 = db * 32 + 8 * g + 4 * hi;
        u32x2 o;
        o.x = valid ? Elem<T>::pack(acc[db][4 * g + 0], acc[db][4 * g + 1]) : 0u;
        o.y = valid ? Elem<T>::pack(acc[db][4 * g + 2], acc[db][4 * g + 3]) : 0u;
        *(u32x2 *)(orow + d0) = o;
      }
    }
  }
}

template <typename T, int D>
static void launch_fwd_t(const KParams &kp, bool causal, bool scoremod, hipStream_t st) {
  constexpr int BM = 128;
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
