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
// Structure (one workgroup = 4 waves = 128 queries of one (batch, head)):
//   * each wave keeps its 32 query rows as MFMA operands in VGPRs;
//   * 64-key tiles of K and V are double-buffered in swizzled LDS tiles, filled
//     by direct global->LDS DMA one tile ahead (no VGPR staging);
//   * per 32-key block: Sᵀ = K·Qᵀ (32x32x16 MFMA chain, K operands read from
//     LDS ahead of the chain), sigmoid on the fp32 accumulators, then
//     Oᵀ += Vᵀ·Pᵀ with Pᵀ taken straight from the accumulator registers and Vᵀ
//     read with ds_read_b64_tr_b16; the next block's Sᵀ chain is independent
//     of the current block's sigmoid, so MFMA and VALU work overlap;
//   * causal: key tiles past the block's last query are never loaded, a wave
//     skips 32-key blocks entirely above its rows, element masks run only on
//     tiles that straddle the diagonal or the seq_lens_k boundary; the grid
//     runs the heaviest query blocks first.
#include <type_traits>

#include "common.h"
#include "launch.h"

namespace sigattn {

template <typename T, int D, bool CAUSAL, bool SCOREMOD>
__global__ __launch_bounds__(256, 2) void fwd_mfma_kernel(const KParams p) {
  constexpr int BM = 128;      // queries per workgroup
  constexpr int BN = 64;       // keys per tile
  constexpr int NKS = D / 16;  // MFMA k-steps over the head dim
  constexpr int NDB = D / 32;  // 32-row blocks of Oᵀ

  __shared__ __attribute__((aligned(16))) uint16_t sK[2][BN * D];
  __shared__ __attribute__((aligned(16))) uint16_t sV[2][BN * D];
  __shared__ __attribute__((aligned(16))) float sC[SCOREMOD ? 2 * BN : 4];

  const int BH = p.B * p.H;
  const int bh = blockIdx.x % BH;
  int qb = blockIdx.x / BH;
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

  TileOffsets<D> to;
  to.init(lane);

  // sigmoid of one 32x32 accumulator block (keys kbase.., this lane's query)
  // into eight packed P words; MASK applies seq_lens_k and causal masks.
  auto sigmoid_block = [&](const f32x16 &s, int st, int kl, int kbase, uint32_t *out,
                           auto mask_tag) SIGATTN_INLINE {
    constexpr bool MASK = decltype(mask_tag)::value;
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
    float pv[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) pv[i] = sigmoid_from_neg_log2(__builtin_fmaf(s[i], nsl, c[i]));
    if constexpr (MASK) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int key = kbase + 8 * (i / 4) + 4 * hi + (i % 4);
        if (key >= Lk || (CAUSAL && key > my_q)) pv[i] = 0.0f;
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) out[i] = Elem<T>::pack(pv[2 * i], pv[2 * i + 1]);
  };

  // Oᵀ[d, q] += Vᵀ[d, key] · Pᵀ[key, q] for the two 16-key steps of block kbi.
  auto pv_block = [&](int st, int kbi, const uint32_t *pk) SIGATTN_INLINE {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const u32x4 bop = (u32x4){pk[4 * j], pk[4 * j + 1], pk[4 * j + 2], pk[4 * j + 3]};
#pragma unroll
      for (int db = 0; db < NDB; ++db)
        acc[db] = Elem<T>::mfma(ld_tr<D>(sV[st], to, 2 * kbi + j, db), bop, acc[db]);
    }
  };

  // Steady-state tile (no masks): four scheduling regions, each interleaving
  // MFMA with the VALU / LDS work that does not depend on it.
  //   A: K reads for block 0, then the Sᵀ0 chain
  //   B: K reads for block 1, Sᵀ1 chain        || sigmoid(Sᵀ0)
  //   C: Oᵀ += Vᵀ·Pᵀ0 (8 MFMA, 16 tr reads)    || sigmoid(Sᵀ1)
  //   D: Oᵀ += Vᵀ·Pᵀ1 (8 MFMA, 16 tr reads)
  auto tile_step = [&](int st, int n0, auto mask_tag) SIGATTN_INLINE {
    u32x4 ka[NKS], kc[NKS];
    f32x16 s0 = zero16(), s1 = zero16();
    uint32_t pk0[8], pk1[8];
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) ka[ks] = ld_row<D>(sK[st], to, 0, ks);
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) s0 = Elem<T>::mfma(ka[ks], qf[ks], s0);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) kc[ks] = ld_row<D>(sK[st], to, 32, ks);
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) s1 = Elem<T>::mfma(kc[ks], qf[ks], s1);
    sigmoid_block(s0, st, 0, n0, pk0, mask_tag);
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 72 / NKS, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    pv_block(st, 0, pk0);
    sigmoid_block(s1, st, 32, n0 + 32, pk1, mask_tag);
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
    for (int i = 0; i < 2 * NDB; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
      __builtin_amdgcn_sched_group_barrier(0x002, 72 / (2 * NDB), 0);
    }
    __builtin_amdgcn_sched_barrier(0);
    pv_block(st, 1, pk1);
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);
#pragma unroll
    for (int i = 0; i < 2 * NDB; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
  };

  float creg = 0.0f;
  auto load_c = [&](int n0) SIGATTN_INLINE {
    if (SCOREMOD && tid < BN) {
      const int key = n0 + tid;
      creg = key < Lk ? -(bias + p.score_mod[(int64_t)b * p.Tk + key]) * kLog2e : 0.0f;
    }
  };
  DmaPlan<BN, D, 4> dma;
  dma.init(w, lane);
  const int kv_stride_bytes = (int)(p.sk_t * 2);
  auto issue = [&](int st, int n0) SIGATTN_INLINE {
    dma.issue(sK[st], Kb, kv_stride_bytes, n0, Lk);
    dma.issue(sV[st], Vb, kv_stride_bytes, n0, Lk);
  };

  if (ntiles > 0) {
    load_c(0);
    issue(0, 0);
  }
  // One tile on LDS stage ST (a compile-time constant, so every swizzled
  // operand address of both stages shares one VGPR plus an immediate offset).
  auto iteration = [&](int it, auto stage_tag) SIGATTN_INLINE {
    constexpr int ST = decltype(stage_tag)::value;
    const int n0 = it * BN;
    wait_dma();
    if (SCOREMOD && tid < BN) sC[ST * BN + tid] = creg;
    __syncthreads();  // tile `it` complete; every wave is done with tile it-1
    if (it + 1 < ntiles) {
      load_c(n0 + BN);
      issue(ST ^ 1, n0 + BN);
    }
    if (!CAUSAL || n0 <= qw + 31) {
      const bool need_mask = (n0 + BN > Lk) || (CAUSAL && n0 + BN - 1 > qw);
      if (need_mask) tile_step(ST, n0, std::true_type{});
      else tile_step(ST, n0, std::false_type{});
    }
  };
  for (int it = 0; it < ntiles; it += 2) {
    iteration(it, std::integral_constant<int, 0>{});
    if (it + 1 < ntiles) iteration(it + 1, std::integral_constant<int, 1>{});
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
        o.x = Elem<T>::pack(acc[db][4 * g + 0], acc[db][4 * g + 1]);
        o.y = Elem<T>::pack(acc[db][4 * g + 2], acc[db][4 * g + 3]);
        if (!valid) o = (u32x2){0u, 0u};
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
