// Split-KV forward for short query blocks (Tq <= 32, non-causal): the decode
// and chunked-prefill shape, where the 256-query tiles of the main forward
// kernel would leave most MFMA rows empty and one workgroup per (batch, head)
// could not fill the GPU.
//
// Semantics are the forward's (src/triton_sigmoid/sigmoid_triton_padded.py:
// 24-171 in the reference, as in fwd.hip): O = sigmoid(Q·Kᵀ·scale + bias +
// score_mod)·V with P rounded to the I/O dtype, fp32 accumulation, padded query
// rows zero.  Sigmoid attention has no row normalisation, so O over a key range
// is the plain sum of O over its parts: the keys of each (batch, head) are cut
// into nsplit chunks, one workgroup per chunk writes an fp32 partial, and a
// second kernel sums the partials in chunk order (deterministic).  With one
// chunk the workgroup writes O itself and no workspace is used.
//
// Workgroup: four waves, 32 queries (the MFMA's 32 columns), one key chunk.
// Wave w takes the 32-key blocks w, w+4, w+8, ... of the chunk.  Each wave
// streams its own blocks through a private two-stage LDS ring with direct
// global->LDS copies and waits for them with its own vmcnt, so the key loop has
// no workgroup barriers.  The kernel is HBM-bound (2·D·2 bytes of K and V per
// key against 4·D·32 MFMA FLOPs), so each block is computed as a plain
// sequence: Sᵀ = K·Qᵀ, P = sigmoid(Sᵀ) on packed words, Oᵀ += Vᵀ·Pᵀ.  The four
// waves' Oᵀ partials are summed through LDS at the end.
#include <atomic>
#include <mutex>

#include "common.h"
#include "launch.h"

namespace sigattn {

// Partials of sigattn_fwd_noalloc's split-KV launches.  In host code the name
// `scratch` is only a stand-in for the symbol: its device address (one per
// GPU) comes from hipGetSymbolAddress and is what kernels are given.  Every
// call on a GPU uses that GPU's one array, so calls that overlap on one GPU
// (two streams, two threads) race.  No clearing is needed: the reduction reads
// exactly the partials the chunk kernel of the same call writes.
static __device__ __align__(256) float scratch[kSplitScratchBytes / sizeof(float)];

namespace {
constexpr int kMaxDevices = 64;
std::atomic<float *> g_scratch[kMaxDevices];
std::mutex g_scratch_mu;
}  // namespace

hipError_t splitkv_scratch(float **ptr) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  float *p = g_scratch[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    // First call on this device (which is current): look the address up.
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    p = g_scratch[dev].load(std::memory_order_relaxed);
    if (p == nullptr) {
      // The first call may come while this thread captures a graph in the
      // global mode, which refuses runtime calls it deems unsafe; the lookup
      // enqueues nothing, so it runs in the relaxed mode, and the thread's
      // mode is restored afterwards.
      hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
      e = hipThreadExchangeStreamCaptureMode(&mode);
      if (e != hipSuccess) return e;
      void *addr = nullptr;
      e = hipGetSymbolAddress(&addr, HIP_SYMBOL(scratch));
      const hipError_t restore = hipThreadExchangeStreamCaptureMode(&mode);
      if (e == hipSuccess) e = restore;
      if (e != hipSuccess) return e;
      if (addr == nullptr) return hipErrorInvalidSymbol;
      p = static_cast<float *>(addr);
      g_scratch[dev].store(p, std::memory_order_release);
    }
  }
  *ptr = p;
  return hipSuccess;
}

template <int N> __device__ __forceinline__ void wait_vmcnt() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Waits until at most `ahead` blocks of copies (PER instructions each) are in
// flight, ahead < 4.
template <int PER> __device__ __forceinline__ void wait_blocks(int ahead) {
  if (ahead <= 0) wait_vmcnt<0>();
  else if (ahead == 1) wait_vmcnt<PER>();
  else if (ahead == 2) wait_vmcnt<2 * PER>();
  else wait_vmcnt<3 * PER>();
}

template <typename T, int D, int NW, int NST, bool SCOREMOD, bool DIRECT>
__global__ __launch_bounds__(64 * NW, 1) void fwd_splitkv_kernel(const KParams p) {
  // NW waves; each streams 32-key blocks through its own NST-stage ring and
  // keeps NST - 1 blocks of copies in flight while it computes one.
  constexpr int KB = 32;         // keys per block (one MFMA contraction of 2 k-steps)
  constexpr int NKS = D / 16, NDB = D / 32;
  static_assert(NST >= 2 && NST <= 4, "ring depth");
  using Plan = DmaPlan<KB, D, 1>;
  constexpr int NI = Plan::NI;   // copy instructions per block and tensor

  __shared__ __attribute__((aligned(16))) uint16_t sK[NW][NST][KB * D];
  __shared__ __attribute__((aligned(16))) uint16_t sV[NW][NST][KB * D];
  static_assert(sizeof(sK) >= NW * 32 * D * sizeof(float), "reduction buffer");

  const int NS = p.nsplit, C = p.chunk;
  const int s = blockIdx.x % NS, bh = blockIdx.x / NS;
  const int b = bh / p.H, h = bh % p.H;
  const int Lq = p.len_q(b), Lk = p.len_k(b);
  const int k0 = s * C, k1 = min(k0 + C, Lk);
  // A chunk past the keys has no partial (the reduction stops before it).
  if (!DIRECT && (k0 >= Lk || Lq == 0)) return;

  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l32 = lane & 31, hi = lane >> 5;

  const int64_t qoff = p.q_base(b, h), koff = p.k_base(b, h);
  const uint16_t *Qb = (const uint16_t *)p.q + qoff;
  const uint16_t *Kb = (const uint16_t *)p.k + koff;
  const uint16_t *Vb = (const uint16_t *)p.v + koff;

  const float scale = *p.scale;
  const float bias = p.bias[b];
  const float nsl = -scale * kLog2e, nbl = -bias * kLog2e;

  // Query l32 as the B operand (k = d = 16s + 8h + j); rows past Lq are zero.
  u32x4 qf[NKS];
  {
    const bool ok = l32 < Lq;
    const uint16_t *qrow = Qb + (int64_t)l32 * p.sq_t + 8 * hi;
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) qf[ks] = ok ? *(const u32x4 *)(qrow + 16 * ks) : zero4();
  }
  // Wait for Q here, before the first tile copy is in flight.
#pragma unroll
  for (int ks = 0; ks < NKS; ++ks) asm volatile("" ::"v"(qf[ks]));

  f32x16 acc[NDB];
#pragma unroll
  for (int db = 0; db < NDB; ++db) acc[db] = zero16();

  TileOffsets<D> to;
  to.init(lane);
  Plan dma;
  dma.init(0, lane);
  const int kv_stride_bytes = (int)(p.sk_t * 2);
  const int nb = k1 > k0 ? (k1 - k0 + KB - 1) / KB : 0;   // blocks of the chunk
  const int nbw = nb > w ? (nb - w + NW - 1) / NW : 0;    // ... of this wave
  auto first_key = [&](int i) SIGATTN_INLINE { return k0 + KB * (w + NW * i); };
  auto issue = [&](int st, int i) SIGATTN_INLINE {
    dma.issue(sK[w][st], Kb, kv_stride_bytes, first_key(i), Lk);
    dma.issue(sV[w][st], Vb, kv_stride_bytes, first_key(i), Lk);
  };

#pragma unroll
  for (int i = 0; i < NST - 1; ++i)
    if (i < nbw) issue(i, i);
  for (int i = 0; i < nbw; ++i) {
    const int st = i % NST;
    // Block i + NST - 1 goes into the stage block i - 1 used; every LDS read
    // of that block has returned (its MFMAs were issued) before the copy.
    if (i + NST - 1 < nbw) {
      asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
      issue((i + NST - 1) % NST, i + NST - 1);
    }
    // Block i has landed once at most the blocks after it are in flight.
    wait_blocks<2 * NI>(min(NST - 1, nbw - 1 - i));
    const uint16_t *tK = sK[w][st];
    const uint16_t *tV = sV[w][st];

    f32x16 sc = zero16();
#pragma unroll
    for (int ks = 0; ks < NKS; ++ks) sc = Elem<T>::mfma(ld_row<D>(tK, to, 0, ks), qf[ks], sc);

    // P words: accumulator element i of lane (l32, hi) is key
    // kb + 8(i/4) + 4hi + i%4 of query l32; keys at or past k1 get P = 0.
    const int kb = first_key(i);
    uint32_t pk[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int i0 = 2 * e;
      const int key = kb + 8 * (i0 / 4) + 4 * hi + (i0 % 4);
      float c0 = nbl, c1 = nbl;
      if (SCOREMOD) {
        const int64_t mb = p.mod_base(b);
        c0 = key < k1 ? -(bias + p.score_mod[mb + key]) * kLog2e : 0.0f;
        c1 = key + 1 < k1 ? -(bias + p.score_mod[mb + key + 1]) * kLog2e : 0.0f;
      }
      float p0 = sigmoid_from_neg_log2(__builtin_fmaf(sc[i0], nsl, c0));
      float p1 = sigmoid_from_neg_log2(__builtin_fmaf(sc[i0 + 1], nsl, c1));
      p0 = key < k1 ? p0 : 0.0f;
      p1 = key + 1 < k1 ? p1 : 0.0f;
      pk[e] = Elem<T>::pack(p0, p1);
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const u32x4 bp = (u32x4){pk[4 * j], pk[4 * j + 1], pk[4 * j + 2], pk[4 * j + 3]};
#pragma unroll
      for (int db = 0; db < NDB; ++db) acc[db] = Elem<T>::mfma(ld_tr<D>(tV, to, j, db), bp, acc[db]);
    }
  }

  // Sum the waves' Oᵀ partials: red[w][q][d] in the tile memory.
  float *red = (float *)&sK[0][0][0];
  __syncthreads();
#pragma unroll
  for (int db = 0; db < NDB; ++db)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d0 = db * 32 + 8 * g + 4 * hi;
      *(float4 *)&red[(w * 32 + l32) * D + d0] =
          make_float4(acc[db][4 * g], acc[db][4 * g + 1], acc[db][4 * g + 2], acc[db][4 * g + 3]);
    }
  __syncthreads();
  const int nrows = DIRECT ? min(32, p.q_rows_out(Lq)) : min(32, Lq);
  for (int it = tid; it < nrows * (D / 4); it += 64 * NW) {
    const int q = it / (D / 4), d0 = 4 * (it % (D / 4));
    float4 v = *(const float4 *)&red[q * D + d0];
#pragma unroll
    for (int x = 1; x < NW; ++x) {
      const float4 u = *(const float4 *)&red[(x * 32 + q) * D + d0];
      v.x += u.x; v.y += u.y; v.z += u.z; v.w += u.w;
    }
    if (DIRECT) {
      u32x2 o;
      o.x = Elem<T>::pack(v.x, v.y);
      o.y = Elem<T>::pack(v.z, v.w);
      if (q >= Lq) o = (u32x2){0u, 0u};
      *(u32x2 *)((uint16_t *)p.out + qoff + (int64_t)q * p.sq_t + d0) = o;
    } else {
      float *ws = p.ws + ((((int64_t)s * p.B + b) * p.H + h) * p.Tq + q) * D;
      *(float4 *)&ws[d0] = v;
    }
  }
}

// O = sum of the chunks' partials, in chunk order; padded query rows are zero.
template <typename T, int D>
__global__ __launch_bounds__(256) void fwd_splitkv_reduce_kernel(const KParams p) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t total = (int64_t)p.B * p.H * p.Tq * (D / 4);
  if (t >= total) return;
  const int d0 = 4 * (int)(t % (D / 4));
  const int64_t r = t / (D / 4);
  const int q = (int)(r % p.Tq);
  const int bh = (int)(r / p.Tq), b = bh / p.H, h = bh % p.H;
  const int Lq = p.len_q(b), Lk = p.len_k(b);
  if (q >= p.q_rows_out(Lq)) return;
  float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  if (q < Lq) {
    const int nvs = (Lk + p.chunk - 1) / p.chunk;
    for (int s = 0; s < nvs; ++s) {
      const float4 u = *(const float4 *)&p.ws[((((int64_t)s * p.B + b) * p.H + h) * p.Tq + q) * D + d0];
      v.x += u.x; v.y += u.y; v.z += u.z; v.w += u.w;
    }
  }
  u32x2 o;
  o.x = Elem<T>::pack(v.x, v.y);
  o.y = Elem<T>::pack(v.z, v.w);
  *(u32x2 *)((uint16_t *)p.out + p.q_base(b, h) + (int64_t)q * p.sq_t + d0) = o;
}

#ifndef SIGATTN_DEC_NW_64
#define SIGATTN_DEC_NW_64 4
#endif
#ifndef SIGATTN_DEC_NST_64
#define SIGATTN_DEC_NST_64 2
#endif
#ifndef SIGATTN_DEC_NW_128
#define SIGATTN_DEC_NW_128 4
#endif
#ifndef SIGATTN_DEC_NST_128
#define SIGATTN_DEC_NST_128 2
#endif

template <typename T, int D>
static void launch_splitkv_t(const KParams &p, bool scoremod, hipStream_t st) {
  constexpr int NW = D == 64 ? SIGATTN_DEC_NW_64 : SIGATTN_DEC_NW_128;
  constexpr int NST = D == 64 ? SIGATTN_DEC_NST_64 : SIGATTN_DEC_NST_128;
  const dim3 grid((unsigned)((int64_t)p.B * p.H * p.nsplit)), block(64 * NW);
  const bool direct = p.nsplit == 1;
  if (direct) {
    if (scoremod) fwd_splitkv_kernel<T, D, NW, NST, true, true><<<grid, block, 0, st>>>(p);
    else fwd_splitkv_kernel<T, D, NW, NST, false, true><<<grid, block, 0, st>>>(p);
    return;
  }
  if (scoremod) fwd_splitkv_kernel<T, D, NW, NST, true, false><<<grid, block, 0, st>>>(p);
  else fwd_splitkv_kernel<T, D, NW, NST, false, false><<<grid, block, 0, st>>>(p);
  const int64_t total = (int64_t)p.B * p.H * p.Tq * (D / 4);
  fwd_splitkv_reduce_kernel<T, D><<<dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st>>>(p);
}

void launch_fwd_splitkv(const KParams &p, int dtype, int D, bool scoremod, hipStream_t st) {
  if (dtype == kBF16) {
    if (D == 128) launch_splitkv_t<__bf16, 128>(p, scoremod, st);
    else launch_splitkv_t<__bf16, 64>(p, scoremod, st);
  } else {
    if (D == 128) launch_splitkv_t<_Float16, 128>(p, scoremod, st);
    else launch_splitkv_t<_Float16, 64>(p, scoremod, st);
  }
}

}  // namespace sigattn
