// C ABI of libsigattn.so (declared in include/sigattn.h).
//
// Validation runs on the host before any HIP call, so every error path is
// testable without a GPU.  Dispatch: rows starting on 16-byte boundaries take
// the MFMA kernels (f16/bf16 the 16-bit ones, fp32 the fp32 ones; D in {16,
// 32, 64, 128}); everything else takes the portable kernels.  Launches are
// asynchronous and ordered on the caller's stream (the concurrent recompute
// backward forks a second stream off it and joins it back); nothing here
// allocates device memory or synchronises the host.
#include <hip/hip_runtime.h>

#include <atomic>
#include <climits>
#include <cstdint>
#include <mutex>

#include "../../include/sigattn.h"
#include "launch.h"

using sigattn::KParams;

namespace {

bool is_pow2_head_dim(int64_t D) { return D == 16 || D == 32 || D == 64 || D == 128; }

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

bool aligned16(const void *ptr) { return ((uintptr_t)ptr & 15u) == 0; }

KParams make_params(const sigattn_problem *p) {
  KParams k{};
  k.ncu = sigattn::device_compute_units();
  k.q = p->q;
  k.k = p->k;
  k.v = p->v;
  k.bias = p->bias;
  k.scale = p->scale;
  k.score_mod = p->score_mod;
  k.seq_q = p->seq_lens_q;
  k.seq_k = p->seq_lens_k;
  k.cu_q = p->cu_seqlens_q;
  k.cu_k = p->cu_seqlens_k;
  k.rows_q = p->rows_q;
  k.rows_k = p->rows_k;
  k.sq_b = p->q_stride_b;
  k.sq_t = p->q_stride_t;
  k.sq_h = p->q_stride_h;
  k.sk_b = p->k_stride_b;
  k.sk_t = p->k_stride_t;
  k.sk_h = p->k_stride_h;
  k.B = (int)p->B;
  k.H = (int)p->H;
  k.Tq = (int)p->Tq;
  k.Tk = (int)p->Tk;
  k.dmem = (int)p->D;
  return k;
}

// T rows of `stride` 16-bit elements span less than 2^31 bytes.
bool rows_fit_2g(int64_t T, int64_t stride) {
  return stride == 0 || T <= (((int64_t)1 << 30) - 1) / stride;
}

// Every row start 16-byte aligned (strides in elements of `esize` bytes) and
// every row of a sequence within 2^31 bytes of the sequence's first row (the
// tile copies address rows with a 32-bit byte offset from that row).
bool rows_dma_ready(const sigattn_problem *p, const void *const *ptrs, int nptr, int esize) {
  const int64_t per16 = 16 / esize, half_units = esize / 2;
  if (!rows_fit_2g(p->Tq, half_units * p->q_stride_t) || !rows_fit_2g(p->Tk, half_units * p->k_stride_t))
    return false;
  const int64_t strides[6] = {p->q_stride_b, p->q_stride_t, p->q_stride_h,
                              p->k_stride_b, p->k_stride_t, p->k_stride_h};
  for (int64_t s : strides)
    if (s % per16 != 0) return false;
  for (int i = 0; i < nptr; ++i)
    if (ptrs[i] && !aligned16(ptrs[i])) return false;
  return true;
}

// True when the 16-bit MFMA kernels can take the problem: f16 / bf16, D of
// 16, 32, 64 or 128, rows as rows_dma_ready requires.
bool use_mfma(const sigattn_problem *p, const void *const *ptrs, int nptr) {
  if (p->dtype == SIGATTN_F32 || !is_pow2_head_dim(p->D)) return false;
  return rows_dma_ready(p, ptrs, nptr, 2);
}

// True when the fp32 MFMA kernels (v_mfma_f32_32x32x2_f32) can take the
// problem: fp32, D of 16, 32, 64 or 128, rows as rows_dma_ready requires.
bool use_f32_mfma(const sigattn_problem *p, const void *const *ptrs, int nptr) {
  if (p->dtype != SIGATTN_F32 || !is_pow2_head_dim(p->D)) return false;
  return rows_dma_ready(p, ptrs, nptr, 4);
}

// Split-KV forward plan: nsplit = 0 when the main forward kernel takes the
// problem.  Chunks are multiples of 128 keys (four waves of 32-key blocks),
// at least 256 keys, and about SIGATTN_SPLIT_TARGET workgroups in all (no
// split once the (batch, head) pairs alone reach that many).  Measured at
// decode shapes, targets from 256 to 2048 workgroups run within noise of each
// other; 512 keeps the partials small.
struct SplitPlan {
  int nsplit = 0, chunk = 0;
};

#ifndef SIGATTN_SPLIT_TARGET
#define SIGATTN_SPLIT_TARGET 512
#endif

// The split-KV kernel and the two-pass backward exist at D = 64 and 128; at
// D = 16 and 32 the main forward and the recompute backward serve every shape.
bool wide_head(const sigattn_problem *p) { return p->D == 64 || p->D == 128; }

// Head dim of the MFMA kernel instance: head_dim 16 runs in the D = 32
// kernels (KParams::dmem = 16).
int mfma_head_dim(const sigattn_problem *p) { return p->D == 16 ? 32 : (int)p->D; }

SplitPlan splitkv_plan(const sigattn_problem *p, bool mfma) {
  SplitPlan sp;
  if (!mfma || !wide_head(p) || p->causal != 0 || p->Tq > 32 || p->Tk < 256 || p->B * p->H == 0) return sp;
  const int64_t want = cdiv(SIGATTN_SPLIT_TARGET, p->B * p->H);
  const int64_t most = cdiv(p->Tk, 256);
  const int64_t n = want < most ? want : most;
  const int64_t chunk = cdiv(cdiv(p->Tk, n), 128) * 128;
  sp.nsplit = (int)cdiv(p->Tk, chunk);
  sp.chunk = (int)chunk;
  return sp;
}

int64_t splitkv_workspace_bytes(const sigattn_problem *p, const SplitPlan &sp) {
  return sp.nsplit > 1 ? (int64_t)sp.nsplit * p->B * p->H * p->Tq * p->D * (int64_t)sizeof(float) : 0;
}

bool is_ragged(const sigattn_problem *p) {
  return p->seq_lens_q != nullptr || p->seq_lens_k != nullptr || p->cu_seqlens_q != nullptr ||
         p->cu_seqlens_k != nullptr;
}

// The recompute backward's dQ and dK/dV kernels run as one launch
// (launch_bwd_fused_mfma) when the problem is dense, its 16-bit kernel
// instance has D <= 64, and the two grids (128 rows per workgroup) together
// need at most one workgroup per CU: apart, each would leave the CUs the
// other needs idle.
bool fuse_backward(const sigattn_problem *p) {
  if (is_ragged(p) || mfma_head_dim(p) > 64) return false;
  const int64_t cus = sigattn::device_compute_units();
  const int64_t wgs = p->B * p->H * (cdiv(p->Tq, 128) + cdiv(p->Tk, 128));
  return cus > 0 && wgs <= cus;
}

// The recompute backward's dQ and dK/dV kernels run concurrently, dK/dV on a
// second stream, for ragged non-causal problems at head_dim 64 with at least
// eight 128-query blocks per CU: the items of such a grid have the lengths of
// their sequences, so each kernel ends in a drain of unevenly finishing
// workgroups, which the other kernel's workgroups fill.  Measured at B=4
// Lmax=8192 H=12 (seq_lens 1078-5599): 603 -> 577 us.  Dense problems of the
// same shape gain nothing (2876 -> 2879 us), and at B=8 Lmax=2048 H=8 causal,
// padded or dense, both kernels on one stream are faster (103-112 against
// 114-121 us padded), so those stay sequential.
#ifndef SIGATTN_CONCURRENT_BWD
#define SIGATTN_CONCURRENT_BWD 1
#endif
bool concurrent_backward(const sigattn_problem *p) {
  if (!SIGATTN_CONCURRENT_BWD || !is_ragged(p) || p->causal != 0 || mfma_head_dim(p) != 64) return false;
  const int64_t cus = sigattn::device_compute_units();
  return cus > 0 && p->B * p->H * cdiv(p->Tq, 128) >= 8 * cus;
}

// Fork / join of a second stream around the caller's: fork() makes the
// device's side stream (created on first use, default priority, never
// destroyed) wait for the work queued on `st` so far and returns it; join()
// makes `st` wait for the work then queued on the side stream.  The events
// are this host thread's own (a fork records into them and the next fork of
// the same thread may reuse them once its waits are queued), so host threads
// never race on them; threads sharing the side stream only order their
// side-stream work one after the other.  Returns nullptr -- run everything on
// `st` -- under stream capture, when `st` belongs to another device than the
// current one (the side stream is the current device's), or when a runtime
// call fails.
class SideStream {
 public:
  hipStream_t fork(hipStream_t st) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    int dev = -1;
    hipDevice_t sdev = -1;
    if (hipStreamIsCapturing(st, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone ||
        hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices ||
        hipStreamGetDevice(st, &sdev) != hipSuccess || sdev != dev) {
      (void)hipGetLastError();
      return nullptr;
    }
    hipStream_t side = stream(dev);
    Events &ev = events_[dev];
    if (side == nullptr || !ev.ready() || hipEventRecord(ev.fork, st) != hipSuccess ||
        hipStreamWaitEvent(side, ev.fork, 0) != hipSuccess) {
      (void)hipGetLastError();
      return nullptr;
    }
    dev_ = dev;
    return side;
  }
  // Returns false if the join could not be queued (then the caller's stream
  // is not ordered after the side stream's work: an error to report).
  bool join(hipStream_t st, hipStream_t side) {
    Events &ev = events_[dev_];
    return hipEventRecord(ev.join, side) == hipSuccess && hipStreamWaitEvent(st, ev.join, 0) == hipSuccess;
  }

 private:
  static constexpr int kMaxDevices = 64;
  struct Events {
    hipEvent_t fork = nullptr, join = nullptr;
    bool ready() {
      if (fork == nullptr && hipEventCreateWithFlags(&fork, hipEventDisableTiming) != hipSuccess) fork = nullptr;
      if (join == nullptr && hipEventCreateWithFlags(&join, hipEventDisableTiming) != hipSuccess) join = nullptr;
      return fork != nullptr && join != nullptr;
    }
  };
  static hipStream_t stream(int dev) {
    static std::mutex mu;
    static hipStream_t streams[kMaxDevices];
    std::lock_guard<std::mutex> lock(mu);
    if (streams[dev] == nullptr) {
      hipStream_t s = nullptr;
      if (hipStreamCreateWithFlags(&s, hipStreamNonBlocking) != hipSuccess) return nullptr;
      streams[dev] = s;
    }
    return streams[dev];
  }
  Events events_[kMaxDevices];
  int dev_ = 0;
};
thread_local SideStream t_side;

// Fewest rows of the streamed range (keys for the forward and dQ kernels,
// queries for dK/dV) that a range-split chunk takes; chunks of at least twice
// as many may run two workgroups per CU.
#ifndef SIGATTN_RS_MIN_ROWS
#define SIGATTN_RS_MIN_ROWS 512
#endif
// Fewest rows an item's split must save (rows - rows / n, the part of its
// range its slowest chunk no longer streams), by head dim: a split pays only
// when those rows outweigh its hand-over (the partial stores, the release /
// acquire around the arrival counter, the partial loads).  Measured on MI355X
// (fp16 D = 64 / bf16 D = 128 non-causal, us, split vs unsplit): D = 64 saving
// 512 rows lost (B=2 L=1024 H=8, two chunks: forward 19.6 vs 16.2, backward
// 49.6 vs 46.8) and saving 1536 gained (B=1 L=2048 H=4, four chunks: forward
// 22.5 vs 26.4, backward 52.5 vs 80.6); at D = 128, with twice the work per
// row, saving 512 rows gains (B=1 L=1024 H=8: forward 27.0 vs 30.3, backward
// 60.6 vs 68.5).
#ifndef SIGATTN_RS_MIN_SAVED_D64
#define SIGATTN_RS_MIN_SAVED_D64 1024
#endif
#ifndef SIGATTN_RS_MIN_SAVED_D128
#define SIGATTN_RS_MIN_SAVED_D128 512
#endif
int64_t rs_min_saved(int64_t D) { return D == 64 ? SIGATTN_RS_MIN_SAVED_D64 : SIGATTN_RS_MIN_SAVED_D128; }

// Range split of a small dense non-causal grid (KParams::rsplit).  A kernel
// whose `items` workgroups leave at least half of the GPU's CUs idle runs
// each item as n chunks of its streamed range of `rows`: the most chunks,
// up to kRangeSplitMax, that keep every chunk at least SIGATTN_RS_MIN_ROWS
// long, save at least `min_saved` rows per item, and keep the grid within
// one workgroup per CU (two when chunks are at least twice that long, and
// never more than the kernel's `per_cu_max` resident workgroups).  Grids
// filling half the GPU or more measured slower split (B=4 L=1024 H=8 D=64:
// 65.8 -> 80.7 us at n = 2).  Each chunk's partial is `part_floats` fp32 per
// item, and each item has an int counter: the workspace holds the counters
// first (256-byte aligned), then the partials.
struct RangeSplit {
  int n = 1;
  int64_t items = 0, part_floats = 0, cnt_bytes = 0, bytes = 0;
};

RangeSplit range_split(int64_t items, int64_t cus, int64_t per_cu_max, int64_t rows, int64_t part_floats,
                       int64_t min_saved) {
  RangeSplit r;
  if (items <= 0 || cus <= 0 || 2 * items > cus) return r;
  int64_t n = sigattn::kRangeSplitMax;
  for (; n >= 2; --n) {
    if (rows < n * SIGATTN_RS_MIN_ROWS || rows - rows / n < min_saved) continue;
    int64_t per_cu = rows >= 2 * n * SIGATTN_RS_MIN_ROWS ? 2 : 1;
    if (per_cu > per_cu_max) per_cu = per_cu_max;
    if (n * items <= cus * per_cu) break;
  }
  if (n < 2) return r;
  r.n = (int)n;
  r.items = items;
  r.part_floats = part_floats;
  r.cnt_bytes = cdiv(items * (int64_t)sizeof(int), 256) * 256;
  r.bytes = r.cnt_bytes + items * n * part_floats * (int64_t)sizeof(float);
  return r;
}

bool splittable(const sigattn_problem *p, bool mfma) {
  return mfma && wide_head(p) && p->causal == 0 && !is_ragged(p) && p->Tq > 0 && p->Tk > 0 && p->B * p->H > 0;
}

RangeSplit fwd_range_split(const sigattn_problem *p, bool mfma) {
  if (!splittable(p, mfma)) return RangeSplit{};
  const int D = (int)p->D, BM = sigattn::fwd_rows_per_workgroup(D);
  return range_split(p->B * p->H * cdiv(p->Tq, BM), sigattn::device_compute_units(),
                     sigattn::fwd_workgroups_per_cu(D), p->Tk, (int64_t)BM * D, rs_min_saved(D));
}

// The recompute backward's split: the dQ kernel splits keys, the D = 64
// dK/dV kernel queries (the D = 128 one runs unsplit, with one key block per
// workgroup when pairs would not fill the GPU).
struct BwdSplit {
  RangeSplit dq, kv;
  int64_t bytes = 0;
};

BwdSplit bwd_range_split(const sigattn_problem *p, bool mfma) {
  BwdSplit s;
  if (!splittable(p, mfma) || (p->D != 64 && p->D != 128)) return s;
  const int D = (int)p->D, cus = sigattn::device_compute_units();
  const int RQ = sigattn::bwd_dq_rows_per_workgroup(), RK = sigattn::bwd_dkdv_rows_per_workgroup();
  s.dq = range_split(p->B * p->H * cdiv(p->Tq, RQ), cus, sigattn::bwd_dq_workgroups_per_cu(D), p->Tk,
                     (int64_t)RQ * D, rs_min_saved(D));
  if (D == 64)
    s.kv = range_split(p->B * p->H * cdiv(p->Tk, RK), cus, sigattn::bwd_dkdv_workgroups_per_cu(D), p->Tq,
                       2 * (int64_t)RK * D, rs_min_saved(D));
  s.bytes = s.dq.bytes + s.kv.bytes;
  return s;
}

// Sets k's range-split fields for `r` over the workspace at `ws`; the caller
// clears the counters (launch_rs_clear) before k's kernel runs.
void use_range_split(KParams &k, const RangeSplit &r, void *ws) {
  k.rsplit = r.n;
  k.rs_cnt = (int *)ws;
  k.rs_part = (float *)((char *)ws + r.cnt_bytes);
}

// Two-pass backward: bytes of dS tiles (DsLayout) per head, over all batches.
int64_t ds_bytes_per_head(const sigattn_problem *p) {
  const int64_t nqb = cdiv(p->Tq, 32), nkb = cdiv(p->Tk, 32);
  const int64_t tiles = p->causal != 0 ? nqb * (nqb + 1) / 2 : nqb * nkb;
  return p->B * tiles * 2048;
}

// The sub-problem of heads [h0, h0 + nh): every tensor is [.., H, D] with
// its own head stride, so the heads are a pointer offset away; bias,
// score_mod and the sequence lengths are per batch and stay as they are.
KParams head_slice(const KParams &k, int64_t h0, int64_t nh, int64_t esize) {
  KParams s = k;
  const int64_t qo = h0 * k.sq_h * esize, ko = h0 * k.sk_h * esize;
  auto adv = [](const void *ptr, int64_t off) -> const char * {
    return ptr == nullptr ? nullptr : (const char *)ptr + off;
  };
  s.q = adv(k.q, qo);
  s.dout = adv(k.dout, qo);
  s.dq = (void *)adv(k.dq, qo);
  s.k = adv(k.k, ko);
  s.v = adv(k.v, ko);
  s.dk = (void *)adv(k.dk, ko);
  s.dv = (void *)adv(k.dv, ko);
  s.H = (int)nh;
  return s;
}

// Packed layout: zeros on the rows of the outputs that no sequence covers
// (rows before cu_seqlens[0], past cu_seqlens[B], past the longest sequence
// Tq / Tk of a longer one), so every row of a packed output is written.
// q_out is the Q-shaped output (O or dQ), k_out0 / k_out1 the K-shaped ones
// (dK, dV); nullptr skips a tensor.  One launch for both axes, on `st`.
// The packed axes whose output rows outside every sequence must be zeroed:
// a for the Q-shaped output, b for the K-shaped ones (rows = 0: none).
void gap_axes(const sigattn_problem *p, void *q_out, void *k_out0, void *k_out1, sigattn::GapAxis &a,
              sigattn::GapAxis &b) {
  a = b = sigattn::GapAxis{};
  if (p->H == 0) return;
  if (p->cu_seqlens_q != nullptr && q_out != nullptr && p->rows_q > 0) {
    a.cu = p->cu_seqlens_q;
    a.B = (int)p->B, a.T = (int)p->Tq, a.H = (int)p->H, a.D = (int)p->D;
    a.rows = p->rows_q, a.st = p->q_stride_t, a.sh = p->q_stride_h;
    a.out[0] = q_out;
  }
  if (p->cu_seqlens_k != nullptr && (k_out0 != nullptr || k_out1 != nullptr) && p->rows_k > 0) {
    b.cu = p->cu_seqlens_k;
    b.B = (int)p->B, b.T = (int)p->Tk, b.H = (int)p->H, b.D = (int)p->D;
    b.rows = p->rows_k, b.st = p->k_stride_t, b.sh = p->k_stride_h;
    b.out[0] = k_out0, b.out[1] = k_out1;
  }
}

// Zeroes those rows with a launch of their own (paths whose kernels do not
// take KParams::gap, and calls that launch no attention kernel).
void zero_packed_gaps(const sigattn_problem *p, void *q_out, void *k_out0, void *k_out1, hipStream_t st) {
  sigattn::GapAxis a, b;
  gap_axes(p, q_out, k_out0, k_out1, a, b);
  sigattn::launch_zero_gaps(a, b, p->dtype == SIGATTN_F32 ? 4 : 2, st);
}

// Hands axes a and b to the kernel launched with `k` (a forward or dQ
// kernel): its first workgroups, a multiple of 8 per axis, zero the axes'
// gap rows (KParams::gap).
void use_gaps(KParams &k, const sigattn::GapAxis &a, const sigattn::GapAxis &b) {
  const sigattn::GapAxis *ax[2] = {&a, &b};
  for (int i = 0; i < 2; ++i) {
    k.gap[i] = *ax[i];
    k.ngap[i] = ax[i]->rows > 0 ? (int)(cdiv(cdiv(ax[i]->rows, 64), 8) * 8) : 0;
  }
}

int launch_status() {
  return hipGetLastError() == hipSuccess ? SIGATTN_OK : SIGATTN_ERR_LAUNCH;
}

}  // namespace

namespace sigattn {
int device_compute_units() {
  static std::atomic<int> cache[64];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n == 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cache[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}
}  // namespace sigattn

extern "C" {

int sigattn_abi_version(void) { return SIGATTN_ABI_VERSION; }

const char *sigattn_strerror(int status) {
  switch (status) {
    case SIGATTN_OK: return "success";
    case SIGATTN_ERR_NULL_ARG: return "a required pointer argument is NULL";
    case SIGATTN_ERR_DTYPE: return "unsupported dtype code (expected f16, bf16 or f32)";
    case SIGATTN_ERR_HEAD_DIM: return "unsupported head dimension (expected 16, 32, 64 or 128)";
    case SIGATTN_ERR_SHAPE: return "invalid or too large problem shape";
    case SIGATTN_ERR_STRIDE: return "invalid (negative) stride";
    case SIGATTN_ERR_DENSE_LENGTHS:
      return "dense attention (no seq_lens) requires the same sequence length for Q and K";
    case SIGATTN_ERR_ABI_VERSION: return "sigattn_problem.abi_version does not match the library";
    case SIGATTN_ERR_LAUNCH: return "HIP kernel launch or HIP runtime call failed";
    case SIGATTN_ERR_LAYOUT:
      return "seq_lens and cu_seqlens cannot both be given for the same sequence axis";
    case SIGATTN_ERR_WORKSPACE:
      return "workspace too small for the call or not 16-byte aligned";
    case SIGATTN_ERR_SCRATCH:
      return "problem needs more than the fixed scratch buffer of sigattn_fwd_noalloc";
    default: return "unknown sigattn status";
  }
}

int sigattn_check(const sigattn_problem *p) {
  if (p == nullptr) return SIGATTN_ERR_NULL_ARG;
  if (p->abi_version != SIGATTN_ABI_VERSION) return SIGATTN_ERR_ABI_VERSION;
  if (p->dtype != SIGATTN_F16 && p->dtype != SIGATTN_BF16 && p->dtype != SIGATTN_F32)
    return SIGATTN_ERR_DTYPE;
  if (!is_pow2_head_dim(p->D)) return SIGATTN_ERR_HEAD_DIM;
  if (p->B < 0 || p->Tq < 0 || p->Tk < 0 || p->H < 0) return SIGATTN_ERR_SHAPE;
  if (p->rows_q < 0 || p->rows_k < 0) return SIGATTN_ERR_SHAPE;
  if ((p->cu_seqlens_q != nullptr && p->seq_lens_q != nullptr) ||
      (p->cu_seqlens_k != nullptr && p->seq_lens_k != nullptr))
    return SIGATTN_ERR_LAYOUT;
  if (p->Tq > (INT_MAX / 2) || p->Tk > (INT_MAX / 2) || p->B > INT_MAX || p->H > INT_MAX)
    return SIGATTN_ERR_SHAPE;
  // Largest grid any kernel launches: ceil(T / 64) row blocks per (b, h).
  const int64_t rows = p->Tq > p->Tk ? p->Tq : p->Tk;
  if (p->B * p->H > 0 && cdiv(rows, 64) > (int64_t)INT_MAX / (p->B * p->H)) return SIGATTN_ERR_SHAPE;
  const int64_t strides[6] = {p->q_stride_b, p->q_stride_t, p->q_stride_h,
                              p->k_stride_b, p->k_stride_t, p->k_stride_h};
  for (int64_t s : strides)
    if (s < 0) return SIGATTN_ERR_STRIDE;
  if (p->seq_lens_q == nullptr && p->seq_lens_k == nullptr && p->cu_seqlens_q == nullptr &&
      p->cu_seqlens_k == nullptr && p->Tq != p->Tk)
    return SIGATTN_ERR_DENSE_LENGTHS;
  if (p->B == 0 || p->H == 0) return SIGATTN_OK;
  if (p->bias == nullptr || p->scale == nullptr) return SIGATTN_ERR_NULL_ARG;
  if (p->Tq > 0 && p->q == nullptr) return SIGATTN_ERR_NULL_ARG;
  if (p->Tk > 0 && (p->k == nullptr || p->v == nullptr)) return SIGATTN_ERR_NULL_ARG;
  return SIGATTN_OK;
}

size_t sigattn_fwd_workspace_bytes(const sigattn_problem *p) {
  if (sigattn_check(p) != SIGATTN_OK || p->B == 0 || p->H == 0 || p->Tq == 0) return 0;
  // Pointers are not known yet: assume aligned rows (a misaligned call later
  // takes the portable kernel and ignores the workspace).
  const void *none[1] = {nullptr};
  const bool mfma = use_mfma(p, none, 0);
  const SplitPlan sp = splitkv_plan(p, mfma);
  if (sp.nsplit > 0) return (size_t)splitkv_workspace_bytes(p, sp);
  return (size_t)fwd_range_split(p, mfma).bytes;
}

static_assert(sigattn::kSplitScratchBytes == SIGATTN_NOALLOC_SCRATCH_BYTES, "scratch size");

// Forward: the split-KV partials go to `workspace` (caller memory), to the
// library's fixed scratch array (static_scratch), or nowhere (one chunk per
// (batch, head)).  The range split of small dense grids runs only with a
// caller workspace.
static int fwd_impl(const sigattn_problem *p, void *out, void *workspace, size_t workspace_bytes,
                    bool static_scratch, void *stream) {
  const int rc = sigattn_check(p);
  if (rc != SIGATTN_OK) return rc;
  const hipStream_t st = (hipStream_t)stream;
  if (p->B == 0 || p->H == 0 || p->Tq == 0) {
    // Packed rows without any sequence (no batches, or no queries) are all
    // written as zeros.
    if (p->cu_seqlens_q == nullptr || p->H == 0 || p->rows_q == 0) return SIGATTN_OK;
    if (out == nullptr) return SIGATTN_ERR_NULL_ARG;
    (void)hipGetLastError();
    zero_packed_gaps(p, out, nullptr, nullptr, st);
    return launch_status();
  }
  if (out == nullptr) return SIGATTN_ERR_NULL_ARG;
  KParams k = make_params(p);
  k.out = out;
  const void *ptrs[4] = {p->q, p->k, p->v, out};
  const bool mfma = use_mfma(p, ptrs, 4);
  SplitPlan sp = splitkv_plan(p, mfma);
  if (sp.nsplit > 1 && static_scratch) {
    if ((size_t)splitkv_workspace_bytes(p, sp) > sigattn::kSplitScratchBytes) return SIGATTN_ERR_SCRATCH;
    float *ws = nullptr;
    if (sigattn::splitkv_scratch(&ws) != hipSuccess) return SIGATTN_ERR_LAUNCH;
    k.ws = ws;
  } else if (sp.nsplit > 1 && workspace != nullptr) {
    if ((size_t)splitkv_workspace_bytes(p, sp) > workspace_bytes || !aligned16(workspace))
      return SIGATTN_ERR_WORKSPACE;
    k.ws = (float *)workspace;
  } else if (sp.nsplit > 1) {
    sp.nsplit = 1;  // no workspace: one chunk per (batch, head), written directly
    sp.chunk = (int)(cdiv(p->Tk, 128) * 128);
  }
  // The range split is an optimisation the caller need not know about: a
  // workspace that cannot hold its partials (one sized for split-KV decode,
  // say) or that is misaligned runs the problem unsplit, as sigattn_fwd does.
  RangeSplit rs;
  if (sp.nsplit == 0 && workspace != nullptr && !static_scratch) {
    rs = fwd_range_split(p, mfma);
    if (rs.n > 1 && ((size_t)rs.bytes > workspace_bytes || !aligned16(workspace))) rs = RangeSplit{};
  }
  (void)hipGetLastError();
  // Packed rows outside every sequence: zeroed by the MFMA forward's leading
  // workgroups, by a launch of their own on the other paths.
  const bool f32mma = use_f32_mfma(p, ptrs, 4);
  if (sp.nsplit == 0 && (mfma || f32mma)) {
    sigattn::GapAxis gq, gk;
    gap_axes(p, out, nullptr, nullptr, gq, gk);
    use_gaps(k, gq, gk);
  } else {
    zero_packed_gaps(p, out, nullptr, nullptr, st);
  }
  if (rs.n > 1) {
    use_range_split(k, rs, workspace);
    sigattn::launch_rs_clear(k.rs_cnt, (int)rs.items, nullptr, 0, st);
  }
  if (sp.nsplit > 0) {
    k.nsplit = sp.nsplit;
    k.chunk = sp.chunk;
    sigattn::launch_fwd_splitkv(k, p->dtype, (int)p->D, p->score_mod != nullptr, st);
  } else if (mfma) {
    sigattn::launch_fwd_mfma(k, p->dtype, mfma_head_dim(p), p->causal != 0, p->score_mod != nullptr, st);
  } else if (f32mma) {
    sigattn::launch_fwd_f32(k, mfma_head_dim(p), p->causal != 0, p->score_mod != nullptr, st);
  } else {
    sigattn::launch_fwd_generic(k, p->dtype, (int)p->D, p->causal != 0, st);
  }
  return launch_status();
}

int sigattn_fwd_ws(const sigattn_problem *p, void *out, void *workspace, size_t workspace_bytes,
                   void *stream) {
  return fwd_impl(p, out, workspace, workspace_bytes, false, stream);
}

int sigattn_fwd(const sigattn_problem *p, void *out, void *stream) {
  return fwd_impl(p, out, nullptr, 0, false, stream);
}

int sigattn_fwd_noalloc(const sigattn_problem *p, void *out, void *stream) {
  return fwd_impl(p, out, nullptr, 0, true, stream);
}

// Which kernels a backward call runs.
enum BwdParts { kBwdAll, kBwdDq, kBwdDkdv };

static int bwd_impl(const sigattn_problem *p, const void *dout, void *dq, void *dk, void *dv,
                    void *workspace, size_t workspace_bytes, void *stream, BwdParts parts) {
  const int rc = sigattn_check(p);
  if (rc != SIGATTN_OK) return rc;
  if (workspace != nullptr && !aligned16(workspace)) return SIGATTN_ERR_WORKSPACE;
  if (p->H == 0) return SIGATTN_OK;
  if (p->B == 0) {
    // Packed rows without any sequence are all written as zeros.
    const bool rows_q = p->cu_seqlens_q != nullptr && p->rows_q > 0;
    const bool rows_k = p->cu_seqlens_k != nullptr && p->rows_k > 0;
    if (!rows_q && !rows_k) return SIGATTN_OK;
    void *zq = parts != kBwdDkdv ? dq : nullptr;
    void *zk = parts != kBwdDq ? dk : nullptr, *zv = parts != kBwdDq ? dv : nullptr;
    (void)hipGetLastError();
    zero_packed_gaps(p, zq, zk, zv, (hipStream_t)stream);
    return launch_status();
  }
  const bool need_dq = parts != kBwdDkdv && p->Tq > 0;
  const bool need_dkdv = parts != kBwdDq && p->Tk > 0;
  const void *ptrs[7] = {p->q, p->k, p->v, dout, dq, dk, dv};
  const bool mfma = use_mfma(p, ptrs, 7);
  const bool f32mma = use_f32_mfma(p, ptrs, 7);

  // Two-pass backward when a workspace holds the dS of at least one head.
  // The halves (kBwdDq, kBwdDkdv) need the whole problem's dS at once: the
  // dQ half reads what a dK/dV half with the same workspace stored.
  int64_t heads_per_pass = 0;
  if (workspace != nullptr && mfma && wide_head(p) && p->Tq > 0 && p->Tk > 0) {
    heads_per_pass = (int64_t)workspace_bytes / ds_bytes_per_head(p);
    if (heads_per_pass > p->H) heads_per_pass = p->H;
  }
  if (parts != kBwdAll && workspace != nullptr) {
    if (!mfma || !wide_head(p)) return SIGATTN_ERR_WORKSPACE;  // no two-pass kernels for this problem
    if (p->Tq > 0 && p->Tk > 0 && heads_per_pass < p->H) return SIGATTN_ERR_WORKSPACE;
  }
  const bool twopass = heads_per_pass > 0;

  if (need_dq && dq == nullptr) return SIGATTN_ERR_NULL_ARG;
  if (need_dkdv && (dk == nullptr || dv == nullptr)) return SIGATTN_ERR_NULL_ARG;
  // dO feeds every kernel except the dQ-from-dS one.
  const bool need_dout = need_dkdv || (need_dq && !(twopass && parts == kBwdDq));
  if (need_dout && p->Tq > 0 && dout == nullptr) return SIGATTN_ERR_NULL_ARG;

  KParams k = make_params(p);
  k.dout = dout;
  k.dq = dq;
  k.dk = dk;
  k.dv = dv;
  const hipStream_t st = (hipStream_t)stream;
  const bool causal = p->causal != 0, sm = p->score_mod != nullptr;
  const int dt = p->dtype, D = mfma || f32mma ? mfma_head_dim(p) : (int)p->D;
  (void)hipGetLastError();
  // Packed rows outside every sequence: zeroed, for dQ and dK / dV alike, by
  // the leading workgroups of the MFMA dQ launch (whose kernels have the
  // registers to spare; in the dK/dV kernel at D = 64 the extra code path
  // pushed spills into the main loop), by a launch of their own when the
  // portable kernels run or no dQ kernel does.
  sigattn::GapAxis gq, gk;
  gap_axes(p, parts != kBwdDkdv ? dq : nullptr, parts != kBwdDq ? dk : nullptr, parts != kBwdDq ? dv : nullptr, gq,
           gk);
  const bool dq_gaps = (mfma || f32mma) && need_dq;
  if (!dq_gaps) sigattn::launch_zero_gaps(gq, gk, dt == SIGATTN_F32 ? 4 : 2, st);
  if (twopass) {
    k.ds = (uint16_t *)workspace;
    k.ds_nqb = (int)cdiv(p->Tq, 32);
    k.ds_nkb = (int)cdiv(p->Tk, 32);
    // Per head group: dK/dV (storing dS), then dQ from dS, on one stream, so
    // the next group's dK/dV overwrites the workspace only after this
    // group's dQ has read it.
    for (int64_t h0 = 0; h0 < p->H; h0 += heads_per_pass) {
      const int64_t nh = p->H - h0 < heads_per_pass ? p->H - h0 : heads_per_pass;
      KParams s = head_slice(k, h0, nh, 2);
      if (parts != kBwdDq) sigattn::launch_bwd_dkdv_mfma(s, dt, D, causal, sm, true, st);
      if (h0 == 0 && dq_gaps) use_gaps(s, gq, gk);  // the first group's dQ launch
      if (parts != kBwdDkdv) sigattn::launch_bwd_dq_ds_mfma(s, dt, D, causal, st);
    }
    return launch_status();
  }
  // Recompute backward.  The two kernels are independent (the sigmoid's
  // backward needs no forward statistics): one launch on small dense grids
  // (fuse_backward), concurrently on two streams for large ragged non-causal
  // ones (concurrent_backward), else one after the other on the caller's
  // stream -- each then fills the GPU on its own, and concurrent launches
  // measured slower there.
  if (need_dq && need_dkdv && mfma && fuse_backward(p)) {
    sigattn::launch_bwd_fused_mfma(k, dt, D, causal, sm, st);
    return launch_status();
  }
  // Concurrent: the dK/dV kernel (the longer one) is queued first, on the
  // side stream, then the dQ kernel on the caller's.
  hipStream_t side = nullptr;
  if (need_dq && need_dkdv && mfma && concurrent_backward(p)) side = t_side.fork(st);
  if (side != nullptr) sigattn::launch_bwd_dkdv_mfma(k, dt, D, causal, sm, false, side);
  KParams kq = k;
  if (dq_gaps) use_gaps(kq, gq, gk);
  if (need_dq) {
    if (mfma) sigattn::launch_bwd_dq_mfma(kq, dt, D, causal, sm, st);
    else if (f32mma) sigattn::launch_bwd_dq_f32(kq, D, causal, sm, st);
    else sigattn::launch_bwd_dq_generic(k, dt, D, causal, st);
  }
  if (need_dkdv && side == nullptr) {
    if (mfma) sigattn::launch_bwd_dkdv_mfma(k, dt, D, causal, sm, false, st);
    else if (f32mma) sigattn::launch_bwd_dkdv_f32(k, D, causal, sm, st);
    else sigattn::launch_bwd_dkdv_generic(k, dt, D, causal, st);
  }
  if (side != nullptr && !t_side.join(st, side)) return SIGATTN_ERR_LAUNCH;
  return launch_status();
}

size_t sigattn_bwd_workspace_bytes(const sigattn_problem *p) {
  if (sigattn_check(p) != SIGATTN_OK || p->B == 0 || p->H == 0 || p->Tq == 0 || p->Tk == 0) return 0;
  const void *none[1] = {nullptr};
  if (!use_mfma(p, none, 0) || !wide_head(p)) return 0;
  return (size_t)(ds_bytes_per_head(p) * p->H);
}

int sigattn_bwd_ws(const sigattn_problem *p, const void *dout, void *dq, void *dk, void *dv,
                   void *workspace, size_t workspace_bytes, void *stream) {
  return bwd_impl(p, dout, dq, dk, dv, workspace, workspace_bytes, stream, kBwdAll);
}

int sigattn_bwd(const sigattn_problem *p, const void *dout, void *dq, void *dk, void *dv,
                void *stream) {
  return bwd_impl(p, dout, dq, dk, dv, nullptr, 0, stream, kBwdAll);
}

size_t sigattn_bwd_split_workspace_bytes(const sigattn_problem *p) {
  if (sigattn_check(p) != SIGATTN_OK || p->B == 0 || p->H == 0) return 0;
  const void *none[1] = {nullptr};
  return (size_t)bwd_range_split(p, use_mfma(p, none, 0)).bytes;
}

int sigattn_bwd_split(const sigattn_problem *p, const void *dout, void *dq, void *dk, void *dv,
                      void *workspace, size_t workspace_bytes, void *stream) {
  const int rc = sigattn_check(p);
  if (rc != SIGATTN_OK) return rc;
  if (p->B == 0 || p->H == 0) return SIGATTN_OK;
  // dq alone, or dk and dv alone, ask for that half of the backward.
  const bool want_dq = dq != nullptr, want_kv = dk != nullptr || dv != nullptr;
  if (!want_dq && !want_kv) return SIGATTN_ERR_NULL_ARG;
  if (want_kv && (dk == nullptr || dv == nullptr)) return SIGATTN_ERR_NULL_ARG;
  const BwdParts parts = want_dq && want_kv ? kBwdAll : (want_dq ? kBwdDq : kBwdDkdv);
  const void *ptrs[7] = {p->q, p->k, p->v, dout, dq, dk, dv};
  const BwdSplit bs = workspace != nullptr ? bwd_range_split(p, use_mfma(p, ptrs, 7)) : BwdSplit{};
  if (bs.bytes == 0) return bwd_impl(p, dout, dq, dk, dv, nullptr, 0, stream, parts);
  if ((size_t)bs.bytes > workspace_bytes || !aligned16(workspace)) return SIGATTN_ERR_WORKSPACE;
  if (dout == nullptr) return SIGATTN_ERR_NULL_ARG;
  KParams k = make_params(p);
  k.dout = dout;
  k.dq = dq;
  k.dk = dk;
  k.dv = dv;
  const hipStream_t st = (hipStream_t)stream;
  const bool sm = p->score_mod != nullptr;
  (void)hipGetLastError();
  // Both kernels' counters are cleared by one launch ahead of them.
  KParams kq = k, kk = k;
  if (want_dq && bs.dq.n > 1) use_range_split(kq, bs.dq, workspace);
  if (want_kv && bs.kv.n > 1) use_range_split(kk, bs.kv, (char *)workspace + bs.dq.bytes);
  sigattn::launch_rs_clear(kq.rs_cnt, kq.rsplit > 1 ? (int)bs.dq.items : 0, kk.rs_cnt,
                           kk.rsplit > 1 ? (int)bs.kv.items : 0, st);
  if (want_dq) sigattn::launch_bwd_dq_mfma(kq, p->dtype, (int)p->D, false, sm, st);
  if (want_kv) sigattn::launch_bwd_dkdv_mfma(kk, p->dtype, (int)p->D, false, sm, false, st);
  return launch_status();
}

int sigattn_bwd_dq(const sigattn_problem *p, const void *dout, void *dq, void *stream) {
  return bwd_impl(p, dout, dq, nullptr, nullptr, nullptr, 0, stream, kBwdDq);
}

int sigattn_bwd_dkdv(const sigattn_problem *p, const void *dout, void *dk, void *dv,
                     void *stream) {
  return bwd_impl(p, dout, nullptr, dk, dv, nullptr, 0, stream, kBwdDkdv);
}

int sigattn_bwd_dkdv_ws(const sigattn_problem *p, const void *dout, void *dk, void *dv,
                        void *workspace, size_t workspace_bytes, void *stream) {
  if (workspace == nullptr) return SIGATTN_ERR_WORKSPACE;
  return bwd_impl(p, dout, nullptr, dk, dv, workspace, workspace_bytes, stream, kBwdDkdv);
}

int sigattn_bwd_dq_ws(const sigattn_problem *p, void *dq, const void *workspace,
                      size_t workspace_bytes, void *stream) {
  if (workspace == nullptr) return SIGATTN_ERR_WORKSPACE;
  return bwd_impl(p, nullptr, dq, nullptr, nullptr, (void *)workspace, workspace_bytes, stream,
                  kBwdDq);
}

}  // extern "C"
