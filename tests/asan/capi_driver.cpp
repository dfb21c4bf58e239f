// Host-only driver for the address/undefined-behaviour sanitizer build of
// csrc/capi.cpp (the C ABI's validation and dispatch).  The kernel launchers
// are replaced by recorders, and hipGetLastError by a stub, so the program
// needs no GPU and no HIP runtime initialisation: every call either returns
// a validation error before any launch or records which launchers a valid
// problem reaches.  Built and run by tests/test_capi_asan_cpu.py.
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

#include "launch.h"
#include "sigattn.h"

namespace {
std::vector<std::string> g_calls;
std::vector<sigattn::KParams> g_hist;  // parameters of each launch since the last calls()
sigattn::KParams g_last{};
int g_D = 0;  // head dim passed to the last kernel launch
hipStream_t g_dq_stream = nullptr, g_dkdv_stream = nullptr;  // streams of the last dQ / dK/dV launches
int g_fail = 0;

void record(const char *name, const sigattn::KParams &p) {
  g_calls.emplace_back(name);
  g_hist.push_back(p);
  g_last = p;
}

#define EXPECT(cond)                                                        \
  do {                                                                      \
    if (!(cond)) {                                                          \
      std::fprintf(stderr, "%s:%d: expectation failed: %s\n", __FILE__, __LINE__, #cond); \
      ++g_fail;                                                             \
    }                                                                       \
  } while (0)

// Device pointers are never dereferenced on the host: any aligned address.
void *const kFake = reinterpret_cast<void *>(uintptr_t(1) << 20);

sigattn_problem base(int64_t B = 2, int64_t T = 16, int64_t H = 2, int64_t D = 64) {
  sigattn_problem p;
  std::memset(&p, 0, sizeof p);
  p.abi_version = SIGATTN_ABI_VERSION;
  p.dtype = SIGATTN_BF16;
  p.B = B, p.Tq = T, p.Tk = T, p.H = H, p.D = D;
  p.q_stride_b = p.k_stride_b = T * H * D;
  p.q_stride_t = p.k_stride_t = H * D;
  p.q_stride_h = p.k_stride_h = D;
  p.q = p.k = p.v = kFake;
  p.bias = p.scale = static_cast<const float *>(kFake);
  return p;
}

std::string calls() {
  std::string s;
  for (auto &c : g_calls) s += (s.empty() ? "" : ",") + c;
  g_calls.clear();
  return s;
}

// Launch i since the previous calls() zeroes gap rows in leading workgroups
// (a multiple of 8 per axis): rq rows of the Q-shaped output q, rk rows of
// the K-shaped outputs k0, k1 (0 rows: none for that axis).
bool gaps_at(size_t i, int64_t rq, const void *q, int64_t rk = 0, const void *k0 = nullptr,
             const void *k1 = nullptr) {
  if (i >= g_hist.size()) return false;
  const sigattn::KParams &k = g_hist[i];
  const auto axis = [&](int a, int64_t rows, const void *o0, const void *o1) {
    if (rows == 0) return k.ngap[a] == 0;
    return k.gap[a].rows == rows && k.ngap[a] == (int)(((rows + 63) / 64 + 7) / 8 * 8) &&
           k.gap[a].out[0] == o0 && k.gap[a].out[1] == o1;
  };
  return axis(0, rq, q, nullptr) && axis(1, rk, k0, k1);
}
}  // namespace

namespace sigattn {
void launch_fwd_mfma(const KParams &p, int, int D, bool, bool, hipStream_t) {
  g_D = D;
  record("fwd_mfma", p);
}
void launch_bwd_dq_mfma(const KParams &p, int, int D, bool, bool, hipStream_t st) {
  g_D = D;
  g_dq_stream = st;
  record("dq_mfma", p);
}
void launch_bwd_dkdv_mfma(const KParams &p, int, int D, bool, bool, bool dsout, hipStream_t st) {
  g_D = D;
  g_dkdv_stream = st;
  record(dsout ? "dkdv_mfma_ds" : "dkdv_mfma", p);
}
void launch_bwd_dq_ds_mfma(const KParams &p, int, int, bool, hipStream_t) { record("dq_ds", p); }
void launch_bwd_fused_mfma(const KParams &p, int, int D, bool, bool, hipStream_t) {
  g_D = D;
  record("bwd_fused", p);
}
void launch_fwd_splitkv(const KParams &p, int, int, bool, hipStream_t) { record("fwd_splitkv", p); }
void launch_fwd_f32(const KParams &p, int D, bool, bool, hipStream_t) {
  g_D = D;
  record("fwd_f32", p);
}
void launch_bwd_dq_f32(const KParams &p, int D, bool, bool, hipStream_t) {
  g_D = D;
  record("dq_f32", p);
}
void launch_bwd_dkdv_f32(const KParams &p, int D, bool, bool, hipStream_t) {
  g_D = D;
  record("dkdv_f32", p);
}
void launch_fwd_generic(const KParams &p, int, int D, bool, hipStream_t) {
  g_D = D;
  record("fwd_generic", p);
}
void launch_bwd_dq_generic(const KParams &p, int, int D, bool, hipStream_t) {
  g_D = D;
  record("dq_generic", p);
}
void launch_bwd_dkdv_generic(const KParams &p, int, int D, bool, hipStream_t) {
  g_D = D;
  record("dkdv_generic", p);
}
int fwd_rows_per_workgroup(int D) { return (D == 64 ? 4 : 8) * 32; }
int fwd_workgroups_per_cu(int D) { return D == 64 ? 3 : 1; }
int bwd_dq_rows_per_workgroup() { return 128; }
int bwd_dkdv_rows_per_workgroup() { return 128; }
int bwd_dq_workgroups_per_cu(int D) { return D == 64 ? 3 : 2; }
int bwd_dkdv_workgroups_per_cu(int D) { return D == 64 ? 2 : 1; }
void launch_rs_clear(int *, int na, int *, int nb, hipStream_t) {
  if (na + nb > 0) g_calls.emplace_back("rs_clear");
}
GapAxis g_gap[2];
void launch_zero_gaps(const GapAxis &a, const GapAxis &b, int, hipStream_t) {
  if (a.rows + b.rows > 0) {
    g_calls.emplace_back("zero_gaps");
    g_gap[0] = a, g_gap[1] = b;
  }
}
// The fixed scratch of sigattn_fwd_noalloc: any aligned address stands in.
hipError_t splitkv_scratch(float **ptr) {
  *ptr = reinterpret_cast<float *>(uintptr_t(3) << 20);
  return hipSuccess;
}
}  // namespace sigattn

// The library maps hipGetLastError() after its launches; no launch happens here.
extern "C" hipError_t hipGetLastError(void) { return hipSuccess; }
// The device the range split sizes itself for: none until g_cus is set.
static int g_cus = 0;
extern "C" hipError_t hipGetDevice(int *dev) {
  *dev = 0;
  return g_cus > 0 ? hipSuccess : hipErrorNoDevice;
}
extern "C" hipError_t hipDeviceGetAttribute(int *value, hipDeviceAttribute_t, int) {
  *value = g_cus;
  return hipSuccess;
}
// The concurrent backward's second stream and its fork / join events: fake
// handles, every record and wait logged as "record <event> <stream>" /
// "wait <stream> <event>" (handles as small numbers; stream 0 = the caller's
// null stream), and a capture status the checks set.
static hipStreamCaptureStatus g_capture = hipStreamCaptureStatusNone;
static int g_nevents = 0;
static std::vector<std::string> g_sync;
static const hipStream_t kSide = (hipStream_t)(uintptr_t)0x5100;
static std::string handle(const void *h) { return std::to_string((unsigned long)(uintptr_t)h); }
extern "C" hipError_t hipStreamIsCapturing(hipStream_t, hipStreamCaptureStatus *status) {
  *status = g_capture;
  return hipSuccess;
}
// Streams belong to device 0, except kOtherDevice.
static const hipStream_t kOtherDevice = (hipStream_t)(uintptr_t)0x7700;
extern "C" hipError_t hipStreamGetDevice(hipStream_t stream, hipDevice_t *device) {
  *device = stream == kOtherDevice ? 1 : 0;
  return hipSuccess;
}
extern "C" hipError_t hipStreamCreateWithFlags(hipStream_t *stream, unsigned int) {
  *stream = kSide;
  return hipSuccess;
}
extern "C" hipError_t hipEventCreateWithFlags(hipEvent_t *event, unsigned) {
  *event = (hipEvent_t)(uintptr_t)(0x100 + ++g_nevents);
  return hipSuccess;
}
extern "C" hipError_t hipEventRecord(hipEvent_t event, hipStream_t stream) {
  g_sync.push_back("record " + handle(event) + " " + handle(stream));
  return hipSuccess;
}
extern "C" hipError_t hipStreamWaitEvent(hipStream_t stream, hipEvent_t event, unsigned int) {
  g_sync.push_back("wait " + handle(stream) + " " + handle(event));
  return hipSuccess;
}
static std::string sync_log() {
  std::string s;
  for (auto &c : g_sync) s += (s.empty() ? "" : ";") + c;
  g_sync.clear();
  return s;
}

// The fp32 kernels' LDS tiles (32 rows x D floats, four waves copying): the
// tile copies place each global element exactly once, at the offset
// F32Tile<D>::elem reads it from; F32RowReads<D> agrees with elem for every
// lane and (g, r, db); the head-dim products' 16-byte reads of 16
// consecutive rows at one piece position fall in 16 different bank groups
// (64 banks of 4 bytes); with half rows (head_dim 16 in the D = 32 tiles)
// the upper 16 columns repeat the lower 16.
template <int D> void check_f32_tiles() {
  using sigattn::DmaPlan;
  using sigattn::F32RowReads;
  using sigattn::F32Tile;
  constexpr int ROWS = 32, CPR = D / 4;
  for (int half = 0; half < (D == 32 ? 2 : 1); ++half) {
    std::vector<int> src(ROWS * D, -1);  // LDS float -> global (row, column) it holds
    for (int w = 0; w < 4; ++w)
      for (int lane = 0; lane < 64; ++lane) {
        DmaPlan<ROWS, 2 * D, 4> dp;
        dp.init(w, lane, half != 0);
        for (int i = 0; i < DmaPlan<ROWS, 2 * D, 4>::NI; ++i) {
          const int row = dp.r0[i] + lane / CPR, slot = lane % CPR;
          EXPECT(row == dp.row[i] && dp.cbyte[i] % 16 == 0);
          for (int e = 0; e < 4; ++e) {
            const int at = row * D + 4 * slot + e;
            EXPECT(src[at] == -1);
            src[at] = row * D + 4 * (dp.cbyte[i] / 16) + e;
          }
        }
      }
    for (int r = 0; r < ROWS; ++r)
      for (int d = 0; d < D; ++d) {
        const int want = r * D + (half ? d % 16 : d);
        EXPECT(src[F32Tile<D>::elem(r, d)] == want);
      }
  }
  for (int lane = 0; lane < 64; ++lane) {
    F32RowReads<D> rr;
    rr.init(lane & 31, lane >> 5);
    for (int g = 0; g < 4; ++g)
      for (int r = 0; r < 4; ++r)
        for (int db = 0; db < D / 32; ++db)
          EXPECT(rr.at(g, r, db) == F32Tile<D>::elem(8 * g + 4 * (lane >> 5) + r, 32 * db + (lane & 31)));
  }
  for (int r0 = 0; r0 < ROWS; r0 += 16)
    for (int c = 0; c < CPR; ++c) {
      unsigned groups = 0;
      for (int r = r0; r < r0 + 16; ++r) groups |= 1u << ((F32Tile<D>::piece(r, c) / 4) % 16);
      EXPECT(groups == 0xffffu);
    }
}

int main() {
  check_f32_tiles<32>();
  check_f32_tiles<64>();
  check_f32_tiles<128>();

  // --- validation: the error codes of tests/test_capi_cpu.py, for every entry point
  struct Bad {
    const char *what;
    void (*change)(sigattn_problem &);
    int code;
  } bad[] = {
      {"abi", [](sigattn_problem &p) { p.abi_version = 99; }, SIGATTN_ERR_ABI_VERSION},
      {"dtype", [](sigattn_problem &p) { p.dtype = 7; }, SIGATTN_ERR_DTYPE},
      {"D48", [](sigattn_problem &p) { p.D = 48; }, SIGATTN_ERR_HEAD_DIM},
      {"D256", [](sigattn_problem &p) { p.D = 256; }, SIGATTN_ERR_HEAD_DIM},
      {"B<0", [](sigattn_problem &p) { p.B = -1; }, SIGATTN_ERR_SHAPE},
      {"Tq huge", [](sigattn_problem &p) { p.Tq = int64_t(1) << 40; }, SIGATTN_ERR_SHAPE},
      {"BH grid", [](sigattn_problem &p) { p.B = p.H = int64_t(1) << 30; }, SIGATTN_ERR_SHAPE},
      {"stride", [](sigattn_problem &p) { p.k_stride_t = -5; }, SIGATTN_ERR_STRIDE},
      {"dense Tq!=Tk", [](sigattn_problem &p) { p.Tk = 8; }, SIGATTN_ERR_DENSE_LENGTHS},
      {"rows<0", [](sigattn_problem &p) { p.rows_q = -1, p.cu_seqlens_q = (const int32_t *)kFake; },
       SIGATTN_ERR_SHAPE},
      {"layout q", [](sigattn_problem &p) {
         p.cu_seqlens_q = (const int32_t *)kFake, p.seq_lens_q = (const int32_t *)kFake; }, SIGATTN_ERR_LAYOUT},
      {"layout k", [](sigattn_problem &p) {
         p.cu_seqlens_k = (const int32_t *)kFake, p.seq_lens_k = (const int32_t *)kFake; }, SIGATTN_ERR_LAYOUT},
      {"bias", [](sigattn_problem &p) { p.bias = nullptr; }, SIGATTN_ERR_NULL_ARG},
      {"scale", [](sigattn_problem &p) { p.scale = nullptr; }, SIGATTN_ERR_NULL_ARG},
      {"q", [](sigattn_problem &p) { p.q = nullptr; }, SIGATTN_ERR_NULL_ARG},
      {"v", [](sigattn_problem &p) { p.v = nullptr; }, SIGATTN_ERR_NULL_ARG},
  };
  for (const Bad &b : bad) {
    sigattn_problem p = base();
    b.change(p);
    EXPECT(sigattn_check(&p) == b.code);
    EXPECT(sigattn_fwd(&p, kFake, nullptr) == b.code);
    EXPECT(sigattn_fwd_ws(&p, kFake, kFake, 1 << 20, nullptr) == b.code);
    EXPECT(sigattn_fwd_noalloc(&p, kFake, nullptr) == b.code);
    EXPECT(sigattn_bwd(&p, kFake, kFake, kFake, kFake, nullptr) == b.code);
    EXPECT(sigattn_bwd_ws(&p, kFake, kFake, kFake, kFake, kFake, 1 << 20, nullptr) == b.code);
    EXPECT(sigattn_bwd_dq(&p, kFake, kFake, nullptr) == b.code);
    EXPECT(sigattn_bwd_dkdv(&p, kFake, kFake, kFake, nullptr) == b.code);
    EXPECT(sigattn_fwd_workspace_bytes(&p) == 0);
    EXPECT(sigattn_bwd_workspace_bytes(&p) == 0);
    if (!g_calls.empty()) std::fprintf(stderr, "case %s launched %s\n", b.what, calls().c_str());
  }
  EXPECT(sigattn_check(nullptr) == SIGATTN_ERR_NULL_ARG);
  EXPECT(sigattn_fwd(nullptr, kFake, nullptr) == SIGATTN_ERR_NULL_ARG);
  EXPECT(sigattn_bwd(nullptr, kFake, kFake, kFake, kFake, nullptr) == SIGATTN_ERR_NULL_ARG);
  EXPECT(sigattn_fwd_workspace_bytes(nullptr) == 0 && sigattn_bwd_workspace_bytes(nullptr) == 0);
  {
    sigattn_problem p = base();
    EXPECT(sigattn_fwd(&p, nullptr, nullptr) == SIGATTN_ERR_NULL_ARG);
    EXPECT(sigattn_bwd(&p, kFake, nullptr, kFake, kFake, nullptr) == SIGATTN_ERR_NULL_ARG);
    EXPECT(sigattn_bwd(&p, nullptr, kFake, kFake, kFake, nullptr) == SIGATTN_ERR_NULL_ARG);
    EXPECT(sigattn_bwd_dkdv_ws(&p, kFake, kFake, kFake, nullptr, 1 << 20, nullptr) == SIGATTN_ERR_WORKSPACE);
    EXPECT(sigattn_bwd_dq_ws(&p, kFake, nullptr, 1 << 20, nullptr) == SIGATTN_ERR_WORKSPACE);
    EXPECT(g_calls.empty());
  }
  for (int code = -11; code <= 0; ++code) EXPECT(std::strlen(sigattn_strerror(code)) > 0);
  EXPECT(std::strcmp(sigattn_strerror(-99), "unknown sigattn status") == 0);

  // --- dispatch of valid problems
  {
    sigattn_problem p = base(2, 300, 3, 128);
    p.causal = 1;
    EXPECT(sigattn_fwd(&p, kFake, nullptr) == 0 && calls() == "fwd_mfma");
    EXPECT(g_last.B == 2 && g_last.H == 3 && g_last.Tq == 300 && g_last.out == kFake);
    EXPECT(sigattn_bwd(&p, kFake, kFake, kFake, kFake, nullptr) == 0 && calls() == "dq_mfma,dkdv_mfma");
    const size_t ws = sigattn_bwd_workspace_bytes(&p);
    EXPECT(ws == size_t(2) * 3 * (10 * 11 / 2) * 2048);
    EXPECT(sigattn_bwd_ws(&p, kFake, kFake, kFake, kFake, kFake, ws, nullptr) == 0 &&
           calls() == "dkdv_mfma_ds,dq_ds");
    // Room for one head: three head groups, each dK/dV then dQ.
    EXPECT(sigattn_bwd_ws(&p, kFake, kFake, kFake, kFake, kFake, ws / 3, nullptr) == 0 &&
           calls() == "dkdv_mfma_ds,dq_ds,dkdv_mfma_ds,dq_ds,dkdv_mfma_ds,dq_ds");
    EXPECT(g_last.H == 1 && g_last.ds_nqb == 10 && g_last.ds_nkb == 10);
    // Less than one head: the recompute kernels.
    EXPECT(sigattn_bwd_ws(&p, kFake, kFake, kFake, kFake, kFake, ws / 3 - 16, nullptr) == 0 &&
           calls() == "dq_mfma,dkdv_mfma");
    EXPECT(sigattn_bwd_ws(&p, kFake, kFake, kFake, kFake, (char *)kFake + 8, ws, nullptr) ==
           SIGATTN_ERR_WORKSPACE);
    EXPECT(sigattn_bwd_dkdv_ws(&p, kFake, kFake, kFake, kFake, ws - 1, nullptr) == SIGATTN_ERR_WORKSPACE);
    EXPECT(g_calls.empty());
  }
  {
    // D = 32 in bf16: the MFMA kernels, recompute backward (no two-pass workspace).
    sigattn_problem p = base(1, 40, 1, 32);
    EXPECT(sigattn_fwd(&p, kFake, nullptr) == 0 && calls() == "fwd_mfma" && g_D == 32 && g_last.dmem == 32);
    EXPECT(sigattn_bwd_workspace_bytes(&p) == 0);
    EXPECT(sigattn_bwd(&p, kFake, kFake, kFake, kFake, nullptr) == 0 && calls() == "dq_mfma,dkdv_mfma");
    // D = 16 in bf16: the D = 32 kernels on 16-column rows.
    p = base(1, 40, 2, 16);
    EXPECT(sigattn_fwd(&p, kFake, nullptr) == 0 && calls() == "fwd_mfma" && g_D == 32 && g_last.dmem == 16);
    EXPECT(sigattn_bwd_workspace_bytes(&p) == 0 && sigattn_fwd_workspace_bytes(&p) == 0);
    EXPECT(sigattn_bwd(&p, kFake, kFake, kFake, kFake, nullptr) == 0 && calls() == "dq_mfma,dkdv_mfma" &&
           g_D == 32 && g_last.dmem == 16);
    // fp32 at D = 16: the fp32 MFMA kernels' D = 32 instances, likewise.
    p.dtype = SIGATTN_F32;
    EXPECT(sigattn_fwd(&p, kFake, nullptr) == 0 && calls() == "fwd_f32" && g_D == 32 && g_last.dmem == 16);
    EXPECT(sigattn_bwd(&p, kFake, kFake, kFake, kFake, nullptr) == 0 && calls() == "dq_f32,dkdv_f32" &&
           g_D == 32 && g_last.dmem == 16);
    EXPECT(sigattn_bwd_workspace_bytes(&p) == 0 && sigattn_fwd_workspace_bytes(&p) == 0);
    // Rows not 16-byte aligned: the portable kernels (a row stride of 4k + 2
    // floats, or of 8k + 4 16-bit elements).
    p.q_stride_t = 34;
    EXPECT(sigattn_fwd(&p, kFake, nullptr) == 0 && calls() == "fwd_generic" && g_D == 16);
    EXPECT(sigattn_bwd(&p, kFake, kFake, kFake, kFake, nullptr) == 0 && calls() == "dq_generic,dkdv_generic" &&
           g_D == 16);
    p.dtype = SIGATTN_BF16;
    p.q_stride_t = 36;
    EXPECT(sigattn_fwd(&p, kFake, nullptr) == 0 && calls() == "fwd_generic" && g_D == 16);
    p = base(1, 40, 1, 32);
    p.D = 64;
    p.dtype = SIGATTN_F32;
    EXPECT(sigattn_bwd(&p, kFake, kFake, kFake, kFake, nullptr) == 0 && calls() == "dq_f32,dkdv_f32" && g_D == 64);
    EXPECT(sigattn_bwd_workspace_bytes(&p) == 0);
    // A misaligned pointer sends fp32 to the portable kernels too.
    EXPECT(sigattn_fwd(&p, (char *)kFake + 4, nullptr) == 0 && calls() == "fwd_generic");
    // fp32 rows spanning 2^31 bytes or more (the copies' 32-bit offsets): portable.
    p.Tq = p.Tk = (1 << 28) / 64 + 1;
    p.q_stride_t = p.k_stride_t = 128;
    p.q_stride_b = p.k_stride_b = p.Tq * 128;
    EXPECT(sigattn_fwd(&p, kFake, nullptr) == 0 && calls() == "fwd_generic");
    p = base(1, 40, 1, 32);
    p.D = 64;
    p.dtype = SIGATTN_F16;
    p.q_stride_t = 68;
    EXPECT(sigattn_fwd(&p, kFake, nullptr) == 0 && calls() == "fwd_generic");
  }
  {
    // Decode shape: split-KV with a workspace, one chunk per (batch, head) without.
    sigattn_problem p = base(1, 1, 1, 128);
    p.Tk = 4096;
    p.seq_lens_q = p.seq_lens_k = (const int32_t *)kFake;
    p.k_stride_b = 4096 * 128;
    const size_t ws = sigattn_fwd_workspace_bytes(&p);
    EXPECT(ws == 16 * 128 * 4);
    EXPECT(sigattn_fwd_ws(&p, kFake, kFake, ws, nullptr) == 0 && calls() == "fwd_splitkv");
    EXPECT(g_last.nsplit == 16 && g_last.chunk == 256 && g_last.ws == kFake);
    EXPECT(sigattn_fwd(&p, kFake, nullptr) == 0 && calls() == "fwd_splitkv");
    EXPECT(g_last.nsplit == 1 && g_last.ws == nullptr);
    EXPECT(sigattn_fwd_ws(&p, kFake, kFake, ws - 1, nullptr) == SIGATTN_ERR_WORKSPACE && g_calls.empty());
    // No allocation, no caller workspace: the partials go to the fixed scratch.
    EXPECT(sigattn_fwd_noalloc(&p, kFake, nullptr) == 0 && calls() == "fwd_splitkv");
    EXPECT(g_last.nsplit == 16 && g_last.ws == reinterpret_cast<float *>(uintptr_t(3) << 20));
    // The largest split plan: one (batch, head) pair, 32 queries, D = 128.
    p.Tq = 32;
    p.Tk = 1 << 20;
    p.k_stride_b = p.Tk * 128;
    EXPECT(sigattn_fwd_workspace_bytes(&p) <= SIGATTN_NOALLOC_SCRATCH_BYTES);
    EXPECT(sigattn_fwd_noalloc(&p, kFake, nullptr) == 0 && calls() == "fwd_splitkv");
    EXPECT(g_last.nsplit == 512);
    // A problem that does not split runs as sigattn_fwd does.
    sigattn_problem d = base(2, 300, 3, 128);
    EXPECT(sigattn_fwd_noalloc(&d, kFake, nullptr) == 0 && calls() == "fwd_mfma");
    EXPECT(g_last.ws == nullptr && g_last.nsplit == 0);
  }
  {
    // Empty problems launch nothing.
    sigattn_problem p = base(0, 16, 2, 64);
    EXPECT(sigattn_fwd(&p, nullptr, nullptr) == 0 && sigattn_bwd(&p, nullptr, nullptr, nullptr, nullptr, nullptr) == 0);
    p = base(2, 0, 2, 64);
    EXPECT(sigattn_fwd(&p, nullptr, nullptr) == 0 && sigattn_bwd(&p, nullptr, nullptr, nullptr, nullptr, nullptr) == 0);
    EXPECT(g_calls.empty());
  }
  {
    // Packed layout: the rows outside every sequence are zeroed by the
    // leading workgroups of the MFMA forward (O) and dQ launch (dQ, and dK /
    // dV too), or by a launch of their own on the portable kernels and when
    // no such kernel runs.
    sigattn_problem p = base(3, 300, 2, 128);
    p.cu_seqlens_q = p.cu_seqlens_k = (const int32_t *)kFake;
    p.rows_q = 700, p.rows_k = 650;
    p.q_stride_b = p.k_stride_b = 0;
    char *o = (char *)kFake, *dq = o + 4096, *dk = o + 8192, *dv = o + 12288;
    g_hist.clear();
    EXPECT(sigattn_fwd(&p, o, nullptr) == 0 && calls() == "fwd_mfma" && gaps_at(0, 700, o));
    EXPECT(g_hist[0].gap[0].T == 300 && g_hist[0].gap[0].B == 3 && g_hist[0].gap[0].cu == kFake);
    g_hist.clear();
    EXPECT(sigattn_bwd(&p, kFake, dq, dk, dv, nullptr) == 0 && calls() == "dq_mfma,dkdv_mfma");
    EXPECT(gaps_at(0, 700, dq, 650, dk, dv) && gaps_at(1, 0, nullptr));
    g_hist.clear();
    EXPECT(sigattn_bwd_dq(&p, kFake, dq, nullptr) == 0 && calls() == "dq_mfma" && gaps_at(0, 700, dq));
    // dK/dV alone: no dQ launch, so a launch of their own.
    g_hist.clear();
    EXPECT(sigattn_bwd_dkdv(&p, kFake, dk, dv, nullptr) == 0 && calls() == "zero_gaps,dkdv_mfma" &&
           gaps_at(0, 0, nullptr));
    EXPECT(sigattn::g_gap[0].rows == 0 && sigattn::g_gap[1].rows == 650 && sigattn::g_gap[1].out[0] == dk);
    // Two-pass backward: the first head group's dQ-from-dS launch.
    const size_t ws = sigattn_bwd_workspace_bytes(&p);
    g_hist.clear();
    EXPECT(sigattn_bwd_ws(&p, kFake, dq, dk, dv, kFake, ws, nullptr) == 0 && calls() == "dkdv_mfma_ds,dq_ds");
    EXPECT(gaps_at(0, 0, nullptr) && gaps_at(1, 700, dq, 650, dk, dv));
    g_hist.clear();
    EXPECT(sigattn_bwd_ws(&p, kFake, dq, dk, dv, kFake, ws / 2, nullptr) == 0 &&
           calls() == "dkdv_mfma_ds,dq_ds,dkdv_mfma_ds,dq_ds");
    EXPECT(gaps_at(0, 0, nullptr) && gaps_at(1, 700, dq, 650, dk, dv) && gaps_at(2, 0, nullptr) &&
           gaps_at(3, 0, nullptr));
    // fp32: the fp32 MFMA kernels, likewise.
    p.dtype = SIGATTN_F32;
    g_hist.clear();
    EXPECT(sigattn_fwd(&p, o, nullptr) == 0 && calls() == "fwd_f32" && gaps_at(0, 700, o));
    g_hist.clear();
    EXPECT(sigattn_bwd(&p, kFake, dq, dk, dv, nullptr) == 0 && calls() == "dq_f32,dkdv_f32" &&
           gaps_at(0, 700, dq, 650, dk, dv) && gaps_at(1, 0, nullptr));
    // Rows off 16-byte boundaries: the portable kernels and one gap launch.
    p.q_stride_t = 2 * 128 + 2;
    g_hist.clear();
    EXPECT(sigattn_fwd(&p, o, nullptr) == 0 && calls() == "zero_gaps,fwd_generic");
    EXPECT(sigattn::g_gap[0].rows == 700 && sigattn::g_gap[0].out[0] == o && sigattn::g_gap[1].rows == 0);
    EXPECT(sigattn_bwd(&p, kFake, dq, dk, dv, nullptr) == 0 && calls() == "zero_gaps,dq_generic,dkdv_generic");
    EXPECT(sigattn::g_gap[0].rows == 700 && sigattn::g_gap[1].rows == 650 && sigattn::g_gap[1].out[0] == dk &&
           sigattn::g_gap[1].out[1] == dv);
    p.q_stride_t = 2 * 128;
    p.dtype = SIGATTN_BF16;
    // No sequences (B = 0) or no queries: every row is a gap; none without rows.
    p.B = 0;
    EXPECT(sigattn_fwd(&p, kFake, nullptr) == 0 && calls() == "zero_gaps");
    EXPECT(sigattn_fwd(&p, nullptr, nullptr) == SIGATTN_ERR_NULL_ARG);
    EXPECT(sigattn_bwd(&p, nullptr, kFake, kFake, kFake, nullptr) == 0 && calls() == "zero_gaps");
    p.rows_q = p.rows_k = 0;
    EXPECT(sigattn_fwd(&p, kFake, nullptr) == 0 && sigattn_bwd(&p, nullptr, kFake, kFake, kFake, nullptr) == 0);
    EXPECT(g_calls.empty());
  }
  {
    // Range split of small dense non-causal grids, on a device of 256 CUs:
    // B=1 L=2048 H=8 D=64 has 128 workgroups per kernel.
    g_cus = 256;
    sigattn_problem p = base(1, 2048, 8, 64);
    // 128 items of 2048 keys: two chunks of 1024 keys (saving 1024 rows per
    // item), one workgroup per CU.
    const size_t fw = sigattn_fwd_workspace_bytes(&p);
    EXPECT(fw == 512 + size_t(128) * 2 * 128 * 64 * 4);  // counters, then 2 partials per item
    EXPECT(sigattn_fwd_ws(&p, kFake, kFake, fw, nullptr) == 0 && calls() == "rs_clear,fwd_mfma");
    EXPECT(g_last.rsplit == 2 && g_last.rs_cnt == kFake && (char *)g_last.rs_part == (char *)kFake + 512);
    // A workspace too small for the partials, or misaligned: unsplit, as sigattn_fwd.
    EXPECT(sigattn_fwd_ws(&p, kFake, kFake, fw - 1, nullptr) == 0 && calls() == "fwd_mfma" && g_last.rsplit == 0);
    EXPECT(sigattn_fwd_ws(&p, kFake, (char *)kFake + 8, fw, nullptr) == 0 && calls() == "fwd_mfma" &&
           g_last.rsplit == 0);
    EXPECT(sigattn_fwd(&p, kFake, nullptr) == 0 && calls() == "fwd_mfma" && g_last.rsplit == 0);
    EXPECT(sigattn_fwd_noalloc(&p, kFake, nullptr) == 0 && calls() == "fwd_mfma" && g_last.rsplit == 0);
    const size_t bw = sigattn_bwd_split_workspace_bytes(&p);
    const size_t dq_bytes = 512 + size_t(128) * 2 * 128 * 64 * 4;
    EXPECT(bw == dq_bytes + 512 + size_t(128) * 2 * 2 * 128 * 64 * 4);
    EXPECT(sigattn_bwd_split(&p, kFake, kFake, kFake, kFake, kFake, bw, nullptr) == 0 &&
           calls() == "rs_clear,dq_mfma,dkdv_mfma");
    EXPECT(g_last.rsplit == 2 && (char *)g_last.rs_cnt == (char *)kFake + dq_bytes);
    EXPECT(sigattn_bwd_split(&p, kFake, kFake, kFake, kFake, kFake, bw - 1, nullptr) == SIGATTN_ERR_WORKSPACE);
    // Halves: dQ alone, dK/dV alone (its counters after dQ's part), neither.
    EXPECT(sigattn_bwd_split(&p, kFake, kFake, nullptr, nullptr, kFake, bw, nullptr) == 0 &&
           calls() == "rs_clear,dq_mfma" && g_last.rsplit == 2 && g_last.rs_cnt == kFake);
    EXPECT(sigattn_bwd_split(&p, kFake, nullptr, kFake, kFake, kFake, bw, nullptr) == 0 &&
           calls() == "rs_clear,dkdv_mfma" && (char *)g_last.rs_cnt == (char *)kFake + dq_bytes);
    EXPECT(sigattn_bwd_split(&p, kFake, nullptr, nullptr, nullptr, kFake, bw, nullptr) == SIGATTN_ERR_NULL_ARG &&
           g_calls.empty());
    EXPECT(sigattn_bwd_split(&p, kFake, kFake, kFake, nullptr, kFake, bw, nullptr) == SIGATTN_ERR_NULL_ARG);
    EXPECT(sigattn_bwd_split(&p, kFake, nullptr, kFake, kFake, nullptr, 0, nullptr) == 0 &&
           calls() == "dkdv_mfma" && g_last.rsplit == 0);
    EXPECT(sigattn_bwd_split(&p, kFake, kFake, kFake, kFake, nullptr, 0, nullptr) == 0 &&
           calls() == "bwd_fused" && g_last.rsplit == 0);
    // Causal, padded, D = 128 backward, or grids that fill the GPU: no split.
    sigattn_problem c = p;
    c.causal = 1;
    EXPECT(sigattn_fwd_workspace_bytes(&c) == 0 && sigattn_bwd_split_workspace_bytes(&c) == 0);
    c = p;
    c.seq_lens_q = c.seq_lens_k = (const int32_t *)kFake;
    EXPECT(sigattn_fwd_workspace_bytes(&c) == 0 && sigattn_bwd_split_workspace_bytes(&c) == 0);
    // D = 128: the forward and the dQ kernel split, the dK/dV kernel does not.
    c = base(2, 1024, 8, 128);
    const size_t bw128 = sigattn_bwd_split_workspace_bytes(&c);
    EXPECT(sigattn_fwd_workspace_bytes(&c) > 0 && bw128 == 512 + size_t(128) * 2 * 128 * 128 * 4);
    EXPECT(sigattn_bwd_split(&c, kFake, kFake, kFake, kFake, kFake, bw128, nullptr) == 0 &&
           calls() == "rs_clear,dq_mfma,dkdv_mfma" && g_last.rsplit == 0);
    c = base(4, 1024, 8, 64);  // 256 items: the GPU is already half full
    EXPECT(sigattn_fwd_workspace_bytes(&c) == 0 && sigattn_bwd_split_workspace_bytes(&c) == 0);
    // At D = 64 a split must save 1024 rows per item: c2 (B=2 L=1024 H=8) in two
    // chunks saves 512; 2000 keys save 1000 in two, and three chunks of 128
    // items exceed one workgroup per CU.
    c = base(2, 1024, 8, 64);
    EXPECT(sigattn_fwd_workspace_bytes(&c) == 0 && sigattn_bwd_split_workspace_bytes(&c) == 0);
    c = base(1, 2000, 8, 64);
    EXPECT(sigattn_fwd_workspace_bytes(&c) == 0 && sigattn_bwd_split_workspace_bytes(&c) == 0);
    // Three chunks of 1536 keys (saving 1024 rows) for 24 items.
    c = base(1, 1536, 2, 64);
    EXPECT(sigattn_fwd_workspace_bytes(&c) == 256 + size_t(24) * 3 * 128 * 64 * 4);
    // Four chunks at 2048 keys per item of 64 items (one workgroup per CU),
    // and at 4096 keys per item of 128 items (chunks of 1024: two per CU).
    c = base(1, 2048, 4, 64);
    EXPECT(sigattn_fwd_workspace_bytes(&c) == 256 + size_t(64) * 4 * 128 * 64 * 4);
    c = base(1, 4096, 4, 64);
    EXPECT(sigattn_fwd_workspace_bytes(&c) == 512 + size_t(128) * 4 * 128 * 64 * 4);
    c = base(1, 2048, 8, 64);  // 128 items: two chunks
    EXPECT(sigattn_fwd_workspace_bytes(&c) == 512 + size_t(128) * 2 * 128 * 64 * 4);
    // The recompute backward as one launch: dense, D <= 64 (16-bit), and the
    // dQ and dK/dV grids together within one workgroup per CU.
    for (int causal = 0; causal < 2; ++causal) {
      c = base(2, 1024, 8, 64);  // c2: 128 + 128 workgroups
      c.causal = causal;
      EXPECT(sigattn_bwd(&c, kFake, kFake, kFake, kFake, nullptr) == 0 && calls() == "bwd_fused" && g_D == 64);
      EXPECT(sigattn_bwd_split(&c, kFake, kFake, kFake, kFake, kFake, 1 << 20, nullptr) == 0 &&
             calls() == "bwd_fused");
      EXPECT(sigattn_bwd_ws(&c, kFake, kFake, kFake, kFake, nullptr, 0, nullptr) == 0 && calls() == "bwd_fused");
      // Halves alone run their own kernel.
      EXPECT(sigattn_bwd_dq(&c, kFake, kFake, nullptr) == 0 && calls() == "dq_mfma");
      EXPECT(sigattn_bwd_dkdv(&c, kFake, kFake, kFake, nullptr) == 0 && calls() == "dkdv_mfma");
    }
    c = base(2, 1024, 8, 16);
    EXPECT(sigattn_bwd(&c, kFake, kFake, kFake, kFake, nullptr) == 0 && calls() == "bwd_fused" && g_D == 32 &&
           g_last.dmem == 16);
    c = base(3, 1024, 8, 64);  // 384 workgroups: two launches
    EXPECT(sigattn_bwd(&c, kFake, kFake, kFake, kFake, nullptr) == 0 && calls() == "dq_mfma,dkdv_mfma");
    c = base(2, 1024, 8, 128);
    EXPECT(sigattn_bwd(&c, kFake, kFake, kFake, kFake, nullptr) == 0 && calls() == "dq_mfma,dkdv_mfma");
    c = base(2, 1024, 8, 64);
    c.seq_lens_q = c.seq_lens_k = (const int32_t *)kFake;
    EXPECT(sigattn_bwd(&c, kFake, kFake, kFake, kFake, nullptr) == 0 && calls() == "dq_mfma,dkdv_mfma");
    c = base(2, 1024, 8, 64);
    c.dtype = SIGATTN_F32;
    EXPECT(sigattn_bwd(&c, kFake, kFake, kFake, kFake, nullptr) == 0 && calls() == "dq_f32,dkdv_f32");
    EXPECT(g_sync.empty());
    // The concurrent recompute backward: ragged, non-causal, D = 64, at least
    // eight 128-query blocks per CU (B=4 T=8192 H=12: 3072 on 256 CUs).  The
    // dK/dV kernel goes first, on the side stream, forked off the caller's
    // stream (0 here) by event 257 and joined back by event 258.
    c = base(4, 8192, 12, 64);
    c.seq_lens_q = c.seq_lens_k = (const int32_t *)kFake;
    const hipStream_t own = nullptr;
    EXPECT(sigattn_bwd(&c, kFake, kFake, kFake, kFake, own) == 0 && calls() == "dkdv_mfma,dq_mfma" &&
           g_dkdv_stream == kSide && g_dq_stream == own);
    EXPECT(sync_log() == "record 257 0;wait 20736 257;record 258 20736;wait 0 258");
    // Again on this thread: the same stream and events.
    EXPECT(sigattn_bwd_split(&c, kFake, kFake, kFake, kFake, nullptr, 0, own) == 0 &&
           calls() == "dkdv_mfma,dq_mfma" && g_dkdv_stream == kSide && g_nevents == 2);
    EXPECT(sync_log() == "record 257 0;wait 20736 257;record 258 20736;wait 0 258");
    // The packed layout alike; the dQ launch zeroes the gap rows (none here).
    sigattn_problem pk = c;
    pk.seq_lens_q = pk.seq_lens_k = nullptr;
    pk.cu_seqlens_q = pk.cu_seqlens_k = (const int32_t *)kFake;
    pk.rows_q = pk.rows_k = 4 * 8192;
    pk.q_stride_b = pk.k_stride_b = 0;
    EXPECT(sigattn_bwd(&pk, kFake, kFake, kFake, kFake, own) == 0 && calls() == "dkdv_mfma,dq_mfma" &&
           g_dkdv_stream == kSide);
    EXPECT(!sync_log().empty());
    // On another device's stream, under stream capture, causal, dense, D = 32
    // or too few blocks: one stream.
    EXPECT(sigattn_bwd(&c, kFake, kFake, kFake, kFake, kOtherDevice) == 0 && calls() == "dq_mfma,dkdv_mfma" &&
           g_dkdv_stream == kOtherDevice && g_dq_stream == kOtherDevice && g_sync.empty());
    g_capture = hipStreamCaptureStatusActive;
    EXPECT(sigattn_bwd(&c, kFake, kFake, kFake, kFake, own) == 0 && calls() == "dq_mfma,dkdv_mfma" &&
           g_dkdv_stream == own);
    g_capture = hipStreamCaptureStatusNone;
    sigattn_problem d = c;
    d.causal = 1;
    EXPECT(sigattn_bwd(&d, kFake, kFake, kFake, kFake, own) == 0 && calls() == "dq_mfma,dkdv_mfma");
    d = c;
    d.seq_lens_q = d.seq_lens_k = nullptr;
    EXPECT(sigattn_bwd(&d, kFake, kFake, kFake, kFake, own) == 0 && calls() == "dq_mfma,dkdv_mfma");
    d = base(4, 8192, 12, 32);
    d.seq_lens_q = d.seq_lens_k = (const int32_t *)kFake;
    EXPECT(sigattn_bwd(&d, kFake, kFake, kFake, kFake, own) == 0 && calls() == "dq_mfma,dkdv_mfma");
    d = base(4, 4096, 8, 64);  // 1024 blocks: four per CU
    d.seq_lens_q = d.seq_lens_k = (const int32_t *)kFake;
    EXPECT(sigattn_bwd(&d, kFake, kFake, kFake, kFake, own) == 0 && calls() == "dq_mfma,dkdv_mfma");
    // Halves alone run on the caller's stream.
    EXPECT(sigattn_bwd_dq(&c, kFake, kFake, own) == 0 && calls() == "dq_mfma" && g_dq_stream == own);
    EXPECT(sigattn_bwd_dkdv(&c, kFake, kFake, kFake, own) == 0 && calls() == "dkdv_mfma" && g_dkdv_stream == own);
    EXPECT(g_sync.empty());
    g_cus = 0;
  }
  if (g_fail == 0) std::printf("capi sanitizer driver: all checks passed\n");
  return g_fail == 0 ? 0 : 1;
}
