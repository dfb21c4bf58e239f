// Shared device-side definitions for the gfx950 sigmoid-attention kernels.
//
// MFMA tiling used by every fast kernel (v_mfma_f32_32x32x16_{bf16,f16}):
//   * A operand: lane l holds row (l % 32), eight k-elements (k-slot h = l / 32).
//   * B operand: lane l holds column (l % 32), eight k-elements (k-slot h).
//     A and B use the same (h, j) -> k mapping, so any product whose two
//     operands are both read from memory may choose that mapping freely; we use
//     k = 8h + j (16 contiguous bytes per lane).
//   * C/D (16 fp32 per lane): lane l holds column (l % 32), register i holds
//     row 8*(i/4) + 4*(l/32) + (i%4).
// A score tile computed as Sᵀ (rows = keys, columns = queries) therefore already
// sits in the B-operand layout of the next product over keys: register group
// i in [8s, 8s+8) of a 32-key block is B k-step s with key = 16s' + 8(j/4) +
// 4h + (j%4).  The matching A operand (e.g. Vᵀ rows) is read from LDS with the
// same key permutation as two 8-byte reads.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace sigattn {

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Kernel-local lambdas capture register arrays by reference; they must be
// inlined or the arrays are demoted to scratch memory.
#define SIGATTN_INLINE __attribute__((always_inline))

// log2(e): sigmoid(x) = 1 / (1 + 2^(-x * log2(e))).
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ int clamp_len(const int32_t *lens, int b, int T) {
  if (lens == nullptr) return T;
  int L = lens[b];
  return L < 0 ? 0 : (L > T ? T : L);
}

// First row of sequence b in a packed [rows, H, D] tensor: cu[b] clamped to
// [0, rows].
__device__ __forceinline__ int64_t packed_first(const int32_t *cu, int64_t rows, int b) {
  const int64_t s = cu[b];
  return s < 0 ? 0 : (s > rows ? rows : s);
}

// Rows of sequence b in a packed tensor: cu[b+1] - cu[b] after both are
// clamped to [0, rows] (so first + length <= rows), at most T.
__device__ __forceinline__ int packed_len(const int32_t *cu, int64_t rows, int b, int T) {
  const int64_t s = packed_first(cu, rows, b);
  int64_t e = cu[b + 1];
  e = e < s ? s : (e > rows ? rows : e);
  return (int)(e - s < T ? e - s : T);
}

// One packed sequence axis whose output rows outside every sequence are to
// be zeroed: cu_seqlens [B + 1], the axis's row count, its longest sequence
// T, the outputs' row and head strides (elements) and up to two output
// tensors (nullptr: none).  See zero_gap_rows.
struct GapAxis {
  const int32_t *cu = nullptr;
  int B = 0, T = 0, H = 0, D = 0;
  int64_t rows = 0, st = 0, sh = 0;
  void *out[2] = {nullptr, nullptr};
};

// Kernel parameters (passed by value).  Strides are in elements.
//
// Each sequence axis (queries, keys) has one of three layouts:
//   * dense: batch b holds T rows at b * stride_b;
//   * padded (seq_* set): the first seq_*[b] of those T rows are valid;
//   * packed (cu_* set): tensors are [rows, H, D] and batch b holds rows
//     cu_*[b] .. cu_*[b+1]-1 (at most T = the longest sequence).
// Padded outputs write zeros to the invalid rows of each batch; packed
// outputs write exactly the rows of each sequence and nothing else.
struct KParams {
  const void *q, *k, *v, *dout;
  void *out, *dq, *dk, *dv;
  const float *bias;       // [B]
  const float *scale;      // 0-d
  const float *score_mod;  // [B, Tk] (packed keys: [rows_k]) fp32 contiguous or nullptr
  const int32_t *seq_q;    // [B] or nullptr (= Tq)
  const int32_t *seq_k;    // [B] or nullptr (= Tk)
  const int32_t *cu_q;     // [B+1] packed query offsets or nullptr
  const int32_t *cu_k;     // [B+1] packed key offsets or nullptr
  int64_t rows_q, rows_k;  // packed row counts (with cu_q / cu_k)
  int64_t sq_b, sq_t, sq_h;  // Q / O / dO / dQ
  int64_t sk_b, sk_t, sk_h;  // K / V / dK / dV
  int B, H, Tq, Tk;
  int nblk;  // number of row blocks along the stationary sequence axis
  // Split-KV forward: keys cut into nsplit chunks of `chunk` keys; fp32
  // partials [nsplit, B, H, Tq, D] in ws when nsplit > 1.
  int nsplit, chunk;
  float *ws;
  // Two-pass backward: dS in the I/O dtype as 32x32 tiles (see DsLayout),
  // written by the dK/dV kernel and read by the dQ-from-dS kernel.
  uint16_t *ds;
  int ds_nqb, ds_nkb;  // 32-row query / key blocks per (batch, head): ceil(Tq/32), ceil(Tk/32)
  // Range split of small dense non-causal grids (rsplit <= 1: off): every
  // work item's streamed range (keys for the forward and dQ kernels, queries
  // for dK/dV) runs as rsplit chunks in rsplit workgroups, which hand their
  // fp32 accumulators over through rs_part (rsplit partials per item) and
  // count themselves in rs_cnt[item] (zero at launch); see split_combine.
  int rsplit;
  float *rs_part;
  int *rs_cnt;
  int ncu;  // compute units of the device (WorkOrder::by_level's dealing rounds)
  // Packed layouts: the first ngap[0] workgroups of the launch zero the rows
  // of gap[0]'s outputs that no sequence covers (zero_gap_rows), the next
  // ngap[1] those of gap[1], and do nothing else; the kernel's work items
  // follow (gap_prologue).  0: none.
  GapAxis gap[2];
  int ngap[2];
  // Head dim of the tensors.  The D = 32 kernels also take head_dim 16
  // (dmem = 16): the stationary rows' upper 16 columns enter as zeros, the
  // streamed tiles repeat the 16 columns there (so every product over the
  // head dim adds exact zeros), and only the first 16 output columns are
  // stored.
  int dmem;
  // The D = 32 kernels computing head_dim 16 (see dmem).
  __device__ __forceinline__ bool half_head(int D) const { return D == 32 && dmem == 16; }

  // Valid query / key rows of batch b.
  __device__ __forceinline__ int len_q(int b) const {
    return cu_q != nullptr ? packed_len(cu_q, rows_q, b, Tq) : clamp_len(seq_q, b, Tq);
  }
  __device__ __forceinline__ int len_k(int b) const {
    return cu_k != nullptr ? packed_len(cu_k, rows_k, b, Tk) : clamp_len(seq_k, b, Tk);
  }
  // Element offset of row 0 of (b, h) in the Q-shaped / K-shaped tensors.
  __device__ __forceinline__ int64_t q_base(int b, int h) const {
    const int64_t r = cu_q != nullptr ? packed_first(cu_q, rows_q, b) * sq_t : (int64_t)b * sq_b;
    return r + (int64_t)h * sq_h;
  }
  __device__ __forceinline__ int64_t k_base(int b, int h) const {
    const int64_t r = cu_k != nullptr ? packed_first(cu_k, rows_k, b) * sk_t : (int64_t)b * sk_b;
    return r + (int64_t)h * sk_h;
  }
  // score_mod entry of key 0 of batch b.
  __device__ __forceinline__ int64_t mod_base(int b) const {
    return cu_k != nullptr ? packed_first(cu_k, rows_k, b) : (int64_t)b * Tk;
  }
  // Rows of batch b an output kernel writes (zeros past the valid length
  // in the padded layout; only the sequence itself in the packed layout).
  __device__ __forceinline__ int q_rows_out(int Lq) const { return cu_q != nullptr ? Lq : Tq; }
  __device__ __forceinline__ int k_rows_out(int Lk) const { return cu_k != nullptr ? Lk : Tk; }
  // Batches differ in length (the work order then follows the lengths).
  __host__ __device__ __forceinline__ bool ragged() const {
    return seq_q != nullptr || seq_k != nullptr || cu_q != nullptr || cu_k != nullptr;
  }
  // Padded layout whose rows hold every head back to back (row stride H*D,
  // head stride D), so the rows of a row block over all heads are one
  // contiguous span of the Q-shaped / K-shaped tensors.
  __device__ __forceinline__ bool q_rows_contiguous(int D) const {
    return cu_q == nullptr && sq_h == D && sq_t == (int64_t)H * D;
  }
  __device__ __forceinline__ bool k_rows_contiguous(int D) const {
    return cu_k == nullptr && sk_h == D && sk_t == (int64_t)H * D;
  }
};

// Zeroes the rows blk*64 .. blk*64+63 of `ax`'s outputs that no sequence
// covers (256 threads): 64 threads find whether their row lies in a
// sequence -- a binary search over cu when cu is non-decreasing (the
// workgroup checks first), else a scan over every sequence -- and the
// workgroup zeroes the uncovered rows' H x D elements.  Rows a sequence
// covers are never written, so this may run in any order with the
// attention work that writes them.  `lds`: 16 bytes of LDS (8-byte aligned)
// the workgroup may use -- a kernel's own tile memory, which its gap
// workgroups never touch otherwise.
template <int ESIZE> __device__ __forceinline__ void zero_gap_rows(const GapAxis &ax, int blk, void *lds) {
  const int64_t r0 = (int64_t)blk * 64;
  unsigned long long &gaps = ((unsigned long long *)lds)[0];
  int &sorted = ((int *)lds)[2];
  if (threadIdx.x == 0) {
    sorted = 1;
    gaps = 0ull;
  }
  __syncthreads();
  for (int b = threadIdx.x; b < ax.B; b += blockDim.x)
    if (ax.cu[b + 1] < ax.cu[b]) sorted = 0;
  __syncthreads();
  if (threadIdx.x < 64) {
    const int64_t r = r0 + threadIdx.x;
    bool covered = false;
    if (r < ax.rows && ax.B > 0) {
      auto covers = [&](int b) {
        const int64_t f = packed_first(ax.cu, ax.rows, b);
        return r >= f && r < f + packed_len(ax.cu, ax.rows, b, ax.T);
      };
      if (sorted) {
        // Largest b with first(b) <= r (first() is non-decreasing here).
        int lo = 0, hi = ax.B - 1;
        while (lo < hi) {
          const int mid = (lo + hi + 1) / 2;
          if (packed_first(ax.cu, ax.rows, mid) <= r) lo = mid;
          else hi = mid - 1;
        }
        covered = covers(lo);
      } else {
        for (int b = 0; b < ax.B && !covered; ++b) covered = covers(b);
      }
    }
    const unsigned long long m = __ballot(r < ax.rows && !covered);
    if (threadIdx.x == 0) gaps = m;
  }
  __syncthreads();
  unsigned long long m = gaps;
  const int per_row = ax.H * ax.D;
  typedef typename std::conditional<ESIZE == 4, uint32_t, uint16_t>::type E;
  while (m != 0ull) {
    const int i = __builtin_ctzll(m);
    m &= m - 1;
    const int64_t row = (r0 + i) * ax.st;
    for (int e = threadIdx.x; e < per_row; e += blockDim.x) {
      const int h = e / ax.D, d = e - h * ax.D;
      const int64_t off = row + (int64_t)h * ax.sh + d;
      for (int t = 0; t < 2; ++t)
        if (ax.out[t] != nullptr) ((E *)ax.out[t])[off] = (E)0;
    }
  }
}

// Work-item id of this workgroup, or -1 for the leading ngap[0] + ngap[1]
// workgroups, which zero the gap rows of KParams::gap (ESIZE-byte elements)
// instead.  Both counts are multiples of 8, so the items keep the XCD each
// would have without them.
template <int ESIZE> __device__ __forceinline__ int gap_prologue(const KParams &p, void *lds) {
  const int id = (int)blockIdx.x;
  if (id >= p.ngap[0] + p.ngap[1]) return id - p.ngap[0] - p.ngap[1];
  if (id < p.ngap[0]) zero_gap_rows<ESIZE>(p.gap[0], id, lds);
  else zero_gap_rows<ESIZE>(p.gap[1], id - p.ngap[0], lds);
  return -1;
}

// Zero rows of the padded layout.  A row block wholly past a batch's valid
// length is a padding work item for each of the H heads; when every head's
// rows are contiguous (KParams::q_rows_contiguous / k_rows_contiguous), the
// rows [row0, row1) of all heads form one span of (row1 - row0) * row_elems
// elements at batch_base + row0 * row_elems, and the item of head `part` of
// `nparts` zeroes its 1/nparts of it with contiguous 16-byte stores (rather
// than its own head's rows, 2*D bytes at a stride of 2*H*D).  row_elems is a
// multiple of 8 and batch_base 16-byte aligned (MFMA-path requirements).
__device__ __forceinline__ void zero_row_span(void *batch_base, int64_t row_elems, int row0, int row1,
                                              int part, int nparts, int tid, int nthreads) {
  if (row1 <= row0) return;
  const int64_t n = (int64_t)(row1 - row0) * row_elems / 8;  // 16-byte pieces
  const int64_t c0 = n * part / nparts, c1 = n * (part + 1) / nparts;
  u32x4 *dst = (u32x4 *)((uint16_t *)batch_base + (int64_t)row0 * row_elems);
  for (int64_t c = c0 + tid; c < c1; c += nthreads) dst[c] = (u32x4){0u, 0u, 0u, 0u};
}

// ---------------------------------------------------------------------------
// Work-item order.  A kernel's grid covers (row block, batch, head) items of
// its stationary sequence (queries for the forward and dQ, keys for dK/dV).
// The hardware deals workgroup ids round-robin over the 8 XCDs and each XCD
// starts them in id order, so ids sorted by decreasing work give every XCD an
// even, heaviest-first share.  Dense grids already are in that order (all
// items equal, or causal row blocks heaviest first); for padded batches the
// work depends on each batch's lengths, so WorkOrder re-derives the item of
// workgroup `id` from seq_lens on the device (no host sync):
//   * by_stream: items of longer streamed sequences first (non-causal: every
//     row block of batch b costs its full streamed length), each batch's
//     items dealt to the XCDs head by head;
//   * by_level: row-block levels in the given direction (causal: the cost
//     grows with the query block, or shrinks with the key block), the batches
//     valid at a level in index order, heads fastest.
// Padding items (row block past a batch's length) come after all valid items,
// batch by batch; their workgroups only write the zero rows (padded layout)
// or nothing (packed layout).  Every lane of
// every wave computes the same answer (lane j holds batch j), so B is limited
// to 64; callers keep the dense order beyond that.
struct WorkItem {
  int b, h, blk;
};
// by_stream deals the equal items of one batch to the XCDs head-major
// (xcd_grouped): measured at B=4 Lmax=8192 H=12 D=64 padded, HBM fetch per
// launch forward 156 -> 86 MB, dQ 170 -> 105 MB, dK/dV 186 -> 115 MB, with
// the kernel times unchanged (within 1 %).  0 = heads fastest.
#ifndef SIGATTN_STREAM_GROUPED
#define SIGATTN_STREAM_GROUPED 1
#endif

// Dealing order of WorkOrder::by_level (see dealt).  Measured on MI355X at
// fp16 B=8 Lmax=2048 H=8 D=64 causal, seq_lens 682-1789 (three runs each,
// kernel times in us, plain / 1 / 2): forward 39.2 / 34.9 / 35.8, dQ 51.3 /
// 52.0 / 51.3, dK/dV 68.1 / 65.5 / 72.3.
#ifndef SIGATTN_LEVEL_DEAL
#define SIGATTN_LEVEL_DEAL 1
#endif

struct WorkOrder {
  // Row blocks of batch `lane` (0 for lanes past B); rows(b) = valid rows.
  template <class Len>
  static __device__ __forceinline__ int row_blocks(Len rows, int RB, int B, int lane) {
    if (lane >= B) return 0;
    return (rows(lane) + RB - 1) / RB;
  }
  static __device__ __forceinline__ int kth_set_bit(uint64_t m, int k) {
    for (int t = 0; t < k; ++t) m &= m - 1;
    return __builtin_ctzll(m);
  }
  // Padding item j (0-based, after all valid items): batches in index order,
  // row blocks nv..nlev-1, heads fastest.
  static __device__ __forceinline__ WorkItem padding(int j, int B, int H, int nv, int nlev) {
    const int lane = __lane_id();
    const int cnt = lane < B ? (nlev - nv) * H : 0;
    int start = 0;
    for (int k = 0; k < B; ++k) start += k < lane ? __builtin_amdgcn_readlane(cnt, k) : 0;
    const uint64_t m = __ballot(lane < B && j >= start && j < start + cnt);
    const int b = m != 0 ? __builtin_ctzll(m) : 0;
    const int r = j - __builtin_amdgcn_readlane(start, b);
    return WorkItem{b, r % H, __builtin_amdgcn_readlane(nv, b) + r / H};
  }
  template <class RowLen, class StreamLen>
  static __device__ __forceinline__ WorkItem by_stream(int id, int B, int H, RowLen rows, int RB, int nlev,
                                                       StreamLen stream) {
    const int lane = __lane_id();
    const int nv = row_blocks(rows, RB, B, lane);
    const int key = lane < B ? stream(lane) : -1;
    const int cnt = nv * H;
    int rank = 0, total = 0;
    for (int k = 0; k < B; ++k) {
      const int kk = __builtin_amdgcn_readlane(key, k);
      rank += (kk > key || (kk == key && k < lane)) ? 1 : 0;
      total += __builtin_amdgcn_readlane(cnt, k);
    }
    if (id >= total) return padding(id - total, B, H, nv, nlev);
    int start = 0;
    for (int k = 0; k < B; ++k) {
      const int rk = __builtin_amdgcn_readlane(rank, k), ck = __builtin_amdgcn_readlane(cnt, k);
      start += rk < rank ? ck : 0;
    }
    const uint64_t m = __ballot(lane < B && id >= start && id < start + cnt);
    const int b = __builtin_ctzll(m);
#if SIGATTN_STREAM_GROUPED
    const int r = xcd_grouped(id, __builtin_amdgcn_readlane(start, b), __builtin_amdgcn_readlane(cnt, b));
    const int nvb = __builtin_amdgcn_readlane(nv, b);
    return WorkItem{b, r / nvb, r % nvb};
#else
    const int r = id - __builtin_amdgcn_readlane(start, b);
    return WorkItem{b, r % H, r / H};
#endif
  }
  // Position, in head-major order (head, then row block), of the unit that
  // workgroup `id` runs among the `cnt` equal units of one batch starting at
  // id `start`: the ids the hardware deals to one XCD (id % 8) take a
  // contiguous range, so an XCD works through few heads at a time and their
  // streamed rows stay in its L2.
  static __device__ __forceinline__ int xcd_grouped(int id, int start, int cnt) {
    const int x = id & 7, s8 = start & 7;
    int base = 0;
    for (int y = 0; y < x; ++y) {
      const int p0 = (y - s8 + 8) & 7;
      base += p0 < cnt ? (cnt - p0 + 7) >> 3 : 0;
    }
    const int p0 = (x - s8 + 8) & 7;
    return base + ((id - start - p0) >> 3);
  }
  // Position in the heaviest-first order of the item that workgroup `id`
  // runs, out of n.  The hardware places workgroup ids breadth-first over
  // the S compute units (ids kS .. kS+S-1 form round k, one per CU, while
  // the slots are free), so in the plain order every round placed at launch
  // (the first `occ`, the kernel's workgroups per CU) gives its heaviest item
  // to the same CUs; dealt in reverse, a round gives the CU that ran a
  // round's heaviest item its lightest (SIGATTN_LEVEL_DEAL: 0 plain, 1 odd
  // rounds reversed, 2 every round after the first reversed).  Later rounds
  // start as slots free and keep the heaviest-first order.
  static __device__ __forceinline__ int dealt(int id, int n, int S, int occ) {
    if (SIGATTN_LEVEL_DEAL == 0 || S <= 0 || id >= n) return id;
    const int k = id / S, j = id - k * S, m = min(S, n - k * S);
    const bool rev = k < occ && (SIGATTN_LEVEL_DEAL == 1 ? (k & 1) != 0 : k > 0);
    return rev ? k * S + (m - 1 - j) : id;
  }
  template <class RowLen>
  static __device__ __forceinline__ WorkItem by_level(int id, int B, int H, RowLen rows, int RB, int nlev,
                                                      bool descending, int ncu = 0, int occ = 1) {
    const int lane = __lane_id();
    const int nv = row_blocks(rows, RB, B, lane);
    if (SIGATTN_LEVEL_DEAL != 0 && occ > 1) {
      int total = 0;
      for (int k = 0; k < B; ++k) total += __builtin_amdgcn_readlane(nv, k);
      id = dealt(id, total * H, ncu, occ);
    }
    int base = 0;
    for (int t = 0; t < nlev; ++t) {
      const int lev = descending ? nlev - 1 - t : t;
      const uint64_t m = __ballot(nv > lev);
      const int cnt = __builtin_popcountll(m) * H;
      if (id < base + cnt) {
        const int r = id - base;
        return WorkItem{kth_set_bit(m, r / H), r % H, lev};
      }
      base += cnt;
    }
    return padding(id - base, B, H, nv, nlev);
  }
};

// Dense grids (every (batch, head) pair has the same `nper` row blocks): the
// pair and row block of workgroup `id`.  The hardware deals workgroup ids
// round-robin over the 8 XCDs, each with its own L2, and each XCD starts its
// ids in order.
//   * Equal items (grouped): XCD x gets the consecutive pairs x*BH/8 .. , all
//     row blocks of one pair back to back, so the rows those blocks share (K
//     and V, or Q and dO) are read while they sit in one L2; with `id % BH`
//     as the pair, every XCD would cycle through BH/8 pairs at once.
//   * Unequal items (causal, !grouped): `id % BH`, `id / BH`, so that every
//     XCD starts the row-block levels in the order the caller maps them to
//     (heaviest first); grouping pairs there broke that order and made the
//     causal kernels slower (measured at B=4 L=4096 H=16 D=128: dQ from dS
//     0.254 -> 0.322 ms, forward 0.30 -> 0.33 ms).  Causal kernels whose
//     workgroups each run a pair of row blocks with equal total work (the
//     D = 128 dK/dV kernel) use the grouped order.
// B*H not a multiple of 8 keeps the plain order.
__device__ __forceinline__ void dense_item(int id, int BH, int nper, bool grouped, int &bh, int &blk) {
  if (!grouped || BH % 8 != 0) {
    bh = id % BH;
    blk = id / BH;
    return;
  }
  const int j = id >> 3;
  bh = (id & 7) * (BH >> 3) + j / nper;
  blk = j % nper;
}

// ---------------------------------------------------------------------------
// dS workspace of the two-pass backward.  dS of (batch, head) is cut into
// 32-query x 32-key tiles of 2 KB, stored column by column (key block kb,
// then query block qb), so the tiles one dQ workgroup reads for one key block
// (its consecutive query blocks) are contiguous, and so are the tiles one
// dK/dV wave writes for consecutive query blocks.  Causal problems keep only
// the tiles that hold a visible pair (qb >= kb: column kb holds qb = kb ..
// nqb-1); the others keep all nqb x nkb.
// Inside a tile, lane l of the dK/dV kernel's accumulator layout (key l % 32,
// query half h = l / 32) holds the 16-bit dS of queries {8g + 4h + i : g =
// 0..3, i = 0..3}; piece c (g = 2c, 2c + 1, 16 bytes in (g, i) order) is
// stored at byte 1024 c + 16 l, so each of the two store instructions writes
// 1 KB of whole cache lines, and each group of four consecutive queries of one
// key is one aligned 8-byte word.
struct DsLayout {
  static constexpr int kTileElems = 1024;
  static __device__ __forceinline__ int64_t per_bh(int nqb, int nkb, bool causal) {
    return causal ? (int64_t)nqb * (nqb + 1) / 2 : (int64_t)nqb * nkb;
  }
  // Tile index of (query block qb, key block kb) relative to the (b, h) base
  // (causal: requires kb <= qb).
  static __device__ __forceinline__ int64_t tile(int qb, int kb, int nqb, bool causal) {
    const int64_t col = causal ? (int64_t)kb * nqb - (int64_t)kb * (kb - 1) / 2 : (int64_t)kb * nqb;
    return col + (causal ? qb - kb : qb);
  }
};

// sigmoid(s*scale + c) given x = s*(-scale*log2e) + (-c*log2e) (one FMA
// before this call).  Hardware exp2 and reciprocal; x = +inf gives exactly 0.
__device__ __forceinline__ float sigmoid_from_neg_log2(float x) {
  return __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(x));
}

// Element-type traits: MFMA call and fp32 -> element conversions (RNE).
template <typename T> struct Elem;

template <> struct Elem<__bf16> {
  static __device__ __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                   __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, bf16x2));
  }
  static __device__ __forceinline__ float to_f32(uint16_t bits) {
    return __builtin_bit_cast(float, (uint32_t)bits << 16);
  }
  static __device__ __forceinline__ uint16_t from_f32(float x) {
    return (uint16_t)(pack(x, 0.0f) & 0xffffu);
  }
};

template <> struct Elem<_Float16> {
  static __device__ __forceinline__ f32x16 mfma(u32x4 a, u32x4 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a),
                                                  __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, f16x2));
  }
  static __device__ __forceinline__ float to_f32(uint16_t bits) {
    return (float)__builtin_bit_cast(_Float16, bits);
  }
  static __device__ __forceinline__ uint16_t from_f32(float x) {
    return __builtin_bit_cast(uint16_t, (_Float16)x);
  }
};

template <> struct Elem<float> {
  static __device__ __forceinline__ float to_f32(float x) { return x; }
};

// Round an fp32 value to the element type and back (P and dS are rounded to
// the I/O dtype before their second product, as the reference kernels do).
template <typename T> __device__ __forceinline__ float round_to(float x) {
  return Elem<T>::to_f32(Elem<T>::from_f32(x));
}
template <> __device__ __forceinline__ float round_to<float>(float x) { return x; }

// Gather element `e` (0..7) of four 16-byte rows into one 8-byte word
// (row r in 16-bit lane r).
__device__ __forceinline__ u32x2 gather4(const u32x4 &r0, const u32x4 &r1, const u32x4 &r2,
                                         const u32x4 &r3, int e) {
  const int w = e >> 1;
  const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
  u32x2 out;
  out.x = __builtin_amdgcn_perm(r1[w], r0[w], sel);
  out.y = __builtin_amdgcn_perm(r3[w], r2[w], sel);
  return out;
}

// Same for two rows into one 4-byte word.
__device__ __forceinline__ uint32_t gather2(const u32x4 &r0, const u32x4 &r1, int e) {
  const int w = e >> 1;
  const uint32_t sel = (e & 1) ? 0x07060302u : 0x05040100u;
  return __builtin_amdgcn_perm(r1[w], r0[w], sel);
}

__device__ __forceinline__ u32x4 zero4() { return (u32x4){0u, 0u, 0u, 0u}; }

// Calls f(std::integral_constant<int, I>) for I = B .. E-1 in order, inlined.
template <int B, int E> struct Unroll {
  template <class F> static __device__ __forceinline__ void run(F &&f) {
    if constexpr (B < E) {
      f(std::integral_constant<int, B>{});
      Unroll<B + 1, E>::run(f);
    }
  }
};

__device__ __forceinline__ f32x16 zero16() {
  f32x16 z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.0f;
  return z;
}


// Reads one accumulator element that lives in an AGPR into a VGPR at this
// point of the instruction stream.  The MFMA accumulators of the kernels sit
// in AGPRs; left to itself the compiler copies a whole accumulator to VGPRs
// in one burst (stalling the matrix pipe and holding 16 extra VGPRs), while
// this spreads the copies over the VALU work that consumes them.  Callers
// only read elements whose MFMA finished several MFMAs earlier.
__device__ __forceinline__ float acc_read(float v) {
  float out;
  asm volatile("v_accvgpr_read_b32 %0, %1" : "=v"(out) : "a"(v));
  return out;
}

// ---------------------------------------------------------------------------
// Swizzled LDS tiles.  A [rows][D] tile of 16-bit elements is stored without
// padding; its 16-byte chunk c of row r lives at chunk position c ^ swz(r).
// With swz(r) = 4*(r&3) + ((r>>2)&3) (D = 128, 16 chunks per row) every access
// pattern the kernels use is bank-conflict free on gfx950 (measured with
// SQ_LDS_BANK_CONFLICT): 16-byte operand reads of 32 consecutive rows, the
// 4-row x 32-column ds_read_b64_tr_b16 groups, and chunk-major 16-byte stores.
// D = 64 (8 chunks per row, two rows per 64-bank line) uses
// swz(r) = 4*((r>>1)&1) + ((r>>2)&3), and D = 32 (4 chunks per row, four
// rows per line) swz(r) = (r>>2)&3: in each case any 16 consecutive rows read
// at one logical chunk land on 16 distinct 16-byte slots of a line.
template <int D> __host__ __device__ __forceinline__ int swz(int row) {
  if constexpr (D >= 128) return 4 * (row & 3) + ((row >> 2) & 3);
  else if constexpr (D == 64) return 4 * ((row >> 1) & 1) + ((row >> 2) & 3);
  else return (row >> 2) & 3;
}
// Element offset of (row, col) in a swizzled tile.
template <int D> __device__ __forceinline__ int toff(int row, int col) {
  return row * D + ((((col >> 3) ^ swz<D>(row)) << 3) | (col & 7));
}

// Stages a ROWS x D tile (rows `row0 ..` of a tensor with row stride
// `stride`, elements) into a swizzled LDS tile through registers.  Thread t
// owns chunks t, t+256, ... in row-major chunk order, so a wave loads whole
// rows (coalesced) and stores them conflict-free.  Rows at or past `nvalid`
// are zero-filled and never read from memory.
template <int ROWS, int D> struct TileStager {
  static constexpr int CPR = D / 8;                 // 16-byte chunks per row
  static constexpr int RPT = ROWS * CPR / 256;      // chunks per thread
  static_assert(RPT >= 1 && ROWS * CPR % 256 == 0, "tile shape");
  u32x4 r[RPT];

  __device__ __forceinline__ void load(const uint16_t *base, int64_t stride, int row0, int nvalid,
                                       int tid) {
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      const int c = tid + 256 * i;
      const int row = c / CPR, ch = c % CPR;
      r[i] = (row0 + row) < nvalid
                 ? *(const u32x4 *)(base + (int64_t)(row0 + row) * stride + 8 * ch)
                 : zero4();
    }
  }
  __device__ __forceinline__ void store(uint16_t *lds, int tid) const {
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      const int c = tid + 256 * i;
      const int row = c / CPR, ch = c % CPR;
      *(u32x4 *)&lds[toff<D>(row, 8 * ch)] = r[i];
    }
  }
};

// Loads rows [row0, row0 + ROWS) of a [*, D] tensor (row stride `stride`
// elements) into the swizzled LDS tile `lds` with direct global->LDS DMA
// (global_load_lds_dwordx4: lane i of a wave writes LDS bytes base + 16 i), so
// no VGPRs hold the tile in flight.  Each wave-instruction fills 1 KB = 512/D
// whole rows; lane i lands on physical chunk i % (D/8) of its row and
// therefore fetches logical chunk (i % (D/8)) ^ swz(row).  Rows at or past
// `nvalid` fetch row nvalid-1 instead (in bounds, finite); callers mask them.
// Requires nvalid >= 1.  Completion is tracked by vmcnt: wait_dma() and a
// barrier must precede reads of the tile.
// The per-lane part (tile row and swizzled chunk byte offset of each of this
// wave's instructions) is computed once; a tile load then costs one min and
// one multiply-add per instruction, with a uniform (SGPR) base pointer and a
// 32-bit byte offset (callers guarantee rows * stride * 2 < 2^31).
template <int ROWS, int D, int NWAVES> struct DmaPlan {
  static constexpr int CPR = D / 8;           // chunks per row
  static constexpr int RPI = 64 / CPR;        // rows per wave-instruction
  static constexpr int NI = ROWS / RPI / NWAVES;  // instructions per wave per tile
  static_assert(ROWS % (RPI * NWAVES) == 0, "tile shape");
  int row[NI];       // tile-relative row of this lane's chunk
  int cbyte[NI];     // byte offset of the swizzled source chunk within its row
  int r0[NI];        // first tile row of each instruction (wave-uniform)

  // half: the row holds D / 2 elements (head_dim 16 in a D = 32 tile); the
  // tile's upper chunks repeat its lower ones.
  __host__ __device__ __forceinline__ void init(int wave, int lane, bool half = false) {
    const int cmask = half ? CPR / 2 - 1 : CPR - 1;
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      r0[i] = (wave * NI + i) * RPI;
      row[i] = r0[i] + lane / CPR;
      cbyte[i] = 16 * (((lane % CPR) ^ swz<D>(row[i])) & cmask);
    }
  }
  // base: uniform pointer to row 0 of the (batch, head) slice.
  //
  // The copy is issued through inline asm rather than the global_load_lds
  // builtin: the compiler cannot tell the ring stages apart, so after the
  // builtin it waits for the whole copy (vmcnt(0)) before the next LDS read
  // of any stage, which serialises the prefetch with the compute it should
  // overlap.  The kernels wait for the copy themselves (wait_dma() and a
  // barrier) before any wave reads the stage it fills.
  __device__ __forceinline__ void issue(uint16_t *lds, const uint16_t *base, int stride_bytes,
                                        int row0, int nvalid) const {
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      const int g = min(row0 + row[i], nvalid - 1);
      const uint32_t off = (uint32_t)g * (uint32_t)stride_bytes + (uint32_t)cbyte[i];
      // The low 32 bits of a generic LDS pointer are its LDS offset.
      const uint32_t dst = __builtin_amdgcn_readfirstlane((uint32_t)(uintptr_t)(lds + r0[i] * D));
      // M0 holds the LDS destination; s_nop covers the M0-write -> LDS-DMA wait state.
      asm volatile("s_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
                   :
                   : "v"(off), "s"(base), "{m0}"(dst)
                   : "memory");
    }
  }
};

// fp32 tiles of rows x D floats in LDS, filled by DmaPlan<rows, 2D, waves>
// (the same bytes as a 16-bit tile of 2D elements): 16-byte piece c of row
// r sits at piece c ^ swz<2D>(r), so each group of 16 rows read at one piece
// position covers every bank once.  Offsets are in floats.
template <int D> struct F32Tile {
  static __host__ __device__ __forceinline__ int piece(int r, int c) { return r * D + 4 * (c ^ swz<2 * D>(r)); }
  static __host__ __device__ __forceinline__ int elem(int r, int d) { return piece(r, d >> 2) + (d & 3); }
};

// Per-lane offsets of the fp32 kernels' row-product reads: element
// (8g + 4hi + r, 32db + l32) of an F32Tile, for lane l32 + 32hi and every
// (g, r, db), is o[g & 1][j] plus a compile-time constant (j = r & 1 when
// D >= 64, r >> 1 when D = 32).  The swizzle term there splits as
// swz<2D>(8g + 4hi + r) = 8(r >> 1) + 4(r & 1) + m (D >= 64) or 4(r >> 1) + m
// (D = 32) with m = (2g + hi) & 3 depending on g only through g & 1, and its
// bits above 2 only move whole 32-float column blocks (db ^ (r >> 1)).
template <int D> struct F32RowReads {
  int o[2][2];
  __host__ __device__ __forceinline__ void init(int l32, int hi) {
    const int x = l32 >> 2;
#pragma unroll
    for (int gp = 0; gp < 2; ++gp)
#pragma unroll
      for (int j = 0; j < 2; ++j)
        o[gp][j] = 4 * hi * D + 4 * (x ^ ((2 * gp + hi) & 3) ^ (4 * j)) + (l32 & 3);
  }
  __host__ __device__ __forceinline__ int at(int g, int r, int db) const {
    const int j = D >= 64 ? (r & 1) : (r >> 1);
    return o[g & 1][j] + (8 * g + r) * D + (D >= 64 ? 32 * (db ^ (r >> 1)) : 0);
  }
};

__device__ __forceinline__ void wait_dma() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Waits until at most N vector-memory operations of this wave are in flight
// (they complete in issue order, so everything older than the N most recent
// has completed).
template <int N> __device__ __forceinline__ void wait_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
  asm volatile("" ::: "memory");
}

// Waits until at most n * STEP operations are in flight (0 <= n <= N, n known
// only at run time).
template <int STEP, int N> __device__ __forceinline__ void wait_vm_steps(int n) {
  if constexpr (N == 0) {
    wait_vm<0>();
  } else {
    if (n >= N) wait_vm<N * STEP>();
    else wait_vm_steps<STEP, N - 1>(n);
  }
}

// Word 3 of a gfx9 buffer resource for raw (untyped, stride 0) access:
// accesses at or past num_records bytes are dropped.
constexpr int kBufferWord3 = 0x00020000;
// Cache-policy operand of the buffer builtins: non-temporal (streaming) store,
// for data the writing kernel never reads back (measured: the dS stream of
// the two-pass backward costs the dK/dV kernel 0.10 ms at the headline shape
// with it, 0.16 ms without).
constexpr int kStoreNT = 2;

// Chunk c of n of a range of nt tiles: tiles [c*nt/n, (c+1)*nt/n).
// (c < n <= 8 and nt < 2^26, so 32-bit arithmetic; wave-uniform, kept in an
// SGPR for the tile copies' base addresses.)
__device__ __forceinline__ int split_tile(int c, int n, int nt) {
  return __builtin_amdgcn_readfirstlane(c * nt / n);
}

// Most chunks a range-split item runs as (KParams::rsplit).
constexpr int kRangeSplitMax = 4;

// End of a range-split work item (KParams::rsplit): the workgroup's fp32
// accumulators -- NACC f32x16 per lane, acc(i) -- become the item's final
// sum, or the workgroup learns that another chunk will write the output.
// Every chunk stores its accumulators to its slot of the item's partials
// (lane-major, 1 KB per store instruction) and, once the workgroup's stores
// have completed, counts itself in; the workgroup whose count completes the
// item adds all n partials in chunk order, its own from registers, so the sum
// does not depend on which chunk finishes last.  The other chunks' partials
// are loaded two accumulators at a time with every chunk's loads in flight
// together (one memory round trip per pair, not one per chunk).
//
// Ordering follows the HIP (HSA) memory model at agent scope, because the
// chunks of an item may run on different XCDs, each with its own L2: the
// counter is an acquire-release agent-scope atomic, so every chunk's partial
// stores (made workgroup-visible by __syncthreads before thread 0's release)
// happen before the last chunk's loads (after its acquire and a second
// __syncthreads).  On gfx950 the compiler lowers that release to buffer_wbl2
// sc1 + s_waitcnt vmcnt(0) and the acquire to buffer_inv sc1.  The partials
// themselves move with agent-coherent (sc1) buffer accesses -- the lowering
// of agent-scope relaxed atomic stores and loads -- which write through past
// the L2 and so leave the release's L2 write-back little to do: measured at
// B=2 L=1024 H=8 D=64 (forward / backward, us), relaxed counter with sc1
// accesses 17.4 / 43.7, this protocol 19.6 / 49.6, plain accesses with the
// acquire-release counter 22.4 / 61.0.  (A full agent-scope fence,
// __threadfence, made a split forward 2.3x slower.)
// Returns false when this workgroup should exit without writing.
template <int NACC, int NW, class Acc>
__device__ __forceinline__ bool split_combine(Acc &&acc, float *part_item, int *cnt, int chunk, int n, int w,
                                              int lane) {
  constexpr int kCoherent = 16;  // cache-policy operand of the buffer builtins: sc1
  constexpr int kWaveBytes = NACC * 4 * 1024;
  constexpr int G = NACC % 2 == 0 ? 2 : 1;  // accumulators per round trip
  constexpr int kOthers = kRangeSplitMax - 1;
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      (void *)part_item, (short)0, n * NW * kWaveBytes, kBufferWord3);
  const int mine = (chunk * NW + w) * kWaveBytes + 16 * lane;
#pragma unroll
  for (int i = 0; i < NACC; ++i)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const f32x16 &a = acc(i);
      const f32x4 v = {a[4 * g], a[4 * g + 1], a[4 * g + 2], a[4 * g + 3]};
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, v), rs, mine + (4 * i + g) * 1024, 0,
                                             kCoherent);
    }
  __shared__ int arrived;
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0) arrived = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
  __syncthreads();
  if (arrived != n - 1) return false;
  asm volatile("" ::: "memory");
  // Slot j of `other` holds chunk j (j < chunk) or chunk j + 1 (j >= chunk).
  int off[kOthers];
#pragma unroll
  for (int j = 0; j < kOthers; ++j) off[j] = ((j < chunk ? j : j + 1) * NW + w) * kWaveBytes + 16 * lane;
#pragma unroll
  for (int i0 = 0; i0 < NACC; i0 += G) {
    f32x4 other[kOthers][G][4];
#pragma unroll
    for (int j = 0; j < kOthers; ++j)
      if (j + 1 < n)  // wave-uniform: chunk count
#pragma unroll
        for (int ii = 0; ii < G; ++ii)
#pragma unroll
          for (int g = 0; g < 4; ++g)
            // Whole-vector casts: hipcc 7.2 compiles a __builtin_bit_cast of
            // a single ext_vector element as a read of element 0.
            other[j][ii][g] = __builtin_bit_cast(
                f32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, off[j] + (4 * (i0 + ii) + g) * 1024, 0, kCoherent));
#pragma unroll
    for (int ii = 0; ii < G; ++ii) {
      f32x16 &a = acc(i0 + ii);
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const f32x4 own = {a[4 * g], a[4 * g + 1], a[4 * g + 2], a[4 * g + 3]};
        f32x4 sum = chunk == 0 ? own : other[0][ii][g];
#pragma unroll
        for (int c = 1; c < kRangeSplitMax; ++c) {
          if (c >= n) break;
          // Chunk c's partial: own (c == chunk), slot c (c < chunk) or slot c - 1.
          const f32x4 below = other[c < kOthers ? c : kOthers - 1][ii][g];
          sum += c == chunk ? own : (c < chunk ? below : other[c - 1][ii][g]);
        }
        a[4 * g] = sum.x, a[4 * g + 1] = sum.y, a[4 * g + 2] = sum.z, a[4 * g + 3] = sum.w;
      }
    }
  }
  return true;
}

// Per-lane element offsets into swizzled [*, D] tiles, computed once per
// kernel.  A row offset that is a multiple of 16 rows leaves swz() unchanged,
// so such offsets (tile stages, 16-row k-steps, 32-row blocks) are added as
// compile-time constants and fold into the ds_read immediate.
template <int D> struct TileOffsets {
  int row_op[D / 16];   // 16-byte operand at row l%32, k-step ks (read_row_operand)
  int tr_op[D / 32][2]; // tr16 reads for column block db, first / second 4-row group
  __device__ __forceinline__ void init(int lane) {
    const int l32 = lane & 31, hi = lane >> 5;
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) row_op[ks] = toff<D>(l32, 16 * ks + 8 * hi);
    const int grp = lane >> 4, s = lane & 15;
    const int row = 4 * (grp >> 1) + (s >> 2);
#pragma unroll
    for (int db = 0; db < D / 32; ++db) {
      const int col = db * 32 + 16 * (grp & 1) + 4 * (s & 3);
      tr_op[db][0] = toff<D>(row, col);
      tr_op[db][1] = toff<D>(row + 8, col);
    }
  }
};

// Operand read at row (row16 + l%32) where row16 is a multiple of 16.
template <int D>
__device__ __forceinline__ u32x4 ld_row(const uint16_t *lds, const TileOffsets<D> &o, int row16,
                                        int ks) {
  return *(const u32x4 *)&lds[row16 * D + o.row_op[ks]];
}

// Transposed operand (see read_tr16_operand) for k-step ks, column block db.
template <int D>
__device__ __forceinline__ u32x4 ld_tr(const uint16_t *lds, const TileOffsets<D> &o, int ks, int db) {
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  const uint16_t *base = lds + 16 * ks * D;
  const s16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4 *)(base + o.tr_op[db][0]));
  const s16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4 *)(base + o.tr_op[db][1]));
  const u32x2 lo = __builtin_bit_cast(u32x2, a);
  const u32x2 hv = __builtin_bit_cast(u32x2, b);
  return (u32x4){lo.x, lo.y, hv.x, hv.y};
}

// 16-byte MFMA operand read from a swizzled tile: row `row`, k-elements
// 16*ks + 8*hi .. +7 (k = 8h + j mapping).
template <int D>
__device__ __forceinline__ u32x4 read_row_operand(const uint16_t *lds, int row, int ks, int hi) {
  return *(const u32x4 *)&lds[toff<D>(row, 16 * ks + 8 * hi)];
}

// Transposed MFMA operand read from a swizzled tile X[k][n] (see
// read_tr16_operand for the lane mapping).
template <int D>
__device__ __forceinline__ u32x4 read_tr16_swz(const uint16_t *lds, int n0, int ks, int lane) {
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  const int grp = lane >> 4, s = lane & 15;
  const int row = 16 * ks + 4 * (grp >> 1) + (s >> 2);
  const int col = n0 + 16 * (grp & 1) + 4 * (s & 3);
  const s16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4 *)(lds + toff<D>(row, col)));
  const s16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4 *)(lds + toff<D>(row + 8, col)));
  const u32x2 lo = __builtin_bit_cast(u32x2, a);
  const u32x2 hv = __builtin_bit_cast(u32x2, b);
  return (u32x4){lo.x, lo.y, hv.x, hv.y};
}

// Stages a ROWS x D tile of 16-bit elements (rows `row0 ..` of a [T, *, D]
// tensor with row stride `stride`) through registers into LDS.  Each of the
// 256 threads owns RPT consecutive rows x 8 columns, so the same registers can
// be written row-major (pitch NP, 16-byte stores) and/or transposed
// ([D][ROWS] with pitch TP, one 4- or 8-byte store per column).  Rows at or
// past `nvalid` are zero-filled and never read from memory.
template <int ROWS, int D> struct Stager {
  static constexpr int RPT = ROWS * D / (8 * 256);
  static constexpr int RG = ROWS / RPT;
  static_assert(RPT == 2 || RPT == 4, "tile shape");
  u32x4 r[RPT];

  __device__ __forceinline__ void load(const uint16_t *base, int64_t stride, int row0, int nvalid,
                                       int tid) {
    const int rg = tid % RG, g = tid / RG;
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      const int row = row0 + rg * RPT + i;
      r[i] = row < nvalid ? *(const u32x4 *)(base + (int64_t)row * stride + 8 * g) : zero4();
    }
  }
  template <int NP> __device__ __forceinline__ void store_nat(uint16_t *lds, int tid) const {
    const int rg = tid % RG, g = tid / RG;
#pragma unroll
    for (int i = 0; i < RPT; ++i) *(u32x4 *)&lds[(rg * RPT + i) * NP + 8 * g] = r[i];
  }
  template <int TP> __device__ __forceinline__ void store_tr(uint16_t *lds, int tid) const {
    const int rg = tid % RG, g = tid / RG;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      uint16_t *dst = &lds[(8 * g + e) * TP + rg * RPT];
      if constexpr (RPT == 4) *(u32x2 *)dst = gather4(r[0], r[1], r[2], r[3], e);
      else *(uint32_t *)dst = gather2(r[0], r[1], e);
    }
  }
};

// MFMA operand read of a row-major LDS tile X[k][n] (pitch NP elements) for
// an operand that needs k along the eight elements of a lane and n = column
// (n0 + l % 32), with the key/query permutation of the C-layout-as-B-operand
// trick: element j of lane l is k = 16*ks + 4h + j (j < 4) or
// 16*ks + 8 + 4h + (j - 4) (j >= 4), h = l / 32.
//
// ds_read_b64_tr_b16 (gfx950): inside each group of 16 lanes, the four
// 16-bit elements read by source lane s form row s of a 16x4 matrix M, and
// lane i receives M[4e + i/4][i%4] as element e.  Source lane s = 4e + m of a
// group therefore supplies &X[k(e)][n_group + 4m]; lane i then holds column
// n_group + i for the four k(e).  Two such reads give the eight elements.
template <int NP>
__device__ __forceinline__ u32x4 read_tr16_operand(const uint16_t *lds, int n0, int ks, int lane) {
  typedef short s16x4 __attribute__((ext_vector_type(4)));
  const int grp = lane >> 4, s = lane & 15;
  const int h = grp >> 1;
  const int row = 16 * ks + 4 * h + (s >> 2);
  const int col = n0 + 16 * (grp & 1) + 4 * (s & 3);
  const uint16_t *p = lds + row * NP + col;
  const s16x4 a = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4 *)(p));
  const s16x4 b = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) s16x4 *)(p + 8 * NP));
  const u32x2 lo = __builtin_bit_cast(u32x2, a);
  const u32x2 hv = __builtin_bit_cast(u32x2, b);
  return (u32x4){lo.x, lo.y, hv.x, hv.y};
}

// A-operand read of a transposed tile ([D][rows] in LDS, pitch TP): row
// `drow`, eight k-elements at rows 16*ks + 4h + {0..3} and 16*ks + 8 + 4h +
// {0..3} — the key/query permutation of the C-layout-as-B-operand trick.
template <int TP>
__device__ __forceinline__ u32x4 read_tr_operand(const uint16_t *lds, int drow, int ks, int hi) {
  const uint16_t *p = lds + drow * TP + 16 * ks + 4 * hi;
  const u32x2 lo = *(const u32x2 *)p;
  const u32x2 hv = *(const u32x2 *)(p + 8);
  return (u32x4){lo.x, lo.y, hv.x, hv.y};
}

}  // namespace sigattn
