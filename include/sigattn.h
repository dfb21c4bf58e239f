/*
 * sigattn.h — C ABI of the MI355X (gfx950) fused sigmoid-attention library
 * (libsigattn.so).
 *
 *   O = sigmoid(Q·Kᵀ·scale + bias[b] + score_mod[b, key]) · V
 *
 * with optional top-left causal masking (key <= query) and right padding
 * (only the first seq_lens_q[b] queries / seq_lens_k[b] keys of batch b are
 * valid), plus the recompute backward (dQ, dK, dV).  Tensors are [B, T, H, D]
 * with unit stride along D.  All pointers are device pointers; nothing here
 * allocates, synchronises the host or throws across the ABI.
 *
 * These entry points replace the kernel launches inside the reference's four
 * torch.library ops (MSDLLCpapers/triton-sigmoid, src/triton_sigmoid/):
 *   sigattn_fwd  <- sigmoid_triton_dense.py:534-560   (_fwd_dense_kernel launch)
 *                <- sigmoid_triton_padded.py:591-621  (_fwd_padded_kernel launch)
 *   sigattn_bwd  <- sigmoid_triton_dense.py:630-686   (dQ + dK/dV launches)
 *                <- sigmoid_triton_padded.py:706-770  (dQ + dK/dV launches)
 * The Python op layer (torch.library custom ops with the reference's names
 * and schemas) calls them through ctypes with torch's current HIP stream.
 */
#ifndef SIGATTN_H
#define SIGATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SIGATTN_ABI_VERSION 2

/* Element type of Q, K, V, dO and of every output. */
enum sigattn_dtype {
  SIGATTN_F16 = 0,
  SIGATTN_BF16 = 1,
  SIGATTN_F32 = 2
};

/* Return codes: 0 on success, negative on error (see sigattn_strerror). */
enum sigattn_status {
  SIGATTN_OK = 0,
  SIGATTN_ERR_NULL_ARG = -1,      /* a required pointer is NULL */
  SIGATTN_ERR_DTYPE = -2,         /* dtype code not in enum sigattn_dtype */
  SIGATTN_ERR_HEAD_DIM = -3,      /* D not in {16, 32, 64, 128} */
  SIGATTN_ERR_SHAPE = -4,         /* negative size, or B*H / T too large */
  SIGATTN_ERR_STRIDE = -5,        /* negative stride */
  SIGATTN_ERR_DENSE_LENGTHS = -6, /* dense call (no seq_lens) with Tq != Tk */
  SIGATTN_ERR_ABI_VERSION = -7,   /* problem.abi_version != SIGATTN_ABI_VERSION */
  SIGATTN_ERR_LAUNCH = -8,        /* hipGetLastError() reported a failure */
  SIGATTN_ERR_LAYOUT = -9,        /* seq_lens and cu_seqlens both set for one axis */
  SIGATTN_ERR_WORKSPACE = -10,    /* workspace too small for the call, or misaligned */
  SIGATTN_ERR_SCRATCH = -11       /* sigattn_fwd_noalloc: scratch need above
                                     SIGATTN_NOALLOC_SCRATCH_BYTES */
};

/*
 * One attention problem.  Strides are in elements; the D stride is 1.
 * Q, O, dO and dQ share the q_stride_* layout; K, V, dK and dV share the
 * k_stride_* layout (the reference passes exactly these two stride sets to
 * every kernel: sigmoid_triton_dense.py:505-506).
 */
typedef struct sigattn_problem {
  int32_t abi_version;    /* must be SIGATTN_ABI_VERSION */
  int32_t dtype;          /* enum sigattn_dtype */
  int64_t B, Tq, Tk, H, D;
  int64_t q_stride_b, q_stride_t, q_stride_h;
  int64_t k_stride_b, k_stride_t, k_stride_h;
  const void *q;          /* [B, Tq, H, D] */
  const void *k;          /* [B, Tk, H, D] */
  const void *v;          /* [B, Tk, H, D] */
  const float *bias;      /* [B] fp32, added after the scale */
  const float *scale;     /* 0-d fp32 device scalar (read by the kernels) */
  const float *score_mod; /* [B, Tk] fp32 contiguous, or NULL */
  const int32_t *seq_lens_q; /* [B] int32 or NULL; NULL with seq_lens_k NULL = dense */
  const int32_t *seq_lens_k; /* [B] int32 or NULL */
  int32_t causal;         /* nonzero: key index <= query index (top-left) */
  /*
   * Packed variable-length layout (no counterpart in the reference's API; it
   * is the layout its benchmark builds for flash_attn_varlen_func,
   * benchmarks/benchmark_sigmoid.py:116-134).  When cu_seqlens_q is set,
   * Q, O, dO and dQ are packed [rows_q, H, D] (q_stride_b is unused):
   * sequence b is rows cu_seqlens_q[b] .. cu_seqlens_q[b+1]-1, clamped to
   * [0, rows_q] and to at most Tq rows (Tq = the longest sequence), and
   * seq_lens_q must be NULL.  Likewise cu_seqlens_k / rows_k / Tk for K, V,
   * dK, dV; score_mod is then packed [rows_k].  Every row of a packed output
   * is written: rows that no sequence covers (before cu_seqlens[0], past
   * cu_seqlens[B], past Tq / Tk rows of a longer sequence) get zeros.
   */
  const int32_t *cu_seqlens_q; /* [B+1] int32 or NULL */
  const int32_t *cu_seqlens_k; /* [B+1] int32 or NULL */
  int64_t rows_q, rows_k;      /* packed row counts (used with cu_seqlens_*) */
} sigattn_problem;

/* ABI version compiled into the library. */
int sigattn_abi_version(void);

/* Human-readable text for a status code (static storage). */
const char *sigattn_strerror(int status);

/* Validates a problem without touching the GPU (0 or a negative status). */
int sigattn_check(const sigattn_problem *p);

/*
 * Forward: out[B, Tq, H, D] (q strides).  Rows at or past seq_lens_q[b] are
 * written as zeros (packed layout: rows outside every sequence are zeros).
 * `stream` is a hipStream_t (NULL = default stream).
 */
int sigattn_fwd(const sigattn_problem *p, void *out, void *stream);

/*
 * Split-KV forward for decode shapes (no counterpart in the reference, whose
 * forward has one workgroup per 16..128 queries of a (batch, head) however
 * few queries there are).  A non-causal f16/bf16 problem at head_dim 64 or
 * 128 with Tq <= 32 and Tk >= 256 taking the MFMA kernels cuts each (batch, head)'s keys into chunks, one
 * workgroup each, and sums the chunks' fp32 partials in a second kernel; the
 * partials need sigattn_fwd_workspace_bytes(p) bytes of device memory
 * (0 when the problem does not split).  sigattn_fwd_ws with workspace NULL (or
 * sigattn_fwd) runs the same kernel with one chunk per (batch, head), so no
 * workspace is touched.  The sum of fp32 partials is deterministic (fixed
 * chunks, fixed order) and matches sigattn_fwd within fp32 summation order.
 *
 * Range split of small dense grids (no counterpart in the reference): a
 * dense non-causal f16/bf16 problem at head_dim 64 or 128 taking the MFMA
 * kernels whose workgroups (one per
 * 128 or 256 queries of every (batch, head)) would leave at least half of
 * the GPU's compute units idle, runs each query block's keys as 2-4 chunks
 * of at least 512 keys in as many workgroups when the chunks save at least
 * 1024 keys of each block's range at head_dim 64 (512 at head_dim 128; so
 * T >= 1536 and T >= 1024), whose fp32 partials the last one to finish adds
 * in chunk order inside the same launch (an agent-scope acquire-release
 * counter orders the hand-over); sigattn_fwd_workspace_bytes then returns the
 * partials' size (it asks the current device for its compute-unit count, and
 * returns 0 without a device).  Deterministic, and equal to sigattn_fwd
 * within fp32 summation order.  A workspace too small for these partials (for
 * instance one sized for split-KV decode) or not 16-byte aligned is not an
 * error here: the problem then runs unsplit, exactly as in sigattn_fwd.  (A
 * split-KV problem given a workspace smaller than its partials still returns
 * SIGATTN_ERR_WORKSPACE.)
 */
size_t sigattn_fwd_workspace_bytes(const sigattn_problem *p);
int sigattn_fwd_ws(const sigattn_problem *p, void *out, void *workspace, size_t workspace_bytes,
                   void *stream);

/*
 * sigattn_fwd_ws without a caller workspace and without any allocation
 * (no counterpart in the reference): for callers that cannot allocate device
 * memory -- code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc.  Split-KV problems keep their fp32 partials in a fixed
 * device array inside the library, SIGATTN_NOALLOC_SCRATCH_BYTES per GPU,
 * held until the process ends; its address is looked up on the first call on
 * each device (which must be current).  Every split plan fits (partials stay
 * below 16 MiB); a larger need returns SIGATTN_ERR_SCRATCH.  Other problems
 * run exactly as in sigattn_fwd, without the range split of small dense
 * grids.  Results equal sigattn_fwd_ws's bit for bit, except on problems
 * that sigattn_fwd_ws range-splits, where they equal sigattn_fwd's bit for
 * bit and sigattn_fwd_ws's within fp32 summation order.
 * All calls on one GPU share its array: calls that overlap on one GPU (other
 * streams, other threads) race and must be serialised by the caller.
 */
#define SIGATTN_NOALLOC_SCRATCH_BYTES ((size_t)16 << 20)
int sigattn_fwd_noalloc(const sigattn_problem *p, void *out, void *stream);

/*
 * Recompute backward: dq (q strides), dk and dv (k strides) from dout
 * (q strides).  No atomics: results are bitwise deterministic.  Padded query
 * rows get dq = 0, padded key rows get dk = dv = 0.  Dense f16/bf16 problems
 * at head_dim <= 64 whose dQ and dK/dV grids (128 rows per workgroup)
 * together fit one workgroup per compute unit run both kernels' work as one
 * launch, bit-identical to the two launches.  Ragged (seq_lens or cu_seqlens)
 * non-causal f16/bf16 problems at head_dim 64 with at least eight 128-query
 * blocks per compute unit run the two kernels concurrently: the dK/dV kernel
 * on a second stream the library keeps per device (default priority),
 * forked off `stream` by an event and joined back by another, so the call
 * stays ordered on `stream` like any other; the events are the calling host
 * thread's own.  Under stream capture, or on a stream of another device than
 * the current one, both kernels stay on `stream`.
 * Results equal the sequential launches' bit for bit.
 */
int sigattn_bwd(const sigattn_problem *p, const void *dout, void *dq, void *dk,
                void *dv, void *stream);

/*
 * The recompute backward with the range split of small dense grids (no
 * counterpart in the reference): for a dense non-causal problem at head_dim
 * 64 or 128 taking the f16/bf16 MFMA kernels, whose dQ or dK/dV grid would leave at
 * least half of the GPU's compute units idle, the dQ kernel runs each query
 * block's keys and (head_dim 64) the dK/dV kernel each key block's queries
 * as 2-4 chunks of at least 512 rows, saving at least 1024 rows of each
 * range at head_dim 64 and 512 at 128 (so T >= 1536 and T >= 1024), the fp32
 * partials added in chunk order by the last chunk to finish, inside the
 * same launch.  sigattn_bwd_split_workspace_bytes(p) is the workspace it
 * needs (0 when nothing splits, or without a device); with workspace NULL
 * or when nothing splits, sigattn_bwd_split runs sigattn_bwd.  Results are
 * deterministic and equal sigattn_bwd's within fp32 summation order.  With
 * dq NULL (or dk and dv NULL) it runs only the other half, like
 * sigattn_bwd_dkdv (sigattn_bwd_dq), on the same workspace size.
 */
size_t sigattn_bwd_split_workspace_bytes(const sigattn_problem *p);
int sigattn_bwd_split(const sigattn_problem *p, const void *dout, void *dq, void *dk, void *dv,
                      void *workspace, size_t workspace_bytes, void *stream);

/*
 * The two halves of sigattn_bwd, one kernel each (the reference launches the
 * dQ kernel and the dK/dV kernel separately: sigmoid_triton_dense.py:630-656
 * and :659-686).  Used to time the kernels one at a time.
 */
int sigattn_bwd_dq(const sigattn_problem *p, const void *dout, void *dq, void *stream);
int sigattn_bwd_dkdv(const sigattn_problem *p, const void *dout, void *dk, void *dv,
                     void *stream);

/*
 * Two-pass backward (replaces the same two launches as sigattn_bwd,
 * sigmoid_triton_dense.py:630-686 and sigmoid_triton_padded.py:706-770; the
 * reference's dQ kernel recomputes S and dP, :162-307).  The dK/dV kernel
 * also stores dS, rounded to the I/O dtype exactly as the dQ product consumes
 * it, to a caller-owned workspace, and a second kernel computes
 * dQ = dS·K·scale from it, so no matrix product is computed twice.  The
 * workspace holds 2 bytes per (query, key) pair of every 32x32 block that has
 * a visible pair (causal: the lower triangle), per batch and head:
 * sigattn_bwd_workspace_bytes(p) for the whole problem, or 0 when the
 * problem has no two-pass form (fp32, D other than 64 or 128, misaligned
 * rows).  sigattn_bwd_ws with a smaller workspace runs the
 * heads in groups that fit, one group after another on `stream`; with room
 * for less than one head, or workspace NULL, it runs sigattn_bwd.  Results
 * equal sigattn_bwd's within fp32 summation order; the workspace must be
 * 16-byte aligned and is only used until the call's kernels finish.
 */
size_t sigattn_bwd_workspace_bytes(const sigattn_problem *p);
int sigattn_bwd_ws(const sigattn_problem *p, const void *dout, void *dq, void *dk, void *dv,
                   void *workspace, size_t workspace_bytes, void *stream);

/*
 * The two kernels of sigattn_bwd_ws, one launch each (used to time them one
 * at a time).  Both need the whole problem's workspace
 * (sigattn_bwd_workspace_bytes(p) bytes, else SIGATTN_ERR_WORKSPACE):
 * sigattn_bwd_dkdv_ws stores dS there, and sigattn_bwd_dq_ws, called after
 * it on the same stream with the same problem and workspace, reads it.
 */
int sigattn_bwd_dkdv_ws(const sigattn_problem *p, const void *dout, void *dk, void *dv,
                        void *workspace, size_t workspace_bytes, void *stream);
int sigattn_bwd_dq_ws(const sigattn_problem *p, void *dq, const void *workspace,
                      size_t workspace_bytes, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* SIGATTN_H */
