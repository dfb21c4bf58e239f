// Host-side launchers shared between the kernel files and the C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include "common.h"

namespace sigattn {

// Element type codes (same values as enum sigattn_dtype in include/sigattn.h).
constexpr int kF16 = 0;
constexpr int kBF16 = 1;
constexpr int kF32 = 2;

// Compute units of the current device (cached per device; 0 if unknown, e.g.
// without a GPU).  Defined with the C ABI.
int device_compute_units();

// Rows per workgroup and resident workgroups per CU of the MFMA forward and
// of the recompute backward's kernels (D in {64, 128}); the range split of
// small dense grids (KParams::rsplit) sizes itself from them.
int fwd_rows_per_workgroup(int D);
int fwd_workgroups_per_cu(int D);
int bwd_dq_rows_per_workgroup();
int bwd_dkdv_rows_per_workgroup();
int bwd_dq_workgroups_per_cu(int D);
int bwd_dkdv_workgroups_per_cu(int D);
// Zeroes two arrays of range-split arrival counters (na at a, nb at b) in
// one launch on `st` (a kernel: no memset node lands in a captured graph).
void launch_rs_clear(int *a, int na, int *b, int nb, hipStream_t st);

// MFMA kernels: dtype in {kF16, kBF16}, D in {32, 64, 128} (head_dim 16 as
// D = 32 with KParams::dmem = 16), 16-byte aligned rows.  The forward, dQ
// and dQ-from-dS launches (and the fp32 forward and dQ below) also run
// KParams::ngap leading workgroups that zero packed gap rows; the dK/dV
// launches take none.
void launch_fwd_mfma(const KParams &p, int dtype, int D, bool causal, bool scoremod,
                     hipStream_t st);
void launch_bwd_dq_mfma(const KParams &p, int dtype, int D, bool causal, bool scoremod,
                        hipStream_t st);
void launch_bwd_dkdv_mfma(const KParams &p, int dtype, int D, bool causal, bool scoremod,
                          bool dsout, hipStream_t st);
// Both recompute kernels in one launch: the first B·H·ceil(Tq/128)
// workgroups run dQ items, the rest dK/dV items (dense problems, D <= 64;
// bit-identical to launch_bwd_dq_mfma + launch_bwd_dkdv_mfma).
void launch_bwd_fused_mfma(const KParams &p, int dtype, int D, bool causal, bool scoremod, hipStream_t st);
// dQ = dS·K·scale from the dS tiles a launch_bwd_dkdv_mfma(dsout = true) on
// the same problem stored in p.ds (two-pass backward).
void launch_bwd_dq_ds_mfma(const KParams &p, int dtype, int D, bool causal, hipStream_t st);

// Split-KV forward (decode shapes: Tq <= 32, non-causal) with the MFMA
// kernels' requirements; p.nsplit / p.chunk set, p.ws holds
// nsplit * B * H * Tq * D floats when nsplit > 1.
void launch_fwd_splitkv(const KParams &p, int dtype, int D, bool scoremod, hipStream_t st);

// Fixed device scratch of the split-KV forward for callers that cannot
// allocate (sigattn_fwd_noalloc): a file-scope __device__ array of this many
// bytes in decode.hip, one per GPU, held until the process ends.  The split
// plan never needs more: fp32 partials of nsplit * B * H * Tq * D floats with
// nsplit * B * H < 1024 (splitting stops at 512 (batch, head) pairs), Tq <= 32
// and D <= 128 stay below 16 MiB.
constexpr size_t kSplitScratchBytes = size_t(16) << 20;
// Device address of the current device's scratch array (looked up once per
// device with hipGetSymbolAddress); hipSuccess or the lookup's error.
hipError_t splitkv_scratch(float **ptr);

// Zeroes the rows of packed outputs that no sequence covers, for two axes in
// one launch (an axis with rows = 0 takes no workgroups); esize = 2 or 4.
void launch_zero_gaps(const GapAxis &a, const GapAxis &b, int esize, hipStream_t st);

// fp32 kernels on the matrix cores (v_mfma_f32_32x32x2_f32): D in {32, 64,
// 128} (head_dim 16 as D = 32 with KParams::dmem = 16), 16-byte aligned rows.
void launch_fwd_f32(const KParams &p, int D, bool causal, bool scoremod, hipStream_t st);
void launch_bwd_dq_f32(const KParams &p, int D, bool causal, bool scoremod, hipStream_t st);
void launch_bwd_dkdv_f32(const KParams &p, int D, bool causal, bool scoremod, hipStream_t st);

// Portable kernels: any dtype, D in {16, 32, 64, 128}, any alignment.
void launch_fwd_generic(const KParams &p, int dtype, int D, bool causal, hipStream_t st);
void launch_bwd_dq_generic(const KParams &p, int dtype, int D, bool causal, hipStream_t st);
void launch_bwd_dkdv_generic(const KParams &p, int dtype, int D, bool causal, hipStream_t st);

}  // namespace sigattn
