// Internal interface between the C-ABI (sqa_capi.hip) and the gfx950 kernels
// (sqa_kernels.hip). Not installed; the public boundary is include/sqa.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace sqa {

constexpr int kHeadDim = 128;   // contract: head_dim 128
constexpr int kPageSize = 16;   // contract: 16-token pages
constexpr int kMaxRows = 64;    // q_len * (Hq / Hkv) rows one work item holds
constexpr int kMaxSplitPages = 2048;  // pages one split may own (LDS page-id table)

// Everything the split-KV partial kernel needs. Element counts, not bytes.
struct PartialArgs {
  const _Float16* q;          // [B, Q, Hq, 128]
  const _Float16* k;          // [num_pages, 16, Hkv, 128]
  const _Float16* v;          // [num_pages, 16, Hkv, 128]
  const int32_t* block_tables;  // [B, max_pages]
  const int32_t* seq_lens;      // [B]
  _Float16* out;              // [B, Q, Hq, 128]; written directly when num_splits == 1
  float* part_o;              // [B, Hkv, num_splits, rows, 128] unnormalised sums
  float* part_ml;             // [B, Hkv, num_splits, rows, 2] (max in log2 units, sum)
  long long num_pages;        // pages in the cache pool; ids outside are clamped to 0
  int batch, q_len, hq, hkv, group, rows;
  int max_pages;              // block_tables row length
  int pages_per_split, num_splits;
  float scale_log2;           // head_dim^-1/2 * log2(e)
};

struct MergeArgs {
  const float* part_o;
  const float* part_ml;
  const int32_t* seq_lens;
  _Float16* out;
  int batch, q_len, hq, hkv, group, rows;
  int max_pages, pages_per_split, num_splits;
};

// Launch shape of the partial kernel for a given number of query rows per kv
// head. A workgroup serves `heads` kv heads of one (sequence, split), one wave
// per head holding all of its rows; all waves walk the same pages, so the
// heads' slices of a page are read together (>= 4 heads keeps HBM accesses at
// >= 1 KiB contiguous). `wg_per_cu` workgroups are resident per CU (register
// file), which sets the split count of the automatic plan.
struct LaunchShape {
  int row_blocks;  // 16-row blocks per wave (1, 2 or 4)
  int heads;       // kv heads per workgroup (one wave each)
  int wg_per_cu;   // resident workgroups per CU
};

inline LaunchShape launch_shape(int rows) {
  // Two 4-wave workgroups per CU (2 waves per SIMD) measured best up to 32
  // rows: a third (possible at <= 16 rows, 165 VGPRs) adds page streams per
  // CU and lowers bandwidth. 64 rows take the whole 512-entry register file
  // (1 wave per SIMD), which beat splitting a head's rows over two waves that
  // each read its pages.
  if (rows <= 16) return {1, 4, 2};
  if (rows <= 32) return {2, 4, 2};
  return {4, 4, 1};
}

hipError_t launch_partial(const PartialArgs& a, hipStream_t stream);
hipError_t launch_merge(const MergeArgs& a, hipStream_t stream);

}  // namespace sqa
