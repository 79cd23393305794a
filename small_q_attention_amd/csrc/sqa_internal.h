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

// Waves per workgroup of the partial kernel. The waves of one workgroup serve
// different kv heads (and, for 64 rows, the two 32-row halves of a head) of
// the same (sequence, split), walking the same pages together.
constexpr int kWgWaves = 8;

// Number of 16-row blocks (1, 2 or 4) for `rows` query rows.
inline int row_blocks(int rows) { return rows <= 16 ? 1 : (rows <= 32 ? 2 : 4); }
// Waves per kv head: one up to 32 rows, two (32 rows each) up to 64.
inline int row_groups(int rows) { return rows <= 32 ? 1 : 2; }

hipError_t launch_partial(const PartialArgs& a, hipStream_t stream);
hipError_t launch_merge(const MergeArgs& a, hipStream_t stream);

}  // namespace sqa
