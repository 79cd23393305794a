// Internal interface between the C-ABI (sqa_capi.hip) and the gfx950 kernels
// (sqa_kernels.hip). Not installed; the public boundary is include/sqa.h.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

namespace sqa {

constexpr int kHeadDim = 128;   // the reference's head_dim; 64 and 256 are also built
constexpr int kMaxRowsHd256 = 32;  // head_dim 256: accumulators of at most two 16-row blocks
constexpr int kPageSize = 16;   // kernel page: 16 tokens (one MFMA tile of keys)
constexpr int kMaxPageShift = 4;  // cache pages of 16 << shift tokens: 16 .. 256
constexpr int kMaxRows = 64;    // q_len * (Hq / Hkv) rows one work item holds
constexpr int kMaxSplitPages = 2048;  // pages one split may own (LDS page-id table)
constexpr int kMinSplitPages = 4;     // fewest pages the automatic plans give a split
constexpr int kMaxBalancedBatch = 256;  // balanced plan: four sequences per lane of one wave
// Partial sums are stored through a buffer resource with 32-bit offsets; a plan
// whose partials need more is refused.
constexpr unsigned long long kMaxPartialBytes = 0xFFFF0000ull;

// Per-sequence split layout of the balanced plan, written by the partial
// kernel for the merge kernel: first slot and number of splits.
struct SeqSplits {
  int first;
  int count;
};

// Everything the split-KV partial kernel needs. Element counts, not bytes.
//
// Two split plans. Fixed (pages_per_split > 0): sequence b owns slots
// b * num_splits + s, split s covering pages [s * pages_per_split, ...).
// Balanced (pages_per_split <= 0, batch <= kMaxBalancedBatch): num_splits =
// T + batch slots for T work items. Every workgroup derives, from all seq_lens,
// the batch's pages laid end to end and one item size P = ceil(total / T)
// (packed_item_pages); item i takes global pages [i P, (i + 1) P), crossing
// sequence ends where they fall, so all items carry the same number of pages
// whatever the length distribution. The part of item i in sequence b (a piece)
// leaves its partial in slot i + b; a sequence inside one piece is written
// straight to the output. The kernel records each sequence's (first slot,
// count) for the merge.
//
// Seams: a workgroup whose item spans the start of a sequence runs a second
// piece, which costs it about seam_pages pages' time (the first piece's
// results written, the second's Q, page ids and first pages fetched). When the
// lengths differ (a ragged batch), every sequence start that does not fall on an
// item boundary of that layout is preceded by seam_pages pages of nothing, and
// the items are cut from the pages laid end to end with those gaps: an item that
// spans such a start then carries seam_pages fewer pages. Batches whose lengths
// are all equal (and so every plan with spec_pages) get no gaps.
//
// spec_pages > 0 (balanced plan only): the page count the caller expects every
// sequence to have (from max_seq_len), with that case's item size computed by
// the host (spec_pps = packed_item_pages(batch * spec_pages, T)). Workgroups
// then know their first piece without the lengths and issue its page-id loads
// together with them; a length that does not match sends the workgroup back to
// the plan from the loaded lengths. Either way the plan is the one the lengths
// give: the expectation only saves a memory round trip and the plan's wave
// reductions when it holds.
//
// The C ABI carries spec_pages in pages_per_split: 0 is the balanced plan,
// -P the balanced plan expecting P pages per sequence.
//
// Paired items (pair_items != 0; the 64-row kernel with two head groups, every
// length as expected and two items of P pages dividing a sequence): items
// 2k and 2k + 1 share 2P pages, the even one taking P + d and the odd one
// P - d, d = round(P * delta), and both workgroups of item i (one per head
// group) run on XCDs of i's parity (blockIdx.x = 4k + 2 head_group + (i & 1);
// workgroups are dealt to the XCDs in turn). The 64-row kernel streams its
// pages more slowly on the odd XCDs: per-workgroup stamps at 16 sequences of
// 32K keys put the odd XCDs' workgroups 6-8% behind the even ones' on every box
// measured (the head group adds 1-2%), so by default (kPairsFixed) the even
// items take kPairDeltaFixed more pages: the split depends on the plan alone
// and equal inputs give equal bits. On request (kPairsAdaptive,
// SQA_FLAG_ADAPTIVE_PAIRS) delta is measured instead: each workgroup records
// its page-loop time and pages, and the merge kernel sets delta for the next
// call from the per-page times of even and odd items. Every workgroup of a call
// reads the same value, and any delta covers every key once, so results stay
// within the parity tolerance; but the split point changes how the
// fp16-normalised partials round, so with adaptive pairs the output bits follow
// the previous call's times.
// Workgroup 0 of an adaptive paired call stamps tune[2] (kTuneStamp), every
// workgroup of it writes its record, and the merge kernel reads the records only
// under that stamp, then clears it: records of an earlier call or another
// shape's data in a reused workspace never feed the delta.
constexpr int kPairsOff = 0, kPairsAdaptive = 1, kPairsFixed = 2;  // PartialArgs::pair_items
constexpr float kPairDeltaFixed = 0.03f;  // even items' extra share with fixed pairs
constexpr unsigned kTuneMagic = 0x51a7u << 16 | 1u;  // tune[0] when tune[1] holds a delta
constexpr unsigned kTuneStamp = 0x51a7u << 16 | 2u;  // tune[2] after a call that ran paired
constexpr float kPairDeltaMax = 0.1f;                // |delta| bound

// Items per head group (hg_items[0] > 0; the balanced plan with an expected
// page count, 8 kv heads in two head groups of four, one wave per head): the
// two head groups cut the same pages into different numbers of items, N0 and
// N1 with N0 + N1 = 2 (num_splits - batch), so the head group that streams its
// half of the token rows more slowly gets the shorter items. Each head group
// then has its own slots, table and item size: group g's slots are g's region
// of the partials, Sg = Ng + batch slots of 4 kv heads each (region 1 after
// region 0's S0: the regions fill the same num_splits x 8 heads), its (first
// slot, count) table is at seq_splits + g * batch, its item size spec_pps
// (group 0) or hg_spec_pps1. Workgroups 2i and 2i + 1 are item i of groups 0
// and 1 up to the smaller count, the rest the larger group's remaining items.
struct HeadGroupItems {
  int group, item;   // this workgroup's head group and item
  int slots;         // Sg
  int slot_base;     // slots of the regions before this group's (0 or S0)
  int spec_pps;      // this group's item size
};
__host__ __device__ inline HeadGroupItems head_group_items(const int (&n)[2], int batch,
                                                           int spec_pps0, int spec_pps1,
                                                           int block) {
  const int nf = n[0] < n[1] ? n[0] : n[1];
  HeadGroupItems h;
  if (block < 2 * nf) {
    h.group = block & 1;
    h.item = block >> 1;
  } else {
    h.group = n[0] > n[1] ? 0 : 1;
    h.item = nf + (block - 2 * nf);
  }
  h.slots = n[h.group] + batch;
  h.slot_base = h.group ? n[0] + batch : 0;
  h.spec_pps = h.group ? spec_pps1 : spec_pps0;
  return h;
}
struct PartialArgs {
  const _Float16* q;          // [B, Q, Hq, head_dim]
  const _Float16* k;          // K of page 0, slot 0, kv head 0
  const _Float16* v;          // V of page 0, slot 0, kv head 0
  const int32_t* block_tables;  // [B, bt_stride] cache-page ids
  const int32_t* seq_lens;      // [B]
  const uint32_t* draft_mask;   // NULL (causal draft chain) or [B, Q, mask_words]
  _Float16* out;              // [B, Q, Hq, head_dim]; written directly when num_splits == 1
  float* part_o;              // [slots, Hkv, rows, head_dim]: fp32 unnormalised sums, or for
                              // fp16 outputs fp16 rows divided by their sum (the first half
                              // of the same region)
  float* part_ml;             // [slots, Hkv, rows, 2] (max in log2 units, sum)
  unsigned part_o_bytes;      // bytes of part_o the partials use (< kMaxPartialBytes)
  SeqSplits* seq_splits;      // [B] (balanced plan only)
  long long num_pages;        // pages in the cache pool; ids outside are clamped to 0
  long long page_stride;      // bytes between consecutive cache pages (K and V alike)
  unsigned token_stride;      // bytes between consecutive slots of a page
  unsigned head_stride;       // bytes between consecutive kv heads
  unsigned page_extent;       // bytes from a kernel page's base that its K (or V) spans
  int mask_words;             // 32-bit words per draft-mask row (1 or 2)
  int batch, q_len, hq, hkv, group, rows;
  int head_dim;               // 64, 128 or 256
  int bt_stride;              // block_tables row length (cache pages)
  int page_shift;             // cache page = 16 << page_shift tokens = 1 << page_shift kernel pages
  int max_pages;              // kernel pages a block-table row addresses (bt_stride << page_shift)
  int pages_per_split, num_splits;
  int spec_pages;             // balanced plan: expected pages of every sequence (0: none)
  int spec_pps;               // the balanced plan's item size when every sequence spans spec_pages
  int seam_pages;             // balanced plan: pages a second piece costs a workgroup (0: no gaps)
  int pair_items;             // kPairsOff, kPairsAdaptive or kPairsFixed (see above)
  int ring_batch;             // every piece expected within the register ring (kRingPages)
  int hg_items[2];            // items per head group (HeadGroupItems below); 0: both
                              // num_splits - batch, the usual layout
  int hg_spec_pps1;           // with hg_items: head group 1's item size (spec_pps: group 0's)
  float* tune;                // adaptive paired items: {magic, delta, stamp, -} then per
                              // workgroup {loop ticks, pages}
  float scale_log2;           // softmax scale * log2(e)
  float out_scale;            // multiplier applied to the normalised output
  int bf16;                   // element type of Q and out (and of K, V unless kv_fp8): 0 fp16, 1 bf16
  int kv_fp8;                 // K and V hold OCP e4m3 bytes
};

// pages_per_split as the C ABI carries it: > 0 fixed plan, 0 balanced, -P balanced
// expecting P pages per sequence.
__host__ __device__ inline bool is_balanced(int pages_per_split) { return pages_per_split <= 0; }
__host__ __device__ inline int spec_pages_of(int pages_per_split) {
  return pages_per_split < 0 ? -pages_per_split : 0;
}

// Partial slots a plan uses.
inline long long plan_slots(int batch, int num_splits, int pages_per_split) {
  return is_balanced(pages_per_split) ? (long long)num_splits : (long long)batch * num_splits;
}

struct MergeArgs {
  const float* part_o;
  const float* part_ml;
  const SeqSplits* seq_splits;  // balanced plan only
  const int32_t* seq_lens;
  _Float16* out;
  int batch, q_len, hq, hkv, group, rows;
  int head_dim;
  int max_pages;  // kernel pages a block-table row addresses
  int pages_per_split, num_splits;
  int spec_pages;   // balanced plan: expected pages of every sequence (0: none)
  int spec_pps;     // the balanced plan's item size when that holds
  int hg_items[2];  // as PartialArgs::hg_items
  int hg_spec_pps1; // as PartialArgs::hg_spec_pps1
  float out_scale;
  int bf16;
  float* tune;      // adaptive paired items: the delta record to update (null: none)
  int tune_records; // workgroup records after it
};

// The balanced plan's item size: pages per work item when `total` pages are
// shared by `target` (= num_splits - batch) items, clamped to [kMinSplitPages,
// kMaxSplitPages]. ceil(total / P) <= target when target >= ceil(total /
// kMaxSplitPages), which the C ABI checks.
__host__ __device__ inline int packed_item_pages(int total, int target) {
  const int p = (total + target - 1) / target;
  return p < kMinSplitPages ? kMinSplitPages : (p > kMaxSplitPages ? kMaxSplitPages : p);
}

// Launch shape of the partial kernel for a given number of query rows per kv
// head. A workgroup serves `heads` kv heads of one (sequence, split), `hpw`
// heads per wave holding all of their rows; all waves walk the same pages, so the
// heads' slices of a page are read together (>= 4 heads keeps HBM accesses at
// >= 1 KiB contiguous). `wg_per_cu` workgroups are resident per CU, which sets
// the split count of the automatic plans.
//
// One workgroup per CU (one wave per SIMD): when two workgroups share a CU the
// older one takes nearly all of the CU's memory issue and the other starts in
// earnest only when it finishes, so equal work items end in two waves and the
// second wave's spread of end times idles the chip. Alone on its CU a
// workgroup keeps a deeper ring (D pages per wave) in the registers the second
// one would have used.
struct LaunchShape {
  int row_blocks;  // 16-row blocks per wave (1, 2 or 4)
  int heads;       // kv heads per workgroup
  int hpw;         // kv heads per wave (2: both halves of a 16-row block)
  int wg_per_cu;   // resident workgroups per CU
  int waves() const { return heads / hpw; }
};

// At head dim 64 a wave holds two kv heads with up to 32 rows each: with up
// to 8 rows per kv head (q_len 2 at GQA 4) both share one block (no padding
// rows), with up to 16 or 32 each has its own one or two (row_blocks 2 or 4;
// q_len 8: 177.7 -> 174.9 us, e4m3 112.1 -> 99.5 us). The
// per-page work (page id, buffer resources, loop) is then spread over twice
// the bytes (a head's page is 4 KiB there); cfg3 lengths, q_len 2: 168.5 ->
// 160.6 us, q_len 4: 169.7 -> 165.6 us (e4m3 100.0 -> 95.3). At head dim 128
// the shared-block shape ran 1-12% slower (half the pages per work item,
// twice the partials) and keeps one head per wave. Needs Hkv % 8 == 0.
inline LaunchShape launch_shape(int rows, int hkv, int head_dim) {
  if (rows <= 8 && hkv % 8 == 0 && head_dim == 64) return {1, 8, 2, 1};
  if (rows <= 16 && hkv % 8 == 0 && head_dim == 64) return {2, 8, 2, 1};
  if (rows <= 32 && hkv % 8 == 0 && head_dim == 64) return {4, 8, 2, 1};
  if (rows <= 16) return {1, 4, 1, 1};
  if (rows <= 32) return {2, 4, 1, 1};
  return {4, 4, 1, 1};
}

// Pages the register ring of the one-wave-per-head kernel holds at head dim 128
// with 16-bit K/V and up to 32 rows: pieces of at most this many pages take the
// whole-ring softmax step (PartialArgs::ring_batch).
constexpr int kRingPages = 4;

// What a second piece costs a workgroup of the balanced plan, in pages of its
// own: ~5.6 us measured at 16 ragged sequences of 2K-32K tokens (q_len 8, head
// dim 128, fp16), where one page of the workgroup's (16 tokens of K and V for 4
// kv heads, 32 KiB) takes ~1.15 us; scaled by the bytes of a workgroup's page
// for other shapes and element types. The 8-wave LDS kernel (33..64 rows, head
// dim 128, 16-bit K/V) restarts a ring behind a barrier per page and writes
// 64 rows per head: 8 pages measured best there (ragged q16 fp16 190.2 -> 187.8
// us, bf16 194.4 -> 190.2; 12 pages 187.8 / 190.8; with one barrier per page
// partial 183.0 / 180.7 / 181.3 us at 5 / 8 / 11 pages).
inline int seam_pages(int rows, int hkv, int head_dim, int kv_bytes) {
  const LaunchShape sh = launch_shape(rows, hkv, head_dim);
  const int wg_page = 16 * sh.heads * head_dim * 2 * kv_bytes;
  const int cost = head_dim == 128 && kv_bytes == 2 && rows > 32 ? 8 : 5;
  const int c = (cost * 32768 + wg_page / 2) / wg_page;
  return c < 1 ? 1 : (c > 32 ? 32 : c);
}

hipError_t launch_partial(const PartialArgs& a, hipStream_t stream);
hipError_t launch_merge(const MergeArgs& a, hipStream_t stream);

}  // namespace sqa
