// C ABI of libsqa.so (declared in include/sqa.h). Validates arguments, plans
// the split-KV decomposition and launches the gfx950 kernels of
// sqa_kernels.hip on the caller's stream. Allocates nothing.
#include "sqa.h"
#include "sqa_internal.h"

#include <math.h>
#include <stdarg.h>
#include <stddef.h>
#include <stdio.h>
#include <string.h>

#include <mutex>
#include <string>
#include <vector>

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  try {  // a message that cannot be stored is lost; the status still returns
    g_last_error = buf;
  } catch (...) {
  }
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(SQA_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

std::mutex g_cu_mutex;
std::vector<int> g_cu_count;  // cached per device

long long ceil_div(long long a, long long b) { return (a + b - 1) / b; }

}  // namespace

extern "C" {

const char* sqa_last_error(void) { return g_last_error.c_str(); }

// The build passes the source hash (small_q_attention_amd/build.py); the loader
// compares it with the sources beside the library.
#ifndef SQA_SOURCE_HASH
#define SQA_SOURCE_HASH "unstamped"
#endif
const char* sqa_version(void) { return "sqa 0.2.0 gfx950 sqa-src-hash:" SQA_SOURCE_HASH; }

int sqa_device_cu_count(int device) {
  if (device < 0) return -1;
  try {  // the lock and the cache's growth may throw; nothing crosses the C boundary
    std::lock_guard<std::mutex> lock(g_cu_mutex);
    if ((int)g_cu_count.size() <= device) g_cu_count.resize(device + 1, 0);
    if (g_cu_count[device] == 0) {
      int n = 0;
      hipError_t e = hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device);
      if (e != hipSuccess || n <= 0) {
        hip_fail(e, "hipDeviceGetAttribute(MultiprocessorCount)");
        return -1;
      }
      g_cu_count[device] = n;
    }
    return g_cu_count[device];
  } catch (...) {
    fail(SQA_ERR_HIP, "sqa_device_cu_count: out of host memory or lock failure");
    return -1;
  }
}

int sqa_plan_splits(int device, int batch, int q_len, int num_query_heads, int num_kv_heads,
                    int head_dim, int max_seq_len, int max_pages, int chunk_keys,
                    int* num_splits, int* pages_per_split) {
  if (!num_splits || !pages_per_split) return fail(SQA_ERR_INVALID, "null output pointer");
  if (batch <= 0 || q_len <= 0 || num_kv_heads <= 0 || num_query_heads <= 0 || max_pages <= 0)
    return fail(SQA_ERR_INVALID, "batch, q_len, heads and max_pages must be positive");
  if (chunk_keys < 0) return fail(SQA_ERR_INVALID, "chunk_keys must be >= 0");
  long long pages = max_pages;
  if (max_seq_len > 0) {
    const long long need = ceil_div(max_seq_len, sqa::kPageSize);
    pages = need < pages ? need : pages;
  }
  long long pps;
  if (chunk_keys > 0) {
    pps = ceil_div(chunk_keys, sqa::kPageSize);
  } else {
    int cus = sqa_device_cu_count(device);
    if (cus <= 0) return SQA_ERR_HIP;
    // One wave of resident workgroups over the whole chip.
    const sqa::LaunchShape sh =
        sqa::launch_shape(q_len * (num_query_heads / num_kv_heads), num_kv_heads, head_dim);
    const long long head_groups = (num_kv_heads + sh.heads - 1) / sh.heads;
    const long long slots_target = ceil_div((long long)cus * sh.wg_per_cu, head_groups);
    if (batch > 1 && batch <= sqa::kMaxBalancedBatch) {
      // Balanced plan: the kernel sizes splits from the batch's total pages,
      // so ragged batches keep every workgroup equally busy. The slot count
      // leaves one spare slot per sequence (rounding up each sequence's last
      // split) and keeps a split within kMaxSplitPages pages.
      long long target = slots_target;
      const long long cap = ceil_div((long long)batch * max_pages, sqa::kMaxSplitPages);
      if (target < cap) target = cap;
      if ((target + batch) * num_kv_heads > 0x7fffffffLL)
        return fail(SQA_ERR_INVALID, "grid too large");
      *num_splits = (int)(target + batch);
      // With a known max_seq_len the kernels first assume every sequence spans
      // that many pages (and check it): -pages.
      *pages_per_split = max_seq_len > 0 ? -(int)pages : 0;
      return SQA_OK;
    }
    const long long splits = ceil_div(slots_target, batch);
    pps = ceil_div(pages, splits);
    // Each split leaves a partial row per query row for the merge. Past 32
    // rows (the 64-row kernel), sequences of more than 64 four-page splits
    // start at 8 pages: there the merge of the extra splits costs more than the
    // shorter splits save (one sequence, KV 8K, q16, per call: 23.9 us at 64 x
    // 8 pages, 26.7 at 128 x 4), while shorter ones gain from 4. Up to 32 rows
    // 4-page pieces take the register ring in one softmax step, and 4 pages win
    // (KV 8K, q8: 18.0 us at 128 x 4, 19.0 at 64 x 8).
    const bool past32 = (long long)q_len * (num_query_heads / num_kv_heads) > 32;
    const long long min_pps = past32 && pages > 64 * sqa::kMinSplitPages
                                  ? 2 * sqa::kMinSplitPages
                                  : sqa::kMinSplitPages;
    if (pps < min_pps) pps = min_pps;
  }
  if (pps > pages) pps = pages;
  if (pps > sqa::kMaxSplitPages) pps = sqa::kMaxSplitPages;
  if (pps < 1) pps = 1;
  long long splits = ceil_div(pages, pps);
  if (splits < 1) splits = 1;
  if ((long long)batch * num_kv_heads * splits > 0x7fffffffLL)
    return fail(SQA_ERR_INVALID, "grid too large");
  *num_splits = (int)splits;
  *pages_per_split = (int)pps;
  return SQA_OK;
}

size_t sqa_workspace_bytes(int batch, int q_len, int num_query_heads, int num_kv_heads,
                           int head_dim, int num_splits, int pages_per_split) {
  if (batch <= 0 || q_len <= 0 || num_kv_heads <= 0 || num_query_heads <= 0 || head_dim <= 0 ||
      num_splits <= 0)
    return 0;
  const bool balanced = sqa::is_balanced(pages_per_split);
  if (!balanced && num_splits == 1) return 0;
  const size_t rows = (size_t)q_len * (num_query_heads / num_kv_heads);
  const size_t items = (size_t)sqa::plan_slots(batch, num_splits, pages_per_split) * num_kv_heads * rows;
  size_t bytes = items * ((size_t)head_dim + 2) * sizeof(float);
  // Balanced plans: the merge table, then the adaptive paired items' delta
  // record (16 bytes) and one 8-byte loop-time record per workgroup (two per
  // slot). With items per head group the second group's table takes the first
  // batch x 8 bytes of that record region (num_splits > batch keeps it inside):
  // those calls (e4m3, at most 32 rows) never pair, and a later paired call
  // reads no magic or stamp there.
  if (balanced)
    bytes += (size_t)batch * sizeof(sqa::SeqSplits) + 16 + (size_t)num_splits * 2 * 8;
  return bytes;
}

}  // extern "C"

namespace {

// Validates a call and launches the kernels. Shared by both entry points.
int run_attention(const sqa_attention_args& a) {
  const int batch = a.batch, q_len = a.q_len, num_query_heads = a.num_query_heads;
  const int num_kv_heads = a.num_kv_heads, head_dim = a.head_dim, page_size = a.page_size;
  const int max_pages = a.max_pages, num_splits = a.num_splits;
  const int pages_per_split = a.pages_per_split;
  const int64_t num_pages = a.kv.num_pages;
  if (!a.query || !a.kv.k || !a.kv.v || !a.block_tables || !a.seq_lens || !a.output)
    return fail(SQA_ERR_INVALID, "null tensor pointer");
  if (batch <= 0 || q_len <= 0 || num_query_heads <= 0 || num_kv_heads <= 0)
    return fail(SQA_ERR_INVALID, "batch, q_len and head counts must be positive");
  if (num_pages <= 0 || max_pages <= 0)
    return fail(SQA_ERR_INVALID, "empty KV cache is not supported");
  if (num_query_heads % num_kv_heads != 0)
    return fail(SQA_ERR_INVALID, "num_query_heads must be divisible by num_kv_heads");
  if (head_dim != 64 && head_dim != 128 && head_dim != 256)
    return fail(SQA_ERR_UNSUPPORTED, "head_dim must be 64, 128 or 256 (got %d)", head_dim);
  int page_shift = -1;
  for (int sh = 0; sh <= sqa::kMaxPageShift; ++sh)
    if (page_size == (sqa::kPageSize << sh)) page_shift = sh;
  if (page_shift < 0)
    return fail(SQA_ERR_UNSUPPORTED, "page_size must be 16, 32, 64, 128 or 256 (got %d)",
                page_size);
  // The kernels work in 16-token pages; a cache page is 1 << page_shift of them.
  const long long kernel_pages = (long long)max_pages << page_shift;
  if (kernel_pages > 0x7fffffffLL) return fail(SQA_ERR_INVALID, "block table too wide");
  const int group = num_query_heads / num_kv_heads;
  const long long rows = (long long)q_len * group;
  const int max_rows = head_dim == 256 ? sqa::kMaxRowsHd256 : sqa::kMaxRows;
  if (rows > max_rows)
    return fail(SQA_ERR_UNSUPPORTED, "q_len * group = %lld exceeds %d at head_dim %d", rows,
                max_rows, head_dim);
  if (a.dtype != SQA_DTYPE_F16 && a.dtype != SQA_DTYPE_BF16)
    return fail(SQA_ERR_UNSUPPORTED, "dtype must be SQA_DTYPE_F16 or SQA_DTYPE_BF16 (got %d)",
                a.dtype);
  if (a.kv_dtype != a.dtype && a.kv_dtype != SQA_DTYPE_FP8_E4M3)
    return fail(SQA_ERR_UNSUPPORTED, "kv_dtype must equal dtype or be SQA_DTYPE_FP8_E4M3 (got %d)",
                a.kv_dtype);
  const bool kv_fp8 = a.kv_dtype == SQA_DTYPE_FP8_E4M3;
  const long long kv_bytes = kv_fp8 ? 1 : 2;
  // Cache layout: 16-byte aligned bases, strides of whole 8-element groups (the
  // kernel's 16- or 8-byte loads), and one kernel page's K (or V) within 2 GiB
  // of its base (32-bit buffer offsets).
  const int64_t ps = a.kv.page_stride, ts = a.kv.token_stride, hs = a.kv.head_stride;
  if (ps < 0 || ts < 0 || hs < 0 || ps % 8 || ts % 8 || hs % 8)
    return fail(SQA_ERR_INVALID, "cache strides must be non-negative multiples of 8 elements");
  if (((uintptr_t)a.kv.k | (uintptr_t)a.kv.v) % 16)
    return fail(SQA_ERR_INVALID, "cache base pointers must be 16-byte aligned");
  // Q rows are read 16 bytes at a time, outputs written 8 bytes at a time.
  if ((uintptr_t)a.query % 16 || (uintptr_t)a.output % 8)
    return fail(SQA_ERR_INVALID, "query must be 16-byte and output 8-byte aligned");
  if (((uintptr_t)a.block_tables | (uintptr_t)a.seq_lens | (uintptr_t)a.draft_mask) % 4)
    return fail(SQA_ERR_INVALID, "block_tables, seq_lens and draft_mask must be 4-byte aligned");
  const long long extent =
      kv_bytes * ((long long)(sqa::kPageSize - 1) * ts + (long long)(num_kv_heads - 1) * hs +
                  head_dim);
  if (extent > 0x7fffffffLL)
    return fail(SQA_ERR_INVALID, "one page of the cache spans more than 2 GiB");
  if (a.draft_mask && (a.mask_words < (q_len + 31) / 32 || a.mask_words > 2))
    return fail(SQA_ERR_INVALID, "draft_mask needs %d..2 words per row, got %d", (q_len + 31) / 32,
                a.mask_words);
  if (!(a.scale > 0.f) || !isfinite(a.scale) || !isfinite(a.out_scale))
    return fail(SQA_ERR_INVALID, "scale must be positive and finite, out_scale finite");
  if (a.flags & ~SQA_FLAG_ADAPTIVE_PAIRS)
    return fail(SQA_ERR_INVALID, "unknown flags %#x", (unsigned)a.flags);
  if (num_splits <= 0) return fail(SQA_ERR_INVALID, "num_splits must be positive");
  if (pages_per_split > sqa::kMaxSplitPages)
    return fail(SQA_ERR_INVALID, "pages_per_split %d exceeds %d", pages_per_split,
                sqa::kMaxSplitPages);
  const bool balanced = sqa::is_balanced(pages_per_split);
  const int spec_pages = sqa::spec_pages_of(pages_per_split);
  if (balanced) {
    // pages_per_split <= 0 selects the balanced plan (sqa_plan_splits); -P expects
    // P pages in every sequence.
    if (spec_pages > kernel_pages)
      return fail(SQA_ERR_INVALID,
                  "balanced plan expects %d pages per sequence; block_tables rows hold %lld",
                  spec_pages, kernel_pages);
    if (batch > sqa::kMaxBalancedBatch)
      return fail(SQA_ERR_INVALID, "balanced plan (pages_per_split 0) needs batch <= %d, got %d",
                  sqa::kMaxBalancedBatch, batch);
    if (kernel_pages >= (1LL << 24))
      return fail(SQA_ERR_INVALID, "balanced plan needs block-table rows under 2^28 tokens");
    if ((long long)batch * kernel_pages >= (1LL << 30))
      return fail(SQA_ERR_INVALID, "balanced plan needs batch * pages per row under 2^30");
    const long long cap = ceil_div((long long)batch * kernel_pages, sqa::kMaxSplitPages);
    if ((long long)num_splits - batch < (cap > 1 ? cap : 1))
      return fail(SQA_ERR_INVALID,
                  "balanced plan needs num_splits >= batch + %lld (batch %d), got %d",
                  cap > 1 ? cap : 1, batch, num_splits);
  }
  // A fixed plan covering fewer than max_pages pages (built from a known
  // max_seq_len) processes only the first num_splits * pages_per_split pages of
  // each sequence, as the reference launchers do with their max_seq_len. The
  // balanced plan processes every page up to seq_lens (clamped to max_pages).
  if (sqa::plan_slots(batch, num_splits, pages_per_split) * num_kv_heads > 0x7fffffffLL)
    return fail(SQA_ERR_INVALID, "grid too large");
  const size_t need = sqa_workspace_bytes(batch, q_len, num_query_heads, num_kv_heads, head_dim,
                                          num_splits, pages_per_split);
  if (need > 0 && (!a.workspace || a.workspace_bytes < need))
    return fail(SQA_ERR_WORKSPACE, "workspace of %zu bytes needed, %zu given", need,
                a.workspace ? a.workspace_bytes : (size_t)0);
  if (need > 0 && (uintptr_t)a.workspace % 16)
    return fail(SQA_ERR_WORKSPACE, "workspace must be 16-byte aligned");

  // fp16 outputs keep fp16 partial rows (half of the region), bf16 fp32 ones.
  const unsigned long long part_o_bytes =
      (unsigned long long)sqa::plan_slots(batch, num_splits, pages_per_split) * num_kv_heads *
      rows * head_dim * (a.dtype == SQA_DTYPE_F16 ? 2 : 4);
  if ((balanced || num_splits > 1) && part_o_bytes > sqa::kMaxPartialBytes)
    return fail(SQA_ERR_INVALID, "the plan's partials (%llu bytes) exceed %llu bytes",
                part_o_bytes, sqa::kMaxPartialBytes);
  hipStream_t s = (hipStream_t)a.stream;
  hipEvent_t* ev = (hipEvent_t*)a.timing_events;
  void* workspace = a.workspace;

  sqa::PartialArgs pa;
  pa.q = (const _Float16*)a.query;
  pa.k = (const _Float16*)a.kv.k;
  pa.v = (const _Float16*)a.kv.v;
  pa.block_tables = a.block_tables;
  pa.seq_lens = a.seq_lens;
  pa.draft_mask = a.draft_mask;
  pa.mask_words = a.draft_mask ? a.mask_words : 0;
  pa.out = (_Float16*)a.output;
  const size_t items =
      (size_t)sqa::plan_slots(batch, num_splits, pages_per_split) * num_kv_heads * rows;
  const bool merged = balanced || num_splits > 1;
  pa.part_o = merged ? (float*)workspace : nullptr;
  pa.part_ml = merged ? (float*)workspace + items * head_dim : nullptr;
  pa.seq_splits = balanced ? (sqa::SeqSplits*)(pa.part_ml + items * 2) : nullptr;
  pa.part_o_bytes = merged ? (unsigned)part_o_bytes : 0u;
  pa.num_pages = num_pages;
  pa.page_stride = kv_bytes * ps;
  pa.token_stride = (unsigned)(kv_bytes * ts);
  pa.head_stride = (unsigned)(kv_bytes * hs);
  pa.page_extent = (unsigned)extent;
  pa.batch = batch;
  pa.q_len = q_len;
  pa.hq = num_query_heads;
  pa.hkv = num_kv_heads;
  pa.group = group;
  pa.rows = (int)rows;
  pa.head_dim = head_dim;
  pa.bt_stride = max_pages;
  pa.page_shift = page_shift;
  pa.max_pages = (int)kernel_pages;
  pa.pages_per_split = balanced ? 0 : pages_per_split;
  pa.num_splits = num_splits;
  pa.spec_pages = spec_pages;
  pa.spec_pps =
      spec_pages > 0 ? sqa::packed_item_pages(batch * spec_pages, num_splits - batch) : 0;
  pa.seam_pages = balanced ? sqa::seam_pages((int)rows, num_kv_heads, head_dim, (int)kv_bytes) : 0;
  // Paired items: the 64-row kernel (33..64 rows, head dim 128) with 16-bit K
  // and V, two head groups of four kv heads, an expected page count that pairs
  // of items divide, and an even item count. By default with the fixed delta
  // (the bits depend on the inputs alone); with SQA_FLAG_ADAPTIVE_PAIRS with the
  // measured one (the bits follow the previous call's times).
  pa.tune = balanced ? (float*)(pa.seq_splits + batch) : nullptr;
  const bool pair_ok = balanced && spec_pages > 0 && pa.spec_pps > 0 &&
                       spec_pages % (2 * pa.spec_pps) == 0 && (num_splits - batch) % 2 == 0 &&
                       head_dim == 128 && kv_bytes == 2 && rows > 32 && rows <= 64 &&
                       num_kv_heads == 8;
  pa.pair_items = !pair_ok                              ? sqa::kPairsOff
                  : (a.flags & SQA_FLAG_ADAPTIVE_PAIRS) ? sqa::kPairsAdaptive
                                                        : sqa::kPairsFixed;
  // Items per head group (sqa_internal.h): e4m3 caches with token rows of 1 KiB
  // (8 kv heads of 128 dims), read as two 512-byte halves by the two head groups
  // of the one-wave kernel (up to 32 rows), under fp16 queries. The half whose
  // address bit 9 is 0 streams more slowly: per-workgroup stamps at 16 x 32K
  // keys, pools at 2 MiB boundaries, 165 against 146 us per workgroup; K's bit
  // sets which half (V's adds or takes away about a third), so the K pool's bit
  // 9 picks the slower group and whether V's agrees sets its extra items (6.5%
  // of the items, best of 4 / 6.5 / 9%, or 2%). Under bf16 queries (more math
  // per page) the same split ran 2.6% slower at q_len 8, so they keep one count.
  pa.hg_items[0] = pa.hg_items[1] = 0;
  pa.hg_spec_pps1 = 0;
  const long long kv_page_bytes = kv_bytes * ps;
  if (balanced && spec_pages > 0 && kv_fp8 && a.dtype == SQA_DTYPE_F16 && head_dim == 128 &&
      num_kv_heads == 8 && rows <= 32 && kv_bytes * hs == 128 && kv_bytes * ts == 1024 &&
      kv_page_bytes % 1024 == 0) {
    const int n = num_splits - batch;
    const bool k_high = ((uintptr_t)a.kv.k >> 9) & 1, v_high = ((uintptr_t)a.kv.v >> 9) & 1;
    const int slow = k_high ? 1 : 0;
    const int extra = (int)lround(n * (k_high == v_high ? 0.065 : 0.02));
    const long long total = (long long)batch * spec_pages;
    const int fewest = (int)ceil_div(total, sqa::kMaxSplitPages);
    if (extra > 0 && n - extra >= (fewest > 1 ? fewest : 1)) {
      pa.hg_items[slow] = n + extra;
      pa.hg_items[1 - slow] = n - extra;
      const int pps0 = sqa::packed_item_pages((int)total, pa.hg_items[0]);
      pa.hg_spec_pps1 = sqa::packed_item_pages((int)total, pa.hg_items[1]);
      pa.spec_pps = pps0;
    }
  }
  // Pieces that fit the register ring take it in one softmax step: fixed plans
  // of at most kRingPages pages per split, balanced plans whose expected items
  // are that short (pieces can only be shorter than their item).
  pa.ring_batch = head_dim == 128 && kv_bytes == 2 && rows <= 32 &&
                  (balanced ? (spec_pages > 0 && pa.spec_pps <= sqa::kRingPages)
                            : pages_per_split <= sqa::kRingPages);
  pa.scale_log2 = (float)(1.4426950408889634 * (double)a.scale);
  pa.out_scale = a.out_scale;
  pa.bf16 = a.dtype == SQA_DTYPE_BF16;
  pa.kv_fp8 = kv_fp8;

  hipError_t e;
  if (ev && (e = hipEventRecord(ev[0], s)) != hipSuccess) return hip_fail(e, "hipEventRecord");
  if ((e = sqa::launch_partial(pa, s)) != hipSuccess) return hip_fail(e, "partial kernel launch");
  if (ev && (e = hipEventRecord(ev[1], s)) != hipSuccess) return hip_fail(e, "hipEventRecord");
  if (merged) {
    sqa::MergeArgs ma;
    ma.part_o = pa.part_o;
    ma.part_ml = pa.part_ml;
    ma.seq_splits = pa.seq_splits;
    ma.seq_lens = a.seq_lens;
    ma.out = pa.out;
    ma.batch = batch;
    ma.q_len = q_len;
    ma.hq = num_query_heads;
    ma.hkv = num_kv_heads;
    ma.group = group;
    ma.rows = (int)rows;
    ma.head_dim = head_dim;
    ma.max_pages = (int)kernel_pages;
    ma.pages_per_split = pa.pages_per_split;
    ma.num_splits = num_splits;
    ma.spec_pages = spec_pages;
    ma.spec_pps = pa.spec_pps;
    ma.hg_items[0] = pa.hg_items[0];
    ma.hg_items[1] = pa.hg_items[1];
    ma.hg_spec_pps1 = pa.hg_spec_pps1;
    ma.out_scale = a.out_scale;
    ma.bf16 = pa.bf16;
    ma.tune = pa.pair_items == sqa::kPairsAdaptive ? pa.tune : nullptr;
    ma.tune_records = (num_splits - batch) * 2;
    if ((e = sqa::launch_merge(ma, s)) != hipSuccess) return hip_fail(e, "merge kernel launch");
  }
  if (ev && (e = hipEventRecord(ev[2], s)) != hipSuccess) return hip_fail(e, "hipEventRecord");
  return SQA_OK;
}

// The reference's separate [num_pages, page, Hkv, head_dim] caches, causal draft
// chain, scale head_dim^-1/2; workspace and timing events left empty.
sqa_attention_args mtp_args(const void* query, const void* key_cache, const void* value_cache,
                            const int32_t* block_tables, const int32_t* seq_lens, void* output,
                            int batch, int q_len, int num_query_heads, int num_kv_heads,
                            int head_dim, int64_t num_pages, int page_size, int max_pages,
                            int num_splits, int pages_per_split, void* stream) {
  sqa_attention_args a;
  memset(&a, 0, sizeof(a));
  a.struct_size = sizeof(a);
  a.query = query;
  a.output = output;
  a.kv.k = key_cache;
  a.kv.v = value_cache;
  a.kv.num_pages = num_pages;
  a.kv.token_stride = (int64_t)num_kv_heads * head_dim;
  a.kv.page_stride = (int64_t)page_size * a.kv.token_stride;
  a.kv.head_stride = head_dim;
  a.block_tables = block_tables;
  a.seq_lens = seq_lens;
  a.max_pages = max_pages;
  a.scale = head_dim > 0 ? (float)(1.0 / sqrt((double)head_dim)) : 1.f;
  a.out_scale = 1.f;
  a.batch = batch;
  a.q_len = q_len;
  a.num_query_heads = num_query_heads;
  a.num_kv_heads = num_kv_heads;
  a.head_dim = head_dim;
  a.page_size = page_size;
  a.num_splits = num_splits;
  a.pages_per_split = pages_per_split;
  a.stream = stream;
  return a;
}

// Scratch of the no-allocation entry point: a file-scope device array every GPU
// the library runs on holds (zero-initialised at load) until the process ends.
// Host code never uses the array's name as an address: the device address comes
// from hipGetSymbolAddress, once per device with that device current, and only
// that address reaches kernels. Every call on a device shares its array, so calls
// that overlap on one GPU (other streams, other threads) race on it.
constexpr size_t kScratchBytes = SQA_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_scratch_mutex;
std::vector<void*> g_scratch_ptr;  // per device, nullptr until looked up

int scratch_address(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess || dev < 0) return hip_fail(e, "hipGetDevice");
  try {  // the lock and the table's growth may throw; nothing crosses the C boundary
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if ((int)g_scratch_ptr.size() <= dev) g_scratch_ptr.resize(dev + 1, nullptr);
    if (!g_scratch_ptr[dev]) {
      void* p = nullptr;
      e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
      if (e != hipSuccess || !p) return hip_fail(e, "hipGetSymbolAddress(scratch)");
      g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return SQA_OK;
  } catch (...) {
    return fail(SQA_ERR_HIP, "scratch lookup: out of host memory or lock failure");
  }
}

}  // namespace

extern "C" {

int sqa_paged_attention(const sqa_attention_args* args) {
  if (!args) return fail(SQA_ERR_INVALID, "null argument struct");
  // The layout before `flags` (callers built against it) runs with flags = 0.
  constexpr size_t kLegacySize = offsetof(sqa_attention_args, flags);
  if (args->struct_size == kLegacySize) {
    sqa_attention_args a;
    memset(&a, 0, sizeof(a));
    memcpy(&a, args, kLegacySize);
    a.struct_size = sizeof(a);
    return run_attention(a);
  }
  if (args->struct_size != sizeof(sqa_attention_args))
    return fail(SQA_ERR_INVALID, "struct_size %zu does not match this library's %zu (or %zu)",
                args->struct_size, sizeof(sqa_attention_args), kLegacySize);
  return run_attention(*args);
}

int sqa_paged_mtp_attention(const void* query, const void* key_cache, const void* value_cache,
                            const int32_t* block_tables, const int32_t* seq_lens, void* output,
                            void* workspace, size_t workspace_bytes, int batch, int q_len,
                            int num_query_heads, int num_kv_heads, int head_dim,
                            int64_t num_pages, int page_size, int max_pages, int num_splits,
                            int pages_per_split, void* stream, void** timing_events) {
  sqa_attention_args a = mtp_args(query, key_cache, value_cache, block_tables, seq_lens, output,
                                  batch, q_len, num_query_heads, num_kv_heads, head_dim, num_pages,
                                  page_size, max_pages, num_splits, pages_per_split, stream);
  a.workspace = workspace;
  a.workspace_bytes = workspace_bytes;
  a.timing_events = timing_events;
  return run_attention(a);
}

int sqa_paged_mtp_attention_noalloc(const void* query, const void* key_cache,
                                    const void* value_cache, const int32_t* block_tables,
                                    const int32_t* seq_lens, void* output, int batch, int q_len,
                                    int num_query_heads, int num_kv_heads, int head_dim,
                                    int64_t num_pages, int page_size, int max_pages,
                                    int num_splits, int pages_per_split, void* stream) {
  const size_t need = sqa_workspace_bytes(batch, q_len, num_query_heads, num_kv_heads, head_dim,
                                          num_splits, pages_per_split);
  if (need > kScratchBytes)
    return fail(SQA_ERR_WORKSPACE,
                "the plan needs %zu bytes of scratch; the no-allocation entry point holds at most "
                "%zu (use sqa_paged_mtp_attention with a caller workspace)",
                need, kScratchBytes);
  void* ws = nullptr;
  if (need > 0) {
    const int rc = scratch_address(&ws);
    if (rc != SQA_OK) return rc;
  }
  sqa_attention_args a = mtp_args(query, key_cache, value_cache, block_tables, seq_lens, output,
                                  batch, q_len, num_query_heads, num_kv_heads, head_dim, num_pages,
                                  page_size, max_pages, num_splits, pages_per_split, stream);
  a.workspace = ws;
  a.workspace_bytes = ws ? kScratchBytes : 0;
  return run_attention(a);
}

}  // extern "C"
