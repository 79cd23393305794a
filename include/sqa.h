/*
 * sqa.h - C ABI of libsqa.so, the MI355X (gfx950) paged small-q attention
 * library. Plain pointers, integers and sizes only; no torch types. Every
 * function returns a status and never throws across the boundary.
 *
 * Tensor contract (reference: /root/reference/csrc/small_q_attention_ext.cu:976-1002,
 * /root/reference/src/small_q_attention/cuda.py:61-78):
 *   query        [batch, q_len, num_query_heads, 128]  fp16, contiguous, device
 *                (head_dim 64 and 256 are also built; 128 is the reference's)
 *   key_cache    [num_pages, page_size, num_kv_heads, 128]  fp16, contiguous, device;
 *                page_size 16 (the reference's), 32, 64, 128 or 256
 *   value_cache  same shape as key_cache
 *   block_tables [batch, max_pages] int32, device
 *   seq_lens     [batch] int32, device; KV length including the q_len draft tokens
 *   output       [batch, q_len, num_query_heads, 128]  fp16, device (written)
 * Draft row qi of sequence b attends to tokens t < seq_lens[b] - q_len + qi + 1,
 * query head h reads kv head h / (num_query_heads / num_kv_heads), scale 128^-1/2.
 * Rows that see no token are written as 0 (reference v2-v5 merge, .cu:365).
 * q_len * (num_query_heads / num_kv_heads) must be <= 64.
 */
#ifndef SQA_H_
#define SQA_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Status codes. */
#define SQA_OK 0
#define SQA_ERR_INVALID 1     /* bad argument (shape, null pointer, ...) */
#define SQA_ERR_UNSUPPORTED 2 /* outside the supported contract (head_dim, page size, rows) */
#define SQA_ERR_WORKSPACE 3   /* workspace missing, too small or not 16-byte aligned */
#define SQA_ERR_HIP 4         /* HIP runtime error (launch, device query) */

/* Element types of sqa_attention_args.dtype (query and output) and .kv_dtype
 * (caches: the query's type, or OCP FP8 E4M3 bytes). */
#define SQA_DTYPE_F16 0
#define SQA_DTYPE_BF16 1
#define SQA_DTYPE_FP8_E4M3 2

/*
 * Chooses the split-KV decomposition.
 * Replaces the reference chunking policy (csrc/small_q_attention_ext.cu:1096-1099,
 * :1171-1178; default chunk_keys=512 at src/small_q_attention/cuda.py:127).
 *   chunk_keys > 0: each split owns ceil(chunk_keys / 16) pages (reference meaning);
 *     sequence b's splits are b * num_splits + s, split s covering pages
 *     [s * pages_per_split, (s + 1) * pages_per_split).
 *   chunk_keys == 0: automatic, sized from the device's compute-unit count.
 *     For 2 <= batch <= 256 this is the balanced plan, *pages_per_split <= 0:
 *     *num_splits slots are shared by the whole batch; on the device the
 *     kernel lays all sequences' pages end to end (from seq_lens) and cuts them
 *     into num_splits - batch equal work items that cross sequence ends, so
 *     ragged batches spread evenly over the chip without a host sync. With
 *     max_seq_len > 0 it is -P, P = ceil(max_seq_len / 16) (at most max_pages):
 *     the kernels first assume every sequence spans P pages, which saves a
 *     memory round trip when it holds, and verify it (the result is the same
 *     either way). Otherwise a fixed plan as above.
 * max_pages: 16-token pages a block-table row addresses (block_tables columns
 * x page_size / 16); num_splits and pages_per_split count 16-token pages too.
 * max_seq_len <= 0 means "unknown": a fixed plan covers max_pages * 16 tokens.
 * head_dim: as passed to the attention call (it sets the kernel's heads per
 * workgroup, hence the split count of the automatic plans).
 * Writes *num_splits >= 1 and *pages_per_split (> 0 fixed plan, 0 or -P balanced).
 */
int sqa_plan_splits(int device, int batch, int q_len, int num_query_heads, int num_kv_heads,
                    int head_dim, int max_seq_len, int max_pages, int chunk_keys,
                    int* num_splits, int* pages_per_split);

/*
 * Device workspace bytes sqa_paged_mtp_attention needs for a plan from
 * sqa_plan_splits and a head_dim (0 for a fixed plan with num_splits == 1). Replaces the
 * per-call torch::empty of the partial buffers in the reference launchers
 * (csrc/small_q_attention_ext.cu:1102-1104). A fresh (even uninitialised) or
 * reused workspace is equally valid: without SQA_FLAG_ADAPTIVE_PAIRS no call
 * reads what an earlier call left in it, and the same inputs and plan give the
 * same output bits on every call. A balanced plan's workspace also holds a small
 * record that only calls with SQA_FLAG_ADAPTIVE_PAIRS use (see there).
 */
size_t sqa_workspace_bytes(int batch, int q_len, int num_query_heads, int num_kv_heads,
                           int head_dim, int num_splits, int pages_per_split);

/*
 * Runs the op asynchronously on `stream` (a hipStream_t; NULL = default stream).
 * Replaces the launchers small_q_attention_v0..v5 and their pybind entries
 * forward, forward_v1..forward_v5 (csrc/small_q_attention_ext.cu:969-1378,
 * :1380-1390). num_splits/pages_per_split come from sqa_plan_splits
 * (pages_per_split 0 or -P: balanced plan, batch <= 256, P <= max_pages * page_size / 16
 * and num_splits >= batch + max(1, ceil(batch * max_pages * page_size / 16 / 2048)));
 * max_pages is the
 * block_tables row length. head_dim is 128 (the reference's), 64 or 256;
 * 256 needs q_len * num_query_heads / num_kv_heads <= 32. `workspace` must hold
 * sqa_workspace_bytes(...) bytes, 16-byte aligned (may be NULL when that is 0). query
 * and the caches must be 16-byte aligned, output 8-byte, block_tables and seq_lens
 * 4-byte (SQA_ERR_INVALID otherwise), and a plan's partial sums must stay within
 * 0xFFFF0000 bytes (SQA_ERR_INVALID; the automatic plans need a few MB to ~40 MB).
 * Allocates nothing and never synchronises.
 * `timing_events`: NULL, or an array of 3 hipEvent_t recorded on `stream`
 * before the partial kernel, between the two kernels and after the merge
 * kernel (used by the benchmark to time the partial kernel alone).
 */
int sqa_paged_mtp_attention(const void* query, const void* key_cache, const void* value_cache,
                            const int32_t* block_tables, const int32_t* seq_lens, void* output,
                            void* workspace, size_t workspace_bytes, int batch, int q_len,
                            int num_query_heads, int num_kv_heads, int head_dim,
                            int64_t num_pages, int page_size, int max_pages, int num_splits,
                            int pages_per_split, void* stream, void** timing_events);

/* Device scratch the no-allocation entry point holds per GPU (64 MiB). */
#define SQA_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)

/*
 * sqa_paged_mtp_attention without a workspace argument. No counterpart in the
 * reference: it serves callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
 * The plan's split partials go to a device array of SQA_NOALLOC_SCRATCH_BYTES
 * in a code object of its own (no kernels), which HIP's deferred loading (its
 * default) places on a GPU when the array's address is first looked up there
 * (hipGetSymbolAddress, at this entry point's first call on the device): from
 * then until the process ends that GPU holds it; a process that never calls
 * this entry point holds none. Same
 * arguments, plans, kernels, results and status codes as
 * sqa_paged_mtp_attention, on the current device's array; a plan whose
 * sqa_workspace_bytes exceeds SQA_NOALLOC_SCRATCH_BYTES is rejected with
 * SQA_ERR_WORKSPACE. Allocates nothing, never synchronises. All calls on one
 * GPU share its array: calls that overlap on one GPU (other streams or host
 * threads) race; serialise them.
 */
int sqa_paged_mtp_attention_noalloc(const void* query, const void* key_cache,
                                    const void* value_cache, const int32_t* block_tables,
                                    const int32_t* seq_lens, void* output, int batch, int q_len,
                                    int num_query_heads, int num_kv_heads, int head_dim,
                                    int64_t num_pages, int page_size, int max_pages,
                                    int num_splits, int pages_per_split, void* stream);

/*
 * Where the K and V of a paged cache live, for sqa_paged_attention. Strides
 * are in fp16 elements; the head dimension is contiguous. Element d of kv head
 * h at slot t of page p is k[p * page_stride + t * token_stride + h *
 * head_stride + d] (V alike from v). Strides must be multiples of 8 elements
 * and k, v 16-byte aligned.
 *   separate caches [P, 16, Hkv, D] (the reference's, D = 128): k = key_cache,
 *     v = value_cache, page_stride 16*Hkv*D, token_stride Hkv*D, head_stride D
 *   interleaved NHD [P, 2, 16, Hkv, D]: k = kv, v = kv + 16*Hkv*D,
 *     page_stride 2*16*Hkv*D, token_stride Hkv*D, head_stride D
 *   interleaved HND [P, 2, Hkv, 16, D]: k = kv, v = kv + 16*Hkv*D,
 *     page_stride 2*16*Hkv*D, token_stride D, head_stride 16*D
 */
typedef struct sqa_kv_cache {
  const void* k;
  const void* v;
  int64_t num_pages;
  int64_t page_stride;
  int64_t token_stride;
  int64_t head_stride;
} sqa_kv_cache;

/*
 * Arguments of sqa_paged_attention (set struct_size = sizeof(sqa_attention_args)).
 * query/output/block_tables/seq_lens/plan/workspace/stream/timing_events mean
 * what they mean for sqa_paged_mtp_attention. Additions:
 *   kv          any layout sqa_kv_cache describes.
 *   draft_mask  NULL: the causal draft chain (row qi sees draft tokens j <= qi).
 *               Otherwise [batch, q_len, mask_words] uint32, bit j of the row's
 *               words (word j / 32, bit j % 32) = row qi sees draft token j,
 *               i.e. token seq_lens[b] - q_len + j; tokens before the draft
 *               block are always visible. This is the packed speculative-
 *               decoding mask of the reference's FlashInfer comparisons
 *               (scripts/run_flashinfer_baseline.py:56-85, viewed as uint32).
 *               mask_words >= ceil(q_len / 32), at most 2.
 *   scale       softmax scale (> 0; the reference uses head_dim^-1/2).
 *   out_scale   multiplier of the normalised output (1 for plain attention).
 *   dtype       SQA_DTYPE_F16 (the reference's) or SQA_DTYPE_BF16 for query
 *               and output; accumulation is fp32.
 *   kv_dtype    dtype (caches of the query's type) or SQA_DTYPE_FP8_E4M3:
 *               one byte per element (strides still count elements), widened
 *               exactly to dtype in registers; per-tensor K / V scales go into
 *               scale / out_scale.
 *   flags       0, or SQA_FLAG_ADAPTIVE_PAIRS. A struct_size that stops
 *               before this field (callers built against the layout without
 *               it) means flags = 0.
 */

/*
 * Paired work items: the balanced plan's 64-row kernel (33..64 rows per kv
 * head, head_dim 128, 16-bit K/V, 8 kv heads, every sequence of the expected
 * max_seq_len, pairs of items dividing a sequence) gives work items 2k and
 * 2k + 1 unequal shares of their pages, the even one 3% more, because the XCDs
 * that run the odd ones stream that kernel's pages more slowly (measured on
 * every box; 2% faster at 16 x 32K keys, q_len 16). The shares follow from the
 * plan alone: equal inputs give equal bits.
 *
 * SQA_FLAG_ADAPTIVE_PAIRS: instead of the fixed 3%, a share measured from the
 * previous call's page-loop times, kept in the workspace. The output then
 * depends on that share within the parity tolerance, so identical calls and
 * graph replays may differ in their last bits; without the flag they never do.
 */
#define SQA_FLAG_ADAPTIVE_PAIRS 1
typedef struct sqa_attention_args {
  size_t struct_size;
  const void* query;
  void* output;
  sqa_kv_cache kv;
  const int32_t* block_tables;
  const int32_t* seq_lens;
  int max_pages;
  const uint32_t* draft_mask;
  int mask_words;
  float scale;
  float out_scale;
  int batch;
  int q_len;
  int num_query_heads;
  int num_kv_heads;
  int head_dim;
  int page_size;
  int num_splits;
  int pages_per_split;
  void* workspace;
  size_t workspace_bytes;
  void* stream;
  void** timing_events;
  int dtype;
  int kv_dtype;
  int flags;
} sqa_attention_args;

/*
 * The general form of sqa_paged_mtp_attention: any cache layout of
 * sqa_kv_cache, a caller-given draft mask and scales. No counterpart in the
 * reference's own launchers; it serves the FlashInfer-shaped entry points its
 * comparison scripts call (xqa_batch_decode_with_kv_cache,
 * trtllm_batch_decode_with_kv_cache and the paged decode/prefill wrappers,
 * scripts/run_flashinfer_baseline.py:99-204, scripts/compare_flashinfer_paths.py:95-160).
 * Same plan, workspace, status codes and asynchrony as sqa_paged_mtp_attention.
 */
int sqa_paged_attention(const sqa_attention_args* args);

/* Compute units of `device` (256 on MI355X), or -1 on error. */
int sqa_device_cu_count(int device);

/* Message for the last non-zero status returned on this thread. */
const char* sqa_last_error(void);

/* Library version string. */
const char* sqa_version(void);

#ifdef __cplusplus
}
#endif

#endif /* SQA_H_ */
