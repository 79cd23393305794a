// Streaming-read probe for bench.py: the practical HBM read ceiling the
// attention kernels are measured against. A measurement aid built into its own
// library (libsqa_probe.so, read_probe.py), not part of libsqa.so.
//
// Each workgroup of 256 threads reads one contiguous chunk of the buffer with
// 16-byte non-temporal loads, eight in flight per thread, and folds what it read
// into one dword per thread (so the loads are not removed). The pattern is the
// one a plain read runs fastest with on MI355X (one workgroup of 256 threads per
// CU over contiguous chunks, 2 GiB: ~299 us, 7.18 TB/s); finer or grid-strided
// patterns, more threads per CU and cached loads all measured slower.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdio>
#include <string>

namespace {

typedef unsigned u4 __attribute__((ext_vector_type(4)));

constexpr int kProbeThreads = 256;
constexpr int kProbeUnroll = 8;

__global__ __launch_bounds__(kProbeThreads) void sqa_read_probe_kernel(const u4* __restrict__ in,
                                                                       size_t per_block,
                                                                       unsigned* sink) {
  const u4* p = in + (size_t)blockIdx.x * per_block;
  u4 acc = {0u, 0u, 0u, 0u};
  size_t i = threadIdx.x;
  // Every index stays below per_block: the unrolled loop runs while its last
  // load is in range, the tail loop one load at a time.
  for (; i + (kProbeUnroll - 1) * kProbeThreads < per_block; i += kProbeUnroll * kProbeThreads) {
    u4 v[kProbeUnroll];
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) v[u] = __builtin_nontemporal_load(p + i + u * kProbeThreads);
    // All eight loads are issued before the first wait (left alone, the
    // scheduler interleaves the folds and waits after four: ~15% slower).
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < kProbeUnroll; ++u) acc ^= v[u];
  }
  for (; i < per_block; i += kProbeThreads) acc ^= __builtin_nontemporal_load(p + i);
  sink[(size_t)blockIdx.x * kProbeThreads + threadIdx.x] = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
}

thread_local std::string g_error;

int fail(int code, const char* msg) {
  g_error = msg;
  return code;
}

}  // namespace

extern "C" {

#ifndef SQA_SOURCE_HASH
#define SQA_SOURCE_HASH "unstamped"
#endif
const char* sqa_probe_version(void) { return "sqa-probe gfx950 sqa-src-hash:" SQA_SOURCE_HASH; }

const char* sqa_probe_last_error(void) { return g_error.c_str(); }

// One pass over `bytes` of `data` in `blocks` contiguous chunks (one workgroup of
// 256 threads each), one folded dword per thread written to `sink` (blocks * 256
// dwords). Returns 0, 1 for invalid arguments (checked before any device call)
// or 2 for a HIP error; sqa_probe_last_error() says which.
int sqa_read_probe(const void* data, size_t bytes, unsigned* sink, int blocks, void* stream) {
  if (!data || !sink) return fail(1, "null pointer");
  if (blocks < 1 || blocks > 65536) return fail(1, "blocks must be 1..65536");
  if ((uintptr_t)data % 16 || (uintptr_t)sink % 4)
    return fail(1, "data must be 16-byte and sink 4-byte aligned");
  if (bytes == 0 || bytes % (16 * (size_t)blocks))
    return fail(1, "bytes must be a positive multiple of 16 * blocks");
  const size_t per_block = bytes / 16 / (size_t)blocks;
  hipLaunchKernelGGL(sqa_read_probe_kernel, dim3((unsigned)blocks), dim3(kProbeThreads), 0,
                     (hipStream_t)stream, (const u4*)data, per_block, sink);
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    char msg[256];
    snprintf(msg, sizeof msg, "read probe launch: %s", hipGetErrorString(e));
    return fail(2, msg);
  }
  return 0;
}

}  // extern "C"
