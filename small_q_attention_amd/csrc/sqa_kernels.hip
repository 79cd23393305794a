// gfx950 kernels for paged small-q (speculative-decoding "MTP") attention.
//
// Semantics (reference: /root/reference/src/small_q_attention/reference.py:46-72,
// csrc/small_q_attention_ext.cu:37-54): query head h reads kv head h / group;
// draft row qi of sequence b sees tokens t < seq_lens[b] - q_len + qi + 1;
// token t is slot t % 16 of page block_tables[b, t / 16]; scale head_dim^-1/2;
// fp32 softmax; fp16 output.
//
// Work decomposition. One workgroup owns one work item (sequence b, split: a
// range of its pages) for 4 kv heads, one wave per kv head. A wave holds every
// query row that reads its kv head: rows = q_len * group, row
// r = qi * group + g <-> query head kvh * group + g, so each K/V byte is loaded
// from HBM once and used by all rows straight from registers. The four waves
// walk the same pages in step, so a page's four 256-byte head slices per token
// are requested together (1 KiB contiguous runs).
//
// Per 16-token page a wave issues 4 K and 4 V 16-byte-per-lane buffer loads
// (1 KiB each).
//   S^T[token][row] = K . Q^T : v_mfma_f32_16x16x32_f16, A = K (lane l: token
//     l%16, 8 consecutive dims), B = Q^T (lane l: row l%16, same dims). The head
//     dimension is contracted in the order d = 32*kk + 8*(l/16) + e, which is
//     the same for A and B, so it needs no data movement.
//   O^T[d][row] += V^T . P^T : v_mfma_f32_16x16x16_f16. The S^T accumulator
//     (lane l: tokens 4*(l/16)+0..3 of row l%16) is exactly the B operand, so
//     P never leaves its registers. Lane l loads V rows 4*(l/16)+0..3, dims
//     8*(l%16)+0..7 (four full 256-byte rows per instruction) and regroups
//     them with one byte permute per half pair: output block mb covers dims
//     d = 8*m + mb, m = 0..15.
// Rows beyond q_len*group (q_len*group not a multiple of 16) carry zero Q and
// are never stored. The figures above are for head dim 128; the kernels are
// also built for 64 and 256 (HD), where the per-lane counts scale with HD
// (Dims<HD>) and a ring slot holds a page of HD-wide rows, and at head dim 64
// a wave takes two kv heads (HPW = 2; a workgroup then serves 8 kv heads):
// with up to 8 rows per kv head in one block (rows 0-7 and 8-15), with up to
// 16 or 32 in one or two blocks each (NB = 2 or 4). The element
// traits swap in the bf16 MFMAs (PV then as one 16x16x32 over P's high and low
// parts) and e4m3 K/V widened in registers; where the registers allow, the
// page loop runs the next page's QK products under this page's softmax.
#include "sqa_internal.h"

#include <math.h>

namespace sqa {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef unsigned u4 __attribute__((ext_vector_type(4)));
typedef unsigned u2 __attribute__((ext_vector_type(2)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef __bf16 b8 __attribute__((ext_vector_type(8)));
typedef __bf16 b4 __attribute__((ext_vector_type(4)));

// Element types of Q, K, V and the output. Operands travel as raw 16-bit
// lanes (u4 = 8 elements, u2 = 4); the traits pick the MFMA and the rounding.
struct ElemF16 {
  // Split partials leave as fp16 rows normalised by their sum (a convex
  // combination of V rows, so within V's fp16 range), with (max, sum) in fp32:
  // half the partial bytes written and merged.
  static constexpr bool kHalfPartials = true;
  // S^T += K . Q^T over 32 head dims.
  static __device__ __forceinline__ f4 mma_qk(u4 k, u4 q, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, k),
                                                  __builtin_bit_cast(h8, q), c, 0, 0, 0);
  }
  // O^T += V^T . P^T over 16 tokens; P is one fp16 operand (relative error
  // 2^-11), with no low part.
  static __device__ __forceinline__ f4 mma_pv(u2 v, u2 p, u2 /*lo*/, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(h4, v),
                                                 __builtin_bit_cast(h4, p), c, 0, 0, 0);
  }
  // Rounds four probabilities once; adds the rounded values to l (v_dot2
  // against ones) so O stays an exact convex combination.
  static __device__ __forceinline__ u2 round_p(float p0, float p1, float p2, float p3, float& l,
                                               u2& /*lo*/) {
    const h2 ones = {(_Float16)1.0f, (_Float16)1.0f};
    const h2 lo = {(_Float16)p0, (_Float16)p1};
    const h2 hi = {(_Float16)p2, (_Float16)p3};
    l = __builtin_amdgcn_fdot2(hi, ones, __builtin_amdgcn_fdot2(lo, ones, l, false), false);
    return __builtin_bit_cast(u2, h4{lo[0], lo[1], hi[0], hi[1]});
  }
  static __device__ __forceinline__ u4 pack8(const float (&x)[8]) {
    h8 o;
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = (_Float16)x[i];
    return __builtin_bit_cast(u4, o);
  }
  static __device__ __forceinline__ unsigned pack2(float x, float y) {
    return __builtin_bit_cast(unsigned, h2{(_Float16)x, (_Float16)y});
  }
  static __device__ __forceinline__ u2 pack4(const float (&x)[4]) {
    return __builtin_bit_cast(u2, h4{(_Float16)x[0], (_Float16)x[1], (_Float16)x[2],
                                     (_Float16)x[3]});
  }
  static __device__ __forceinline__ unsigned short pack1(float x) {
    return __builtin_bit_cast(unsigned short, (_Float16)x);
  }
  // Four OCP e4m3 values (bytes of w, low first) -> four fp16 (exact).
  static __device__ __forceinline__ u2 widen_fp8x4(unsigned w) {
    return u2{__builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.f, false)),
              __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w, 1.f, true))};
  }
  // Eight OCP e4m3 values (bytes of w, low first) -> eight fp16 (exact).
  static __device__ __forceinline__ u4 widen_fp8(u2 w) {
    return u4{__builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w[0], 1.f, false)),
              __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w[0], 1.f, true)),
              __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w[1], 1.f, false)),
              __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(w[1], 1.f, true))};
  }
};

struct ElemBF16 {
  // bf16 V can exceed fp16's range and bf16's 8 bits would cost accuracy:
  // partials stay unnormalised fp32.
  static constexpr bool kHalfPartials = false;
  // One bf16 P (relative error 2^-9) would cost up to ~1% on rows that average
  // a few keys; P goes in as hi + lo bf16 parts (~2^-17), both in one PV
  // product.
  static __device__ __forceinline__ f4 mma_qk(u4 k, u4 q, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(b8, k),
                                                   __builtin_bit_cast(b8, q), c, 0, 0, 0);
  }
  // O^T += V^T . (P_hi + P_lo)^T in one 16x16x32 MFMA (on gfx950 as many
  // cycles as the 16x16x16 one): k-slots 0-3 of a lane group take its four
  // tokens with P_hi, slots 4-7 the same tokens with P_lo, so every operand is
  // already in the lane (bf16 q16: 395 -> 358 us against two 16x16x16
  // products).
  static __device__ __forceinline__ f4 mma_pv(u2 v, u2 hi, u2 lo, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(
        __builtin_bit_cast(b8, u4{v[0], v[1], v[0], v[1]}),
        __builtin_bit_cast(b8, u4{hi[0], hi[1], lo[0], lo[1]}), c, 0, 0, 0);
  }
  static __device__ __forceinline__ u2 round_p(float p0, float p1, float p2, float p3, float& l,
                                               u2& lo) {
    const b4 hi = {(__bf16)p0, (__bf16)p1, (__bf16)p2, (__bf16)p3};
    const float h0 = (float)hi[0], h1 = (float)hi[1], h2v = (float)hi[2], h3 = (float)hi[3];
    const b4 lw = {(__bf16)(p0 - h0), (__bf16)(p1 - h1), (__bf16)(p2 - h2v), (__bf16)(p3 - h3)};
    // The row sum takes p itself: hi + lo is within 2^-17 of p, and summing p
    // saves the conversions back (bf16 q16: 363 -> 350 us).
    l += (p0 + p1) + (p2 + p3);
    lo = __builtin_bit_cast(u2, lw);
    return __builtin_bit_cast(u2, hi);
  }
  static __device__ __forceinline__ u4 pack8(const float (&x)[8]) {
    b8 o;
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = (__bf16)x[i];
    return __builtin_bit_cast(u4, o);
  }
  static __device__ __forceinline__ unsigned pack2(float x, float y) {
    typedef __bf16 bb2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(unsigned, bb2{(__bf16)x, (__bf16)y});
  }
  static __device__ __forceinline__ u2 pack4(const float (&x)[4]) {
    return __builtin_bit_cast(u2, b4{(__bf16)x[0], (__bf16)x[1], (__bf16)x[2], (__bf16)x[3]});
  }
  static __device__ __forceinline__ unsigned short pack1(float x) {
    return __builtin_bit_cast(unsigned short, (__bf16)x);
  }
  static __device__ __forceinline__ u2 widen_fp8x4(unsigned w) {
    return u2{__builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.f, false)),
              __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w, 1.f, true))};
  }
  static __device__ __forceinline__ u4 widen_fp8(u2 w) {
    return u4{__builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[0], 1.f, false)),
              __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[0], 1.f, true)),
              __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[1], 1.f, false)),
              __builtin_bit_cast(unsigned, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(w[1], 1.f, true))};
  }
};

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Split partials leave as write-through stores (relaxed agent-scope atomics:
// global_store with sc1, which the XCD's L2 passes on to memory) rather than
// write-back ones: the merge kernel reads them from other XCDs anyway, and
// dirty lines left in the L2s would be written back at the end of the partial
// kernel, before the merge kernel can start (stamped on one box: the merge
// began 1.6 us after the last partial workgroup at 2 MB of partials, 4.5 us at
// 8 MB). Whole calls back to back: one sequence of 32K keys, q_len 8, 34.6 ->
// 31.8 us; 4 x 8K, q_len 4, 30.6 -> 29.7 us; 16 x 32K +-0.7 us.
__device__ __forceinline__ void store_through(void* p, unsigned long long x) {
  __hip_atomic_store((unsigned long long*)p, x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__device__ __forceinline__ float xor_max(float x) {
  x = fmaxf(x, __shfl_xor(x, 16));
  return fmaxf(x, __shfl_xor(x, 32));
}

__device__ __forceinline__ float xor_sum(float x) {
  x += __shfl_xor(x, 16);
  return x + __shfl_xor(x, 32);
}

// Buffer-resource word 3 for gfx9-family raw (untyped, 32-bit) accesses.
constexpr int kBufferFlags = 0x00020000;
// Cache-policy operand of the K/V buffer loads: non-temporal (read once).
constexpr int kStreamAux = 2;
// Cache-policy operand of the partials' buffer stores: device scope (sc1), a
// write-through store, as store_through.
constexpr int kThroughAux = 16;
// A buffer-store offset past every bounded resource here (their sizes stay
// below it): the hardware drops such a store.
constexpr unsigned kDroppedOffset = 0xFFFFFFF0u;

// Per-lane shapes for head dim HD (64, 128 or 256): KK = HD/32 K fragments of
// 8 dims, MB = HD/16 output dim blocks, VW = HD/32 dwords of V per token (HD/16
// dims of one token in 16-bit elements), each lane owning HD/4 output dims.
template <int HD>
struct Dims {
  static constexpr int KK = HD / 32;
  static constexpr int MB = HD / 16;
  static constexpr int VW = HD / 32;
};

// K/V storage. Per page a lane holds K for token l%16 and V for tokens
// 4*(l/16) + 0..3, dims (HD/16)*(l%16) + 0..HD/16-1. The head dims of K
// fragment kk are q_dims(kk, l/16) + 0..7 (Q is loaded with the same map, so
// the QK contraction is unchanged); V and the output mapping are the same for
// every storage type. expand_k() / expand_v() hand the MFMAs 16-bit elements.

template <int HD>
struct KvNative {  // the query's 16-bit type
  static constexpr int kBytes = 2;
  static constexpr int KK = Dims<HD>::KK, VW = Dims<HD>::VW;
  // One 16-byte load per fragment: dims 32*kk + 8*g.
  static __device__ __forceinline__ int q_dims(int kk, int g) { return 32 * kk + 8 * g; }
  static __device__ __forceinline__ unsigned k_lane_bytes(int g) { return 16 * g; }
  static __device__ __forceinline__ unsigned v_lane_bytes(int l16) { return 4 * VW * l16; }
  struct Regs {
    u4 k[KK];
    unsigned v[4][VW];
  };
  static __device__ __forceinline__ void load(Regs& r, __amdgpu_buffer_rsrc_t kr,
                                              __amdgpu_buffer_rsrc_t vr, unsigned k_lane,
                                              unsigned v_lane, unsigned tok) {
#pragma unroll
    for (int kk = 0; kk < KK; ++kk)
      r.k[kk] = __builtin_amdgcn_raw_buffer_load_b128(kr, k_lane + 64 * kk, 0, kStreamAux);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if constexpr (VW == 2) {
        const u2 x = __builtin_amdgcn_raw_buffer_load_b64(vr, v_lane, e * tok, kStreamAux);
        r.v[e][0] = x[0];
        r.v[e][1] = x[1];
      } else {
#pragma unroll
        for (int h = 0; h < VW / 4; ++h) {
          const u4 x = __builtin_amdgcn_raw_buffer_load_b128(vr, v_lane + 16 * h, e * tok,
                                                             kStreamAux);
#pragma unroll
          for (int i = 0; i < 4; ++i) r.v[e][4 * h + i] = x[i];
        }
      }
    }
  }
  template <typename E>
  static __device__ __forceinline__ void expand_k(const Regs& r, u4 (&k)[KK]) {
#pragma unroll
    for (int i = 0; i < KK; ++i) k[i] = r.k[i];
  }
  template <typename E>
  static __device__ __forceinline__ void expand_v(const Regs& r, unsigned (&v)[4][VW]) {
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
      for (int i = 0; i < VW; ++i) v[e][i] = r.v[e][i];
  }
};

template <int HD>
struct KvFp8 {  // OCP e4m3 bytes, widened exactly to the query's type
  static constexpr int kBytes = 1;
  static constexpr int KK = Dims<HD>::KK, VW = Dims<HD>::VW;
  // K rows are HD bytes: 16-byte loads per lane (64 bytes of a row per
  // instruction, as for the 16-bit types; 8-byte loads used 32 bytes per row
  // request and ran at 58% of peak instead of 78%). Load i holds dims
  // 64*i + 16*g + 0..15, i.e. fragments kk = 2i, 2i+1.
  static __device__ __forceinline__ int q_dims(int kk, int g) {
    return 64 * (kk >> 1) + 16 * g + 8 * (kk & 1);
  }
  static __device__ __forceinline__ unsigned k_lane_bytes(int g) { return 16 * g; }
  static __device__ __forceinline__ unsigned v_lane_bytes(int l16) { return 2 * VW * l16; }
  struct Regs {
    u4 k[KK / 2];
    unsigned v[4][VW / 2];  // HD/16 e4m3 bytes per token
  };
  static __device__ __forceinline__ void load(Regs& r, __amdgpu_buffer_rsrc_t kr,
                                              __amdgpu_buffer_rsrc_t vr, unsigned k_lane,
                                              unsigned v_lane, unsigned tok) {
#pragma unroll
    for (int i = 0; i < KK / 2; ++i)
      r.k[i] = __builtin_amdgcn_raw_buffer_load_b128(kr, k_lane + 64 * i, 0, kStreamAux);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if constexpr (VW == 2) {
        r.v[e][0] = __builtin_amdgcn_raw_buffer_load_b32(vr, v_lane, e * tok, kStreamAux);
      } else if constexpr (VW == 4) {
        const u2 x = __builtin_amdgcn_raw_buffer_load_b64(vr, v_lane, e * tok, kStreamAux);
        r.v[e][0] = x[0];
        r.v[e][1] = x[1];
      } else {
        const u4 x = __builtin_amdgcn_raw_buffer_load_b128(vr, v_lane, e * tok, kStreamAux);
#pragma unroll
        for (int i = 0; i < 4; ++i) r.v[e][i] = x[i];
      }
    }
  }
  template <typename E>
  static __device__ __forceinline__ void expand_k(const Regs& r, u4 (&k)[KK]) {
#pragma unroll
    for (int i = 0; i < KK / 2; ++i) {
      k[2 * i] = E::widen_fp8(u2{r.k[i][0], r.k[i][1]});
      k[2 * i + 1] = E::widen_fp8(u2{r.k[i][2], r.k[i][3]});
    }
  }
  template <typename E>
  static __device__ __forceinline__ void expand_v(const Regs& r, unsigned (&v)[4][VW]) {
#pragma unroll
    for (int e = 0; e < 4; ++e)
#pragma unroll
      for (int i = 0; i < VW / 2; ++i) {
        const u2 w = E::widen_fp8x4(r.v[e][i]);
        v[e][2 * i] = w[0];
        v[e][2 * i + 1] = w[1];
      }
  }
};

template <int NB, int HD>
struct WaveState {
  f4 acc[Dims<HD>::MB][NB];  // O^T blocks: lane l holds dims (HD/4)*(l/16)+(HD/16)*r+mb of row 16*nb+l%16
  float m[NB];     // reference max (log2 units, within kMaxLag of the true row max), same in all 4 lane groups
  float l[NB];     // partial row sum over this lane's tokens
  // Kept with m by the page-pair steps (pair_finish): m + kMaxLag, and the
  // exponent offset -(m, or 0 while m is -inf).
  float thr[NB];
  float nmu[NB];
};

// Padding of the LDS page-id table beyond the split's last page: covers the
// ring's look-ahead (at most 2 * D + 1 entries past the end).
constexpr int kIdPad = 64;

__device__ __forceinline__ int clamp_page(int pid, long long num_pages) {
  return (pid >= 0 && (long long)pid < num_pages) ? pid : 0;
}

// The running row max may trail the true max by up to this many log2 units
// (probabilities up to 2^8 = 256, still exact to fp16 precision in P and far
// from any fp32 range limit in the sums). Rows only pay for the cross-lane max
// and the accumulator rescale when a new score exceeds the running max by
// more than this, which after the first page is rare.
constexpr float kMaxLag = 8.0f;

// max(a, b, c) as one v_maximum3_f32 (IEEE maximum: a NaN operand gives NaN).
// fmaxf (maxnum) makes the compiler quiet every operand it cannot prove
// canonical, MFMA results among them, with an extra v_max_f32 x, x, x first,
// which doubled the instructions of the per-page score maxima. The two agree
// except where a score is NaN, and such a score's row is NaN either way (its
// probability enters the row's sums). Invisible tokens are masked to -inf
// before any maximum is taken.
__device__ __forceinline__ float max3_raw(float a, float b, float c) {
  return __builtin_elementwise_maximum(__builtin_elementwise_maximum(a, b), c);
}
__device__ __forceinline__ float max4(f4 v) { return max3_raw(max3_raw(v[0], v[1], v[2]), v[3], v[3]); }

// Bytes {a.lo16, b.lo16} and {a.hi16, b.hi16} of two dwords (v_perm_b32).
__device__ __forceinline__ unsigned pack_lo(unsigned a, unsigned b) {
  return __builtin_amdgcn_perm(b, a, 0x05040100u);
}
__device__ __forceinline__ unsigned pack_hi(unsigned a, unsigned b) {
  return __builtin_amdgcn_perm(b, a, 0x07060302u);
}

// One 16-token page for one wave, in two steps: page_scores() runs the QK
// products, page_finish() masks, updates the softmax state and runs the PV
// products. The pipelined loop issues the next page's scores before this
// page's finish, so those MFMAs run under the softmax.
// sm_q: Q fragments in LDS, [nb][kk][lane] (the B-operand layout).
// HPW = 2 with NB = 1 (one 16-row block, rows 0-7 of kv head 0 of the wave
// and rows 8-15 of head 1): the QK and PV products run once per head over all
// 16 rows; each lane keeps the scores of its own row's head (`upper`: row >=
// 8), and each head's PV product gets the probabilities of its own rows only,
// so both land in the one set of accumulators. HPW = 2 with NB = 2 or 4:
// blocks nb of head nb / (NB / 2) take only that head's K and V.
// A page's K and V widened to the MFMAs' 16-bit type (a register copy for
// 16-bit caches).
template <int HD, int HPW>
struct PageK {
  u4 k[HPW][Dims<HD>::KK];
};
template <int HD, int HPW>
struct PageV {
  unsigned v[HPW][4][Dims<HD>::VW];
};

template <typename E, typename KV, int HD, int HPW>
__device__ __forceinline__ PageK<HD, HPW> widen_k(const typename KV::Regs (&raw)[HPW]) {
  PageK<HD, HPW> kf;
#pragma unroll
  for (int h = 0; h < HPW; ++h) KV::template expand_k<E>(raw[h], kf.k[h]);
  return kf;
}
template <typename E, typename KV, int HD, int HPW>
__device__ __forceinline__ PageV<HD, HPW> widen_v(const typename KV::Regs (&raw)[HPW]) {
  PageV<HD, HPW> pv;
#pragma unroll
  for (int h = 0; h < HPW; ++h) KV::template expand_v<E>(raw[h], pv.v[h]);
  return pv;
}

template <int NB, int HD, typename E, typename KV, int HPW>
__device__ __forceinline__ void page_scores(f4 (&s)[NB], const PageK<HD, HPW>& kf,
                                            const u4* sm_q, int lane, bool upper) {
  constexpr int KK = Dims<HD>::KK;
  static_assert(HPW == 1 || NB <= 4, "two heads per wave: one shared block or NB / 2 each");
  // Raw scores S^T[token][row] = K . Q^T for this page.
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    s[nb] = f4{0.f, 0.f, 0.f, 0.f};
    f4 s1 = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      const u4 qf = sm_q[(nb * KK + kk) * 64 + lane];
      if constexpr (HPW == 2 && NB >= 2) {
        s[nb] = E::mma_qk(kf.k[nb / (NB / 2)][kk], qf, s[nb]);  // head nb / (NB / 2)
      } else {
        s[nb] = E::mma_qk(kf.k[0][kk], qf, s[nb]);
        if constexpr (HPW == 2) s1 = E::mma_qk(kf.k[HPW - 1][kk], qf, s1);
      }
    }
    if constexpr (HPW == 2 && NB == 1) {
#pragma unroll
      for (int e = 0; e < 4; ++e) s[nb][e] = upper ? s1[e] : s[nb][e];
    }
  }
}

// c = softmax scale * log2(e); scores stay raw until the exponent, where the
// scale and the running max meet in one FMA. Visibility on masked pages: token
// t < len is seen by a row when it lies before the draft block
// (t < draft_base = len - q_len) or when bit t - draft_base of the row's draft
// bits is set.
// Scores of tokens a row does not see set to -inf; tok0 = absolute index of
// this lane's first token (4 consecutive tokens).
template <int NB>
__device__ __forceinline__ void mask_scores(f4 (&s)[NB], const unsigned long long (&dbits)[NB],
                                            int draft_base, int tok0, int len) {
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      // Bitwise, not short-circuit, logic: one select per score, no
      // lane-divergent control flow around the scores.
      const int t = tok0 + e;
      const int j = t - draft_base;  // < q_len <= 64 whenever t < len
      const unsigned bit = (unsigned)(dbits[nb] >> (j & 63)) & 1u;
      const unsigned seen = (unsigned)(t < len) & ((unsigned)(j < 0) | bit);
      s[nb][e] = seen ? s[nb][e] : -INFINITY;
    }
  }
}

// Masked pages: scores of tokens a row does not see become -inf, and V rows
// past the sequence end may hold anything (even NaN; 0 * NaN would poison the
// product), so they are zeroed.
template <int NB, int HD, int HPW>
__device__ __forceinline__ void mask_page(f4 (&s)[NB], PageV<HD, HPW>& pv,
                                          const unsigned long long (&dbits)[NB], int draft_base,
                                          int tok0, int len) {
  constexpr int VW = Dims<HD>::VW;
  mask_scores<NB>(s, dbits, draft_base, tok0, len);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    if (tok0 + e >= len) {
#pragma unroll
      for (int h = 0; h < HPW; ++h)
#pragma unroll
        for (int i = 0; i < VW; ++i) pv.v[h][e][i] = 0u;
    }
  }
}

// The running max: lm[nb] holds this lane's max of its new scores (times c); the
// row max is only reduced across the four 16-lane groups when some lane runs
// ahead of its running max.
template <int NB, int HD>
__device__ __forceinline__ void raise_max(WaveState<NB, HD>& st, const float (&lm)[NB]) {
  constexpr int MB = Dims<HD>::MB;
  bool grow = false;
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) grow |= lm[nb] > st.m[nb] + kMaxLag;
  if (__any(grow)) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const float mn = fmaxf(st.m[nb], xor_max(lm[nb]));
      const float alpha = fast_exp2(st.m[nb] - (mn == -INFINITY ? 0.f : mn));
      st.m[nb] = mn;
      st.l[nb] *= alpha;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) st.acc[mb][nb] *= alpha;
    }
  }
}

// One page's probabilities against the running max and its PV products.
template <int NB, int HD, typename E, typename KV, int HPW>
__device__ __forceinline__ void page_pv(WaveState<NB, HD>& st, const f4 (&s)[NB],
                                        const PageV<HD, HPW>& pv, bool upper, float c) {
  constexpr int MB = Dims<HD>::MB;
  // P = 2^(c*s - m), rounded once to the element type; with fp16 the row sum
  // is taken over the rounded values so O is an exact convex combination (with
  // bf16, P is hi + lo and the sum is within 2^-17 of it).
  u2 ph[NB], pl[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const float mu = st.m[nb] == -INFINITY ? 0.f : st.m[nb];
    pl[nb] = u2{0u, 0u};  // stays zero where P has no low part
    ph[nb] = E::round_p(fast_exp2(fmaf(s[nb][0], c, -mu)), fast_exp2(fmaf(s[nb][1], c, -mu)),
                        fast_exp2(fmaf(s[nb][2], c, -mu)), fast_exp2(fmaf(s[nb][3], c, -mu)),
                        st.l[nb], pl[nb]);
  }

  // O^T += V^T . P^T, one 16x16x16 MFMA per (dim block, row block, head). Dim
  // block mb takes half mb%2 of dword mb/2 from the four token rows this lane
  // holds.
  const u2 zero = {0u, 0u};
#pragma unroll
  for (int mb = 0; mb < MB; ++mb) {
    const int j = mb >> 1;
#pragma unroll
    for (int h = 0; h < HPW; ++h) {
      const unsigned w0 = pv.v[h][0][j], w1 = pv.v[h][1][j], w2 = pv.v[h][2][j],
                     w3 = pv.v[h][3][j];
      const u2 av = (mb & 1) == 0 ? u2{pack_lo(w0, w1), pack_lo(w2, w3)}
                                  : u2{pack_hi(w0, w1), pack_hi(w2, w3)};
      // With two heads, head h's product takes only the probabilities of its
      // own rows (the other rows' lanes pass zeros).
      const bool mine = HPW == 1 || NB >= 2 || (h == 1) == upper;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        if (HPW == 2 && NB >= 2 && h != nb / (NB / 2)) continue;  // its own head's V only
        st.acc[mb][nb] =
            E::mma_pv(av, mine ? ph[nb] : zero, mine ? pl[nb] : zero, st.acc[mb][nb]);
      }
    }
  }
}

template <int NB, int HD, typename E, typename KV, int HPW>
__device__ __forceinline__ void page_finish(WaveState<NB, HD>& st, f4 (&s)[NB],
                                            PageV<HD, HPW>& pv, bool upper,
                                            const unsigned long long (&dbits)[NB],
                                            int draft_base, int tok0, int len, bool masked,
                                            float c) {
  if (masked) mask_page<NB, HD, HPW>(s, pv, dbits, draft_base, tok0, len);
  float lm[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) lm[nb] = max4(s[nb]) * c;
  raise_max<NB, HD>(st, lm);
  page_pv<NB, HD, E, KV, HPW>(st, s, pv, upper, c);
}

// Two pages in one softmax step: fp16 queries over an e4m3 cache at head dim
// 128, one kv head per wave (the 64-row kernel, where the math, not the bytes,
// sets the time). s0 / s1: the raw scores of pages p and p + 1; r0 / r1 their
// raw K/V registers. One running-max update covers the 32 tokens, and each PV
// product is one v_mfma_f32_16x16x32_f16 over both pages (k-slots 0-3 of a lane
// group take its four tokens of page p, slots 4-7 the same tokens of page
// p + 1), which costs the cycles of one 16x16x16 product over one page: half
// the PV MFMA time. V is widened per dim block from its bytes, after the bytes
// of tokens past the sequence end are zeroed (they may hold NaN). have1 false:
// page p + 1 is past the piece (its slot holds a zero page); its scores become
// -inf. Same sums as two page_finish steps up to fp32 rounding and the point
// at which the lagging max is raised.
template <int NB>
__device__ __forceinline__ void pair_finish(WaveState<NB, 128>& st, f4 (&s0)[NB], f4 (&s1)[NB],
                                            KvFp8<128>::Regs r0, KvFp8<128>::Regs r1,
                                            bool have1, const unsigned long long (&dbits)[NB],
                                            int draft_base, int tok0, int len, bool masked,
                                            float c) {
  using E = ElemF16;
  constexpr int MB = Dims<128>::MB;
  // Both conditions are uniform over the wave and rare (pages at the draft
  // block or the sequence end; the last pair of a piece of odd length): one
  // branch keeps their selects out of the common step.
  if (masked || !have1) {
    if (masked) {
      mask_scores<NB>(s0, dbits, draft_base, tok0, len);
      mask_scores<NB>(s1, dbits, draft_base, tok0 + kPageSize, len);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (tok0 + e >= len) r0.v[e][0] = r0.v[e][1] = 0u;
        if (tok0 + kPageSize + e >= len) r1.v[e][0] = r1.v[e][1] = 0u;
      }
    }
    if (!have1) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) s1[nb] = f4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
    }
  }

  // The step is VALU-bound (fp8 widening, 32 exponentials per lane): the
  // pair's maxima as four v_maximum3 (no operand quieting), and the threshold and
  // exponent offset kept with the running max instead of recomputed per step
  // (cfg3 shape q16: 214.0 -> 205.0 us, bit-identical).
  float lm[NB];
  bool grow = false;
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    lm[nb] = max3_raw(max3_raw(s0[nb][0], s0[nb][1], s0[nb][2]),
                      max3_raw(s0[nb][3], s1[nb][0], s1[nb][1]),
                      max3_raw(s1[nb][2], s1[nb][3], s1[nb][3])) * c;
    grow |= lm[nb] > st.thr[nb];
  }
  if (__any(grow)) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const float mn = fmaxf(st.m[nb], xor_max(lm[nb]));
      const float alpha = fast_exp2(st.m[nb] - (mn == -INFINITY ? 0.f : mn));
      st.m[nb] = mn;
      st.thr[nb] = mn + kMaxLag;
      st.nmu[nb] = -(mn == -INFINITY ? 0.f : mn);
      st.l[nb] *= alpha;
#pragma unroll
      for (int mb = 0; mb < MB; ++mb) st.acc[mb][nb] *= alpha;
    }
  }

  u4 pp[NB];  // P^T of both pages: this lane's 4 tokens of page p, then of p + 1
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const float nmu = st.nmu[nb];
    u2 unused;
    const u2 a0 = E::round_p(fast_exp2(fmaf(s0[nb][0], c, nmu)), fast_exp2(fmaf(s0[nb][1], c, nmu)),
                             fast_exp2(fmaf(s0[nb][2], c, nmu)), fast_exp2(fmaf(s0[nb][3], c, nmu)),
                             st.l[nb], unused);
    const u2 a1 = E::round_p(fast_exp2(fmaf(s1[nb][0], c, nmu)), fast_exp2(fmaf(s1[nb][1], c, nmu)),
                             fast_exp2(fmaf(s1[nb][2], c, nmu)), fast_exp2(fmaf(s1[nb][3], c, nmu)),
                             st.l[nb], unused);
    pp[nb] = u4{a0[0], a0[1], a1[0], a1[1]};
  }

  // Dim block mb = 2 j + h takes byte 2 (j % 2) + h of the lane's e4m3 dword
  // j / 2 from each of its four token rows of each page. The
  // bytes of token rows 2i and 2i + 1 are interleaved first (one v_perm_b32:
  // {t0 b, t1 b, t0 b+1, t1 b+1}), so each fp8 -> fp16 conversion of a 16-bit
  // word yields the MFMA operand dword itself (tokens 2i, 2i + 1 at one dim):
  // 8 conversions and 4 permutes per j instead of 8 conversions and 8 permutes
  // (widen each token row, then pair the rows' halves). Same values, same bits.
  const unsigned sel = 0x05010400u;  // bytes {t0.b0, t1.b0, t0.b1, t1.b1}; + 0x02020202: b2, b3
#pragma unroll
  for (int j = 0; j < MB / 2; ++j) {
    const unsigned sj = (j & 1) ? sel + 0x02020202u : sel;
    const int d = j >> 1;
    const unsigned x[4] = {__builtin_amdgcn_perm(r0.v[1][d], r0.v[0][d], sj),
                           __builtin_amdgcn_perm(r0.v[3][d], r0.v[2][d], sj),
                           __builtin_amdgcn_perm(r1.v[1][d], r1.v[0][d], sj),
                           __builtin_amdgcn_perm(r1.v[3][d], r1.v[2][d], sj)};
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int mb = 2 * j + h;
      u4 av;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        av[i] = __builtin_bit_cast(
            unsigned, h == 0 ? __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(x[i], 1.f, false)
                             : __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(x[i], 1.f, true));
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
        st.acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(
            __builtin_bit_cast(h8, av), __builtin_bit_cast(h8, pp[nb]), st.acc[mb][nb], 0, 0, 0);
    }
  }
}

// The page range one workgroup owns and where its sequence's result goes.
struct ItemRange {
  int b;        // sequence (-1: no work item for this workgroup)
  int split;    // split index within the sequence
  int p_begin;  // first page (logical index within the sequence)
  int p_end;    // one past the last page
  int len;      // seq_lens[b], clamped to >= 0
  int n_valid;  // splits of this sequence that own pages
  int slot0;    // partial slot of split 0 of this sequence
  int g_end;    // balanced plan: where the piece ends along the item's pages
  int paired;   // a paired item of the expected-page plan (its loop time is timed)
};

// Fixed plan: sequence b owns slots b * num_splits + s.
__device__ __forceinline__ ItemRange fixed_item(const PartialArgs& a, int item) {
  ItemRange r;
  r.b = item / a.num_splits;
  r.split = item - r.b * a.num_splits;
  r.p_begin = r.split * a.pages_per_split;
  r.len = max(a.seq_lens[r.b], 0);
  const int pages = min((r.len + kPageSize - 1) / kPageSize, a.max_pages);
  r.p_end = min(r.p_begin + a.pages_per_split, pages);
  r.n_valid = min((pages + a.pages_per_split - 1) / a.pages_per_split, a.num_splits);
  r.slot0 = r.b * a.num_splits;
  r.g_end = 0;
  r.paired = 0;
  return r;
}

// threadIdx.x through an empty asm statement: what a piece of work derives from
// it is computed inside that piece, not hoisted by the compiler in front of the
// loop over pieces, where it would hold registers through every page loop.
__device__ __forceinline__ int piece_tid() {
  int t = threadIdx.x;
  asm volatile("" : "+v"(t));
  return t;
}

// Inclusive prefix sum over the wave's 64 lanes with DPP: within rows of 16
// lanes by shifts of 1, 2, 4 and 8 (lanes past the row start add 0), then each
// row's total broadcast into the rows after it (lane 15 into rows 1 and 3, lane
// 31 into rows 2 and 3). Six VALU operations instead of six LDS permutes.
__device__ __forceinline__ int wave_inclusive_scan_int(int x) {
  x += __builtin_amdgcn_update_dpp(0, x, 0x111, 0xf, 0xf, true);   // row_shr:1
  x += __builtin_amdgcn_update_dpp(0, x, 0x112, 0xf, 0xf, true);   // row_shr:2
  x += __builtin_amdgcn_update_dpp(0, x, 0x114, 0xf, 0xf, true);   // row_shr:4
  x += __builtin_amdgcn_update_dpp(0, x, 0x118, 0xf, 0xf, true);   // row_shr:8
  x += __builtin_amdgcn_update_dpp(0, x, 0x142, 0xa, 0xf, false);  // row_bcast:15
  x += __builtin_amdgcn_update_dpp(0, x, 0x143, 0xc, 0xf, false);  // row_bcast:31
  return x;
}

// Balanced plan (batch <= kMaxBalancedBatch = 4 x 64), packed: num_splits =
// T + batch slots, T = the work items one wave of resident workgroups holds. The
// pages of all sequences, concatenated in batch order (sequence b's pages start
// at start_b, the sum of the page counts before it), are cut into items of
// P = ceil(total / T) pages (clamped to [kMinSplitPages, kMaxSplitPages]):
// item i is global pages [i P, min((i + 1) P, total)), whatever the lengths,
// so every workgroup streams the same number of pages and none waits for a
// second wave. An item visits each sequence it overlaps as a piece, with its own
// softmax state, rows and partial slot i + b (unique: walking the pages in
// order, each next piece has the next item or the next sequence and neither
// index ever falls, so i + b grows strictly). Sequence b thus owns slots
// [i0_b + b, i1_b + b], i0_b = start_b / P, i1_b = (start_b + pages_b - 1) / P;
// a sequence inside one item is finished by the partial kernel. In a ragged
// batch the positions include the seam gaps (start_b then counts the gaps
// before sequence b too; an item may end inside a gap). Lane l holds
// sequences l, l + 64, l + 128, l + 192: every wave derives the plan on its own
// with wave reductions (no LDS, no barrier), and wave 0 of workgroup 0 writes
// each sequence's (first slot, count) for the merge kernel.
constexpr int kSeqPerLane = kMaxBalancedBatch / 64;

// The per-lane view of the batch a packed plan works from (lane l: sequences
// l + 64 k). Page counts are recomputed from the lengths where needed, which
// keeps the view at two registers per sequence slot: it stays live through the
// item's pieces.
struct PackedBatch {
  int start[kSeqPerLane];  // first global page of each sequence
  int len[kSeqPerLane];    // lengths (0 past the batch)
  int P;                   // pages per item
  int total;               // pages of the batch
};

// A workgroup's view of the balanced plan: its head group's slot count, merge
// table and item size, and whether it writes that table (the first workgroup of
// the call, or with items per head group the first of its group).
struct PlanView {
  int num_splits;
  SeqSplits* table;
  int spec_pps;
  bool writer;
};
__device__ __forceinline__ PlanView plan_view(const PartialArgs& a) {
  return PlanView{a.num_splits, a.seq_splits, a.spec_pps, blockIdx.x == 0};
}
__device__ __forceinline__ PlanView plan_view(const PartialArgs& a, const HeadGroupItems& h) {
  return PlanView{h.slots, a.seq_splits + h.group * a.batch, h.spec_pps, h.item == 0};
}

// Kernel pages of a sequence of `len` tokens within a block-table row.
__device__ __forceinline__ int pages_of(const PartialArgs& a, int len) {
  return min((len + kPageSize - 1) / kPageSize, a.max_pages);
}

// Prefix sums of the page counts and the item size; with write_table, the
// merge kernel's table.
__device__ __forceinline__ void packed_plan(const PartialArgs& a, const PlanView& v,
                                            PackedBatch& pb, bool write_table) {
  const int lane = threadIdx.x & 63;
  // Groups of 64 sequences past the batch hold no pages: their scans are skipped
  // (a uniform branch), and a group's sum is the last lane of its scan.
  const int groups = (a.batch + 63) / 64;
  int base = 0;  // pages of the groups of 64 sequences before this one
  int pages[kSeqPerLane];
#pragma unroll
  for (int k = 0; k < kSeqPerLane; ++k) {
    pages[k] = pages_of(a, pb.len[k]);
    pb.start[k] = base;
    if (k < groups) {
      const int incl = wave_inclusive_scan_int(pages[k]);
      pb.start[k] += incl - pages[k];
      base += __builtin_amdgcn_readlane(incl, 63);
    }
  }
  // Wave sums are the same in every lane; readfirstlane says so to the
  // compiler, which keeps the loop over pieces (and the page ids loaded in it)
  // uniform rather than wrapping each buffer load in a waterfall loop.
  pb.total = __builtin_amdgcn_readfirstlane(base);
  const int target = v.num_splits - a.batch;
  pb.P = packed_item_pages(pb.total, target);
  // Seams (ragged batches): seam_pages of nothing before every sequence start
  // that is not on an item boundary of the layout without them, so an item that
  // spans the start carries fewer pages; skipped where the gaps would need
  // items over kMaxSplitPages pages, or items are too short for them to matter.
  const int first_pages = __builtin_amdgcn_readfirstlane(pages[0]);
  bool ragged = false;
#pragma unroll
  for (int k = 0; k < kSeqPerLane; ++k) ragged |= 64 * k + lane < a.batch && pages[k] != first_pages;
  const int seam = a.seam_pages;
  if (seam > 0 && pb.P >= 4 * seam && __any(ragged)) {  // uniform
    int gap_base = 0;
    int vstart[kSeqPerLane];
#pragma unroll
    for (int k = 0; k < kSeqPerLane; ++k) {
      const int gap = pages[k] > 0 && pb.start[k] % pb.P != 0 ? seam : 0;
      vstart[k] = pb.start[k] + gap_base;
      if (k < groups) {
        const int incl = wave_inclusive_scan_int(gap);
        vstart[k] += incl;
        gap_base += __builtin_amdgcn_readlane(incl, 63);
      }
    }
    const int total = pb.total + __builtin_amdgcn_readfirstlane(gap_base);
    if (total <= target * kMaxSplitPages) {  // uniform
#pragma unroll
      for (int k = 0; k < kSeqPerLane; ++k) pb.start[k] = vstart[k];
      pb.total = total;
      pb.P = packed_item_pages(total, target);
    }
  }
  if (write_table && threadIdx.x < 64) {
#pragma unroll
    for (int k = 0; k < kSeqPerLane; ++k) {
      const int sq = 64 * k + lane;
      if (sq < a.batch) {
        const int i0 = pb.start[k] / pb.P;
        const int count = pages[k] > 0 ? (pb.start[k] + pages[k] - 1) / pb.P - i0 + 1 : 0;
        v.table[sq] = SeqSplits{min(i0 + sq, v.num_splits - 1), count};
      }
    }
  }
}

// The piece of item `item` from position g on (g inside the item): the first
// sequence with pages that end after g (the one holding g, or the next one if g
// lies in the gap before a sequence start), its page range (within the
// sequence), length, split count and slot, and where the piece ends. The wave
// finds the lane holding that sequence with one ballot per sequence slot;
// everything after is scalar.
__device__ __forceinline__ ItemRange packed_piece(const PartialArgs& a, const PackedBatch& pb,
                                                 int item, int g, int item_end) {
  int b = -1, st = 0, len = 0;
#pragma unroll
  for (int k = 0; k < kSeqPerLane; ++k) {
    // Lengths are 0 past the batch: those slots have no pages.
    const int np = pages_of(a, pb.len[k]);
    const bool mine = np > 0 && g < pb.start[k] + np;
    const unsigned long long hit = __ballot(mine);
    if (hit && b < 0) {
      const int src = __builtin_ctzll(hit);
      b = 64 * k + src;
      st = __builtin_amdgcn_readlane(pb.start[k], src);  // src is uniform
      len = __builtin_amdgcn_readlane(pb.len[k], src);
    }
  }
  ItemRange r;
  const int np = pages_of(a, len);
  const int g_end = min(item_end, pb.total);
  r.b = b;
  r.split = 0;
  r.len = len;
  r.p_begin = max(g - st, 0);
  r.p_end = min(g_end, st + np) - st;  // <= p_begin: the item ends in the gap
  r.n_valid = (st + np - 1) / pb.P - st / pb.P + 1;
  r.slot0 = item + b;
  r.g_end = st + r.p_end;
  r.paired = 0;
  return r;
}

// Lengths of sequences l, l + 64, l + 128, l + 192 in lane l (0 past the
// batch). The loads are unconditional, from clamped in-bounds addresses, and
// selected afterwards: a load under a branch is waited for where the branch
// joins, which would put a full memory round trip in front of whatever follows.
__device__ __forceinline__ void load_lengths(const PartialArgs& a, int (&len)[kSeqPerLane]) {
  const int lane = threadIdx.x & 63;
  int raw[kSeqPerLane];
#pragma unroll
  for (int k = 0; k < kSeqPerLane; ++k) raw[k] = a.seq_lens[min(64 * k + lane, a.batch - 1)];
#pragma unroll
  for (int k = 0; k < kSeqPerLane; ++k) len[k] = 64 * k + lane < a.batch ? max(raw[k], 0) : 0;
}

// The rows of a wave: row slot r (0..15) of 16-row block nb is row row(nb, r)
// (= qi * group + g) of kv head head(nb, r), real() unless it is padding (past
// the rows of a head, or a head past the last). One kv head per wave (HPW = 1):
// blocks nb hold rows 16 nb + r. Two (HPW = 2, head dim 64): one shared block,
// rows 0-7 of the first head in slots 0-7 and of the second in 8-15, or NB / 2
// blocks per head.
template <int NB, int HPW>
struct WaveRows {
  int kvh, rows, hkv;  // the wave's first kv head; rows per kv head; kv heads
  static constexpr int kBlocksPerHead = NB >= 2 ? NB / HPW : 1;
  __device__ __forceinline__ int head(int nb, int r) const {
    return kvh + (HPW == 1 ? 0 : (NB == 1 ? r >> 3 : nb / kBlocksPerHead));
  }
  __device__ __forceinline__ int row(int nb, int r) const {
    return HPW == 1 ? nb * 16 + r : (NB == 1 ? (r & 7) : (nb % kBlocksPerHead) * 16 + r);
  }
  __device__ __forceinline__ bool real(int nb, int r) const {
    return head(nb, r) < hkv && row(nb, r) < rows;
  }
};

// Runs `piece(range, first_id)` for every piece of workgroup item `item`, with
// the ids of the piece's first D pages loaded (index clamped into the
// block-table row; ids past the piece are never used). Fixed plan: one piece
// whose page range follows from `item` alone, so its ids are issued before the
// sequence length is read and both arrive in one round trip. Balanced plan:
// all lengths, the packed plan's wave reductions, then each piece's ids; with
// an expected page count (every sequence spec_pages pages, item size spec_pps
// from the host) the plan needs no lengths, so the first piece's ids go out
// with them, and a length that does not match falls back to the plan from the
// loaded lengths. Piece fields are the same in every lane (readfirstlane): the
// piece, and the buffer-resource addresses built from it, stay in scalar
// registers. Consecutive pieces are separated by a barrier (they reuse the
// workgroup's LDS). Returns whether the item ran as a paired item (every
// workgroup of a call returns the same).
template <int D, typename Piece>
__device__ __forceinline__ bool for_each_piece(const PartialArgs& a, const PlanView& v, int item,
                                               Piece&& piece) {
  const int lane = threadIdx.x & 63;
  const bool balanced = is_balanced(a.pages_per_split);
  int first_id[D];
  auto load_first_ids = [&](int seq, int p0) {
    const int32_t* row = a.block_tables + (size_t)max(seq, 0) * a.bt_stride;
#pragma unroll
    for (int j = 0; j < D; ++j)
      first_id[j] = row[min(max(p0 + j, 0), a.max_pages - 1) >> a.page_shift];
  };
  PackedBatch pb;
  ItemRange it;
  bool ids_loaded = false;
  int g = 0, g_end = 1;  // global pages still to visit (fixed plan: one piece)
  int item_end = 0;      // balanced plan: where the item ends
  bool paired = false;
  if (!balanced) {
    const int seq = item / a.num_splits;
    load_first_ids(seq, (item - seq * a.num_splits) * a.pages_per_split);
    ids_loaded = true;
    it = fixed_item(a, item);
  } else {
    if (a.spec_pages > 0) {
      // Every sequence spec_pages pages: sequence b starts at b * spec_pages;
      // the item size comes from the host. The first piece's ids go out with
      // the lengths (index clamped: an item past the batch never uses them).
      const int P = a.spec_pages;
#pragma unroll
      for (int k = 0; k < kSeqPerLane; ++k) pb.start[k] = min(64 * k + lane, a.batch) * P;
      pb.total = a.batch * P;
      pb.P = v.spec_pps;
      if (v.writer && threadIdx.x < 64) {
#pragma unroll
        for (int k = 0; k < kSeqPerLane; ++k) {
          const int sq = 64 * k + lane;
          if (sq < a.batch) {
            const int i0 = pb.start[k] / pb.P;
            v.table[sq] = SeqSplits{i0 + sq, (pb.start[k] + P - 1) / pb.P - i0 + 1};
          }
        }
      }
      // Paired items: the shared boundary of items 2k and 2k + 1 moves by d
      // pages; delta is the fixed one, or (adaptive pairs) the record's, read
      // with the lengths, the first ids after.
      paired = a.pair_items != 0;
      int g0 = item * pb.P;
      item_end = g0 + pb.P;
      if (paired) {
        float dl = kPairDeltaFixed;
        if (a.pair_items == kPairsAdaptive) {
          const float2 rec = *(const float2*)a.tune;
          dl = __float_as_uint(rec.x) == kTuneMagic ? rec.y : 0.f;
        }
        load_lengths(a, pb.len);
        dl = dl == dl ? fminf(fmaxf(dl, -kPairDeltaMax), kPairDeltaMax) : 0.f;
        // Both items of a pair stay within kMaxSplitPages (the page-id table).
        const int dmax = kMaxSplitPages - pb.P;
        const int d = __builtin_amdgcn_readfirstlane(
            min(max((int)rintf((float)pb.P * dl), -dmax), dmax));
        g0 = (item >> 1) * 2 * pb.P + ((item & 1) ? pb.P + d : 0);
        item_end = (item >> 1) * 2 * pb.P + ((item & 1) ? 2 * pb.P : pb.P + d);
      }
      const int b0 = min(g0 / P, a.batch - 1);
      load_first_ids(b0, g0 - b0 * P);
      if (!paired) load_lengths(a, pb.len);
      bool differs = false;
#pragma unroll
      for (int k = 0; k < kSeqPerLane; ++k)
        differs |= 64 * k + lane < a.batch && pages_of(a, pb.len[k]) != P;
      if (__any(differs)) {
        packed_plan(a, v, pb, v.writer);  // rewrites the table
        paired = false;
      } else {
        ids_loaded = true;
      }
      if (paired) g = g0;
    } else {
      load_lengths(a, pb.len);
      packed_plan(a, v, pb, v.writer);
    }
    if (!paired) {
      g = item * pb.P;
      item_end = g + pb.P;
    }
    g_end = min(item_end, pb.total);
  }
  // The same in every lane (readfirstlane tells the compiler, which otherwise
  // runs the loop under an exec mask).
  g = __builtin_amdgcn_readfirstlane(g);
  g_end = __builtin_amdgcn_readfirstlane(g_end);
  for (bool first = true; g < g_end; first = false) {  // uniform
    if (balanced) it = packed_piece(a, pb, item, g, item_end);
    it.paired = paired;
    it.b = __builtin_amdgcn_readfirstlane(it.b);
    it.split = __builtin_amdgcn_readfirstlane(it.split);
    it.p_begin = __builtin_amdgcn_readfirstlane(it.p_begin);
    it.p_end = __builtin_amdgcn_readfirstlane(it.p_end);
    it.len = __builtin_amdgcn_readfirstlane(it.len);
    it.n_valid = __builtin_amdgcn_readfirstlane(it.n_valid);
    it.slot0 = __builtin_amdgcn_readfirstlane(it.slot0);
    // A piece has a sequence and at least one page unless the item ends in the
    // gap before a sequence start (no further pieces then); the check also keeps
    // the loop finite whatever the inputs.
    if (balanced && (it.b < 0 || it.p_end <= it.p_begin)) break;
    // Uniform addresses (the fields above) make the ids uniform values: the
    // buffer resources built from them stay in scalar registers.
    if (!ids_loaded) load_first_ids(it.b, it.p_begin);
    ids_loaded = false;
    if (!first) __syncthreads();  // the previous piece is done with the LDS
    piece(it, first_id);
    g = __builtin_amdgcn_readfirstlane(balanced ? it.g_end : g + 1);
  }
  return paired;
}

// Draft bits of a row of sequence b, draft row qi: bit j = the row sees draft
// token j (the caller's mask, or the causal chain j <= qi); 0 for padding rows.
// Both mask words are loaded unconditionally (without a mask: from seq_lens,
// never used) and selected by bit masks, not by branches on loaded values, so
// the compiler need not wait for them before later loads are issued.
__device__ __forceinline__ unsigned long long draft_bits(const PartialArgs& a, int b, int qi,
                                                         bool real) {
  const bool has_mask = a.draft_mask != nullptr;
  const uint32_t* mp = has_mask ? a.draft_mask + (size_t)(b * a.q_len + qi) * a.mask_words
                                : (const uint32_t*)a.seq_lens;
  const unsigned long long lo = mp[0];
  const unsigned long long hi = mp[a.mask_words > 1 ? 1 : 0];
  const unsigned long long causal = qi >= 63 ? ~0ull : (2ull << qi) - 1ull;
  const unsigned long long use_mask = 0ull - (unsigned long long)(has_mask && real);
  const unsigned long long use_hi = 0ull - (unsigned long long)(a.mask_words > 1);
  const unsigned long long use_causal = 0ull - (unsigned long long)(!has_mask && real);
  return ((lo | ((hi << 32) & use_hi)) & use_mask) | (causal & use_causal);
}

// Leaves one wave's results: normalised rows of the output (`direct`: the
// sequence's pages fit one split) or the unnormalised partial sums and (max in
// log2 units, sum) of each row at partial slot `slot`. Row slot r of block nb is
// map.real(nb, r), kv head map.head(nb, r), row map.row(nb, r) of that head.
// `mark_done` (a fixed plan with several splits, finished here) also writes
// l = -1 at the slot, which tells the merge kernel the row is in the output.
// The results leave through LDS one 16-row block at a time: every lane writes
// its dims (HD/4) (l/16) + (HD/16) rr + mb of row l % 16 row-major into the
// wave's `stage` (16 rows of HD + 4 floats; the pad spreads rows over banks),
// then reads back 4 contiguous values of a row, so a store instruction writes
// whole rows (1 KiB runs of partial sums) instead of 64 scattered 16-byte
// pieces, which ran at a quarter of the store rate (the epilogue of a 64-row
// wave took 5 us).
template <int NB, int HD, typename E, typename Map>
__device__ __forceinline__ void write_results(const PartialArgs& a, WaveState<NB, HD>& st,
                                              float* stage, const Map& map, bool direct,
                                              bool mark_done, int b, size_t slot,
                                              int slot_heads, int head0) {
  constexpr int MB = Dims<HD>::MB;
  constexpr int kStageRow = HD + 4;  // floats per staged row
  constexpr int CPR = HD / 4;        // 4-value chunks per row
  const int lane = piece_tid() & 63;
  const int g16 = lane >> 4, l16 = lane & 15;
  // Partial slots of slot_heads kv heads from head0 on: all of them (hkv, 0), or
  // with items per head group the group's four (4, 4 group; slot counts from
  // the start of the group's region).
  auto item_of = [&](int nb, int r) {
    return (slot * slot_heads + map.head(nb, r) - head0) * a.rows;
  };
  // Row sums over the four lane groups.
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) st.l[nb] = xor_sum(st.l[nb]);
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    if (map.row(nb, 0) >= a.rows) break;  // uniform
    // l = 0: the row saw no key (written as 0). A NaN l (a NaN score or
    // probability the row saw) passes, so the NaN reaches the row's output.
    const float inv_l = !(st.l[nb] <= 0.f) ? 1.f / st.l[nb] : 0.f;
    const float sc = direct ? a.out_scale * inv_l : (E::kHalfPartials ? inv_l : 1.f);
    if (map.real(nb, l16)) {
      float* dst = stage + l16 * kStageRow + (HD / 4) * g16;
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
#pragma unroll
        for (int h = 0; h < MB / 4; ++h) {
          f4 o;
#pragma unroll
          for (int mb = 0; mb < 4; ++mb) o[mb] = st.acc[4 * h + mb][nb][rr] * sc;
          *(f4*)(dst + MB * rr + 4 * h) = o;
        }
      }
    }
    // The staging rows are this wave's own: LDS keeps a wave's accesses in
    // order, the fences keep the compiler from moving them. All reads are
    // issued before the first store, so the block pays one LDS latency.
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    if (direct) {
      f4 v[CPR / 4];
#pragma unroll
      for (int i = 0; i < CPR / 4; ++i) {
        const int e = i * 64 + lane;  // row e / CPR (< 16), chunk e % CPR
        v[i] = *(const f4*)(stage + (e / CPR) * kStageRow + 4 * (e % CPR));
      }
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      if (mark_done && g16 == 0 && map.real(nb, l16)) {
        const size_t pitem = item_of(nb, l16) + map.row(nb, l16);
        a.part_ml[pitem * 2 + 0] = -INFINITY;
        a.part_ml[pitem * 2 + 1] = -1.f;
      }
#pragma unroll
      for (int i = 0; i < CPR / 4; ++i) {
        const int e = i * 64 + lane;
        const int rs = e / CPR;
        if (map.real(nb, rs)) {
          const int r = map.row(nb, rs);
          const int qi = r / a.group;
          const int gg = r - qi * a.group;
          _Float16* op = a.out + ((size_t)(b * a.q_len + qi) * a.hq +
                                  map.head(nb, rs) * a.group + gg) * HD + 4 * (e % CPR);
          const float o[4] = {v[i][0], v[i][1], v[i][2], v[i][3]};
          *(u2*)op = E::pack4(o);
        }
      }
    } else {
      // Partial rows: 16 bytes per lane (8 fp16 or 4 fp32 values), each store
      // a write-through buffer store (sc1) through a resource bounded to the
      // partials, with padding rows sent past its end, where the hardware drops
      // them: no branch per store, and half the store instructions of 8-byte
      // stores, whose issue took 0.9 us per 16-row block (stamped; whole calls
      // back to back: 16 x 32K keys q_len 8 320.9 -> 319.5 us, 16 x 8K 89.8 ->
      // 88.8 us, one sequence of 8K keys q_len 8 19.3 -> 18.8 us).
      constexpr int DPL = E::kHalfPartials ? 8 : 4;  // values per lane and store
      constexpr int PPR = HD / DPL;                   // 16-byte pieces per row
      constexpr int esz = E::kHalfPartials ? 2 : 4;
      f4 w[PPR / 4][DPL / 4];
#pragma unroll
      for (int i = 0; i < PPR / 4; ++i) {
        const int e = i * 64 + lane;  // row e / PPR (< 16), piece e % PPR
#pragma unroll
        for (int h = 0; h < DPL / 4; ++h)
          w[i][h] = *(const f4*)(stage + (e / PPR) * kStageRow + DPL * (e % PPR) + 4 * h);
      }
      __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
      const __amdgpu_buffer_rsrc_t pr = __builtin_amdgcn_make_buffer_rsrc(
          (void*)a.part_o, (short)0, (int)a.part_o_bytes, kBufferFlags);
#pragma unroll
      for (int i = 0; i < PPR / 4; ++i) {
        const int e = i * 64 + lane;
        const int rs = e / PPR;
        const unsigned at =
            (unsigned)(((item_of(nb, rs) + map.row(nb, rs)) * HD + DPL * (e % PPR)) * esz);
        const unsigned off = map.real(nb, rs) ? at : kDroppedOffset;
        u4 data;
        if constexpr (E::kHalfPartials) {
          const float o[8] = {w[i][0][0], w[i][0][1], w[i][0][2], w[i][0][3],
                              w[i][1][0], w[i][1][1], w[i][1][2], w[i][1][3]};
          data = E::pack8(o);
        } else {
          data = __builtin_bit_cast(u4, w[i][0]);
        }
        __builtin_amdgcn_raw_buffer_store_b128(data, pr, off, 0, kThroughAux);
      }
      if (g16 == 0 && map.real(nb, l16)) {
        const size_t pitem = item_of(nb, l16) + map.row(nb, l16);
        // A NaN sum travels with a finite max, so the merge counts the split.
        const float m_out = st.l[nb] == st.l[nb] ? st.m[nb] : 0.f;
        store_through(a.part_ml + pitem * 2,
                      __builtin_bit_cast(unsigned long long, float2{m_out, st.l[nb]}));
      }
    }
  }
}

// A fixed-plan split past its sequence's pages (the balanced plan has none):
// the merge reads every split of a sequence without its length, so the split's
// rows say "no keys" (l = 0), or, when the sequence fitted one split and is
// already in the output, "done" (l = -1).
template <int NB, typename Map>
__device__ __forceinline__ void write_empty_split(const PartialArgs& a, const Map& map,
                                                  size_t slot, float mark) {
  const int lane = piece_tid() & 63;
  if ((lane >> 4) != 0) return;
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    if (map.real(nb, lane)) {
      const size_t pitem = (slot * a.hkv + map.head(nb, lane)) * a.rows + map.row(nb, lane);
      a.part_ml[pitem * 2 + 0] = -INFINITY;
      a.part_ml[pitem * 2 + 1] = mark;
    }
  }
}

// One workgroup = one (sequence b, split) x WW waves; wave w serves the HPW kv
// heads from (head_group * WW + w) * HPW with all of their rows (NB blocks of
// 16; with HPW = 2 either one block, rows 0-7 of the first head and 8-15 of
// the second, or one block per head); WPE = waves per SIMD the register
// budget allows. All waves walk the
// same pages in the same order, so the heads' 256-byte slices of each page are
// requested together and HBM sees 1 KiB (4 heads) or 2 KiB (8 heads) runs; the
// head groups of a page range are dispatch neighbours. Each wave keeps its own
// softmax state and writes its own partials (or, with a single split, the
// output). Every K/V byte is read by one wave only, so the loads are
// non-temporal.
template <int NB, int D, int WW, int WPE, int HD, typename E, typename KV, int HPW,
          bool RB = false>
__global__ __launch_bounds__(WW * 64) __attribute__((amdgpu_waves_per_eu(WPE)))
void sqa_partial_kernel(PartialArgs a) {
  constexpr int KK = Dims<HD>::KK, MB = Dims<HD>::MB;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

  // blockIdx.x = item * head_groups + head_group, or with items per head group
  // (hg_items) as head_group_items() deals them.
  const int head_groups = (a.hkv + WW * HPW - 1) / (WW * HPW);
  const bool hg_split = a.hg_items[0] > 0;
  const HeadGroupItems hgi =
      head_group_items(a.hg_items, a.batch, a.spec_pps, a.hg_spec_pps1, blockIdx.x);
  const int hgrp = hg_split ? hgi.group : (int)blockIdx.x % head_groups;
  const int item = hg_split ? hgi.item : (int)blockIdx.x / head_groups;
  const PlanView view = hg_split ? plan_view(a, hgi) : plan_view(a);
  const int slot_heads = hg_split ? WW : a.hkv;  // partial slot layout (write_results)
  const int head0 = hg_split ? hgrp * WW : 0;
  const int slot_base = hg_split ? hgi.slot_base : 0;
  const int kvh = (hgrp * WW + wave) * HPW;  // the wave's first kv head
  // Waves past the last kv head (hkv not a multiple of WW * HPW) idle but stay
  // for the barrier.
  const bool active = kvh < a.hkv;
  const WaveRows<NB, HPW> map{kvh, a.rows, a.hkv};

  const bool balanced = is_balanced(a.pages_per_split);
  const bool single = !balanced && a.num_splits == 1;  // no merge kernel follows
  static_assert(2 * D + 1 <= kIdPad, "page-id table padding must cover the ring's look-ahead");
  constexpr int kIdSlots = (kMaxSplitPages + kIdPad + WW * 64 - 1) / (WW * 64);
  // LDS: the Q fragments of this wave's rows, [wave][nb][kk][lane] (the
  // B-operand layout; each lane stores exactly the fragments it reads back),
  // and the piece's page ids: ids of [p_begin, p_end) clamped into the pool,
  // then -1 for the ring's look-ahead. Waves read ids back a step ahead of
  // use, so no page waits on a block-table load from memory. sm_stage holds
  // each wave's results on their way out (the epilogue below).
  __shared__ u4 sm_q[WW * NB * KK * 64];
  __shared__ float sm_stage[WW * 16 * (HD + 4)];
  __shared__ int sm_ids[kIdSlots * WW * 64];

  // Each piece of the work item (one, except where a balanced item spans the
  // end of a sequence): its page range of one sequence, with the ids of its
  // first D pages already requested.
  for_each_piece<D>(a, view, item, [&](const ItemRange& it, const int (&first_id)[D]) {
  const int tid = piece_tid();
  const int lane = tid & 63;
  const int g16 = lane >> 4;
  const int l16 = lane & 15;
  const int b = max(it.b, 0);
  const int split = it.split;
  const int len = it.len;
  const int p_begin = it.p_begin;
  const int p_end = it.p_end;
  const int32_t* bt_row = a.block_tables + (size_t)b * a.bt_stride;
  const int shift = a.page_shift;
  const int sub_mask = (1 << shift) - 1;
  if (it.b < 0) return;  // uniform: no work item
  // A sequence with at most one split is finished here; otherwise this
  // workgroup leaves a partial for the merge kernel.
  const bool direct = it.n_valid <= 1;
  const size_t slot = (size_t)it.slot0 + split;
  if (p_begin >= p_end && !single) {  // fixed plan only
    if (active) write_empty_split<NB>(a, map, slot, it.n_valid == 1 ? -1.f : 0.f);
    return;  // uniform
  }
  const int n_split = p_end - p_begin;
  const int n_pages = active ? n_split : 0;

  // Second: Q fragments, the rest of the split's page ids and the first D
  // pages, all in flight at once (Q and ids first, so waiting for them leaves
  // the page loads outstanding).
  u4 qreg[NB][KK];
  unsigned long long dbits[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    // Loads are unconditional from an in-bounds address (padding rows and idle
    // waves read row 0 of kv head 0) and the value is selected afterwards, so
    // no lane-divergent branch splits the load stream.
    const int r = map.row(nb, l16);
    const bool real = map.real(nb, l16);
    const int qi = real ? r / a.group : 0;
    const int gg = real ? r - qi * a.group : 0;
    const int hh = real ? map.head(nb, l16) * a.group + gg : 0;
    const _Float16* qp = a.q + ((size_t)(b * a.q_len + qi) * a.hq + hh) * HD;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      const u4 x = *(const u4*)(qp + KV::q_dims(kk, g16));
      qreg[nb][kk] = real ? x : u4{0u, 0u, 0u, 0u};
    }
    dbits[nb] = draft_bits(a, b, qi, real);
  }
  int idreg[kIdSlots];
  const int last_id = n_split > 0 ? n_split - 1 : 0;  // p_begin + last_id < max_pages
#pragma unroll
  for (int k = 0; k < kIdSlots; ++k) {
    const int i = tid + k * WW * 64;
    const int x = bt_row[(p_begin + min(i, last_id)) >> shift];
    idreg[k] = i < n_split ? x : -1;
  }

  // K/V pages are read with buffer loads: the resource (4 SGPRs) is rebuilt per
  // page at the page's base address and bounded to the page, and the lane
  // offsets below stay in one VGPR each for the whole loop.
  const int kvh_c = active ? kvh : 0;
  const unsigned tok_bytes = a.token_stride;
  const unsigned k_lane = l16 * tok_bytes + kvh_c * a.head_stride + KV::k_lane_bytes(g16);
  const unsigned v_lane = 4 * g16 * tok_bytes + kvh_c * a.head_stride + KV::v_lane_bytes(l16);
  // Offset of the wave's second head (the first head again if it does not exist).
  const unsigned head1 = HPW == 2 && kvh_c + 1 < a.hkv ? a.head_stride : 0u;
  // pid < 0 gives a zero-length resource: the loads return zeros without
  // touching memory, so every slot refill below is unconditional and the
  // compiler's wait counts stay exact (one page retires per step). K/V are
  // streamed once, so the loads are non-temporal.
  // Kernel page p of the sequence is sub-page p & sub_mask of cache page
  // block_tables[b][p >> shift].
  const size_t sub_bytes = (size_t)kPageSize * tok_bytes;
  auto load_page = [&](int pid, int p, typename KV::Regs (&pg)[HPW]) {
    // The page is the same for the whole wave: its resource lives in SGPRs.
    pid = __builtin_amdgcn_readfirstlane(pid);
    const size_t off =
        pid >= 0 ? (size_t)pid * (size_t)a.page_stride + (size_t)(p & sub_mask) * sub_bytes : 0;
    const int nrec = pid >= 0 ? (int)a.page_extent : 0;
    const __amdgpu_buffer_rsrc_t kr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)((const char*)a.k + off), (short)0, nrec, kBufferFlags);
    const __amdgpu_buffer_rsrc_t vr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)((const char*)a.v + off), (short)0, nrec, kBufferFlags);
    KV::load(pg[0], kr, vr, k_lane, v_lane, tok_bytes);
    if constexpr (HPW == 2) KV::load(pg[HPW - 1], kr, vr, k_lane + head1, v_lane + head1, tok_bytes);
  };
  // Ring of D pages in flight: page i is processed from slot i % D, which is
  // then refilled with page i + D.
  typename KV::Regs ring[D][HPW];
#pragma unroll
  for (int j = 0; j < D; ++j) {
    load_page(j < n_pages ? clamp_page(first_id[j], a.num_pages) : -1, p_begin + j, ring[j]);
  }

  u4* my_q = sm_q + wave * NB * KK * 64;
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) my_q[(nb * KK + kk) * 64 + lane] = qreg[nb][kk];
  }
#pragma unroll
  for (int k = 0; k < kIdSlots; ++k) {
    const int i = tid + k * WW * 64;
    sm_ids[i] = idreg[k] >= 0 ? clamp_page(idreg[k], a.num_pages) : -1;
  }
  auto page_id = [&](int i) -> int { return active ? sm_ids[i] : -1; };
  // Pages holding a token >= mask_from (draft block or past the end) are masked.
  const int mask_from = len - a.q_len;

  WaveState<NB, HD> st;
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    st.m[nb] = -INFINITY;
    st.l[nb] = 0.f;
    st.thr[nb] = -INFINITY;
    st.nmu[nb] = -0.f;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) st.acc[mb][nb] = f4{0.f, 0.f, 0.f, 0.f};
  }

  __syncthreads();  // sm_q and sm_ids written

  // With two or four row blocks whose accumulators take at most 64 VGPRs
  // (NB * HD <= 256) the page loop is software-pipelined: the scores of page
  // i + 1 are issued before page i's mask, softmax and PV products, so their
  // MFMAs run under the softmax (16 x 32K keys, head dim 64: q16 177.7 -> 173.8
  // us, e4m3 q8 / q16 117.2 / 168.5 -> 111.6 / 154.2 us; head dim 128 q8 317.5
  // -> 316.1 us; bit-identical results). Page i + 1 must then be resident one
  // step earlier and its scores held alongside: with 128 accumulator VGPRs
  // (head dim 128 at 64 rows) the extra registers spill (e4m3 q16 261 -> 269
  // us), with a ring of 2 the wait is longer (head dim 256: 662 -> 916 us),
  // and at one block there is little softmax to hide (e4m3 head dim 64 q4:
  // -1.5%).
  constexpr bool kPipelined = NB >= 2 && D >= 3 && NB * HD <= 256;
  // fp16 queries over an e4m3 cache at 64 rows and head dim 128 take the
  // pages two at a time (pair_finish).
  constexpr bool kPairSteps = __is_same(E, ElemF16) && KV::kBytes == 1 && HD == 128 &&
                              NB == 4 && HPW == 1 && D % 2 == 0;
  // A piece that fits the ring in one softmax step (below), in the RB
  // instantiations only (the host picks them for plans whose pieces fit the
  // ring: with the step in it, the kernel's page loop for long pieces ran 1-2%
  // slower): 16-bit K/V, whose ring registers the MFMAs read as they are.
  constexpr bool kRingBatch = RB && KV::kBytes == 2 && HD <= 128;
  const bool upper = l16 >= 8;
  int next_pid = page_id(D);
  if constexpr (kPairSteps) {
    // The Q fragments stay in registers for the whole loop (16 x 4 dwords; the
    // ring, scores and accumulators take the 256 arch VGPRs, so they live in
    // AGPRs, which the MFMAs read directly). Left to itself the compiler
    // copied every fragment to a second set of AGPRs before each pair (104
    // v_accvgpr_mov per 4 pages); the empty asm below states that the values
    // sit in AGPRs at that point, and the copies are gone (cfg3 shape q16:
    // 217.8 -> 209.6 us).
    u4 qf[NB][KK];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) qf[nb][kk] = my_q[(nb * KK + kk) * 64 + lane];
    for (int i = 0; i < n_pages; i += D) {
#pragma unroll
      for (int j = 0; j < D; j += 2) {
        const int ii = i + j;
        if (ii < n_pages) {
          const int p = p_begin + ii;
          const bool masked = (p + 2) * kPageSize > mask_from;
#pragma unroll
          for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int kk = 0; kk < KK; ++kk) asm volatile("" : "+a"(qf[nb][kk]));
          f4 s0[NB], s1[NB];
          // One page's scores after the other: one widened K page live at a time
          // (interleaving the two pages' MFMA chains kept both live and spilled
          // registers to AGPRs; cfg3 shape q16 202.9 -> 200.5 us, ragged 114.0 ->
          // 110.3 us).
          {
            const PageK<HD, 1> k0 = widen_k<E, KV, HD, 1>(ring[j]);
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
              s0[nb] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
              for (int kk = 0; kk < KK; ++kk) s0[nb] = E::mma_qk(k0.k[0][kk], qf[nb][kk], s0[nb]);
            }
          }
          {
            const PageK<HD, 1> k1 = widen_k<E, KV, HD, 1>(ring[j + 1]);
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
              s1[nb] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
              for (int kk = 0; kk < KK; ++kk) s1[nb] = E::mma_qk(k1.k[0][kk], qf[nb][kk], s1[nb]);
            }
          }
          pair_finish<NB>(st, s0, s1, ring[j][0], ring[j + 1][0], ii + 1 < n_pages, dbits,
                          mask_from, p * kPageSize + 4 * g16, len, masked, a.scale_log2);
        }
        const int pid0 = next_pid;
        const int pid1 = page_id(ii + D + 1);
        next_pid = page_id(ii + D + 2);
        load_page(pid0, p_begin + ii + D, ring[j]);
        load_page(pid1, p_begin + ii + D + 1, ring[j + 1]);
      }
    }
  } else if (kRingBatch && n_pages <= D) {  // uniform: the whole piece is in the ring
    // Short pieces (one sequence of 8K keys in 4-page splits, every piece of a
    // 1K-key sequence): the ring's pages arrive together, so they are taken in
    // one softmax step, all scores first, one running-max update, then the PV
    // products, instead of D dependent page steps (the MFMAs of all pages
    // issue back to back; one sequence of 8K keys, whole calls: q_len 2 14.1
    // -> 13.7 us, q_len 4 14.8 -> 14.2 us). Zero pages past the piece take no
    // part.
    f4 sb[D][NB];
    PageV<HD, HPW> pvb[D];
#pragma unroll
    for (int j = 0; j < D; ++j) {
      page_scores<NB, HD, E, KV, HPW>(sb[j], widen_k<E, KV, HD, HPW>(ring[j]), my_q, lane, upper);
      pvb[j] = widen_v<E, KV, HD, HPW>(ring[j]);
    }
    float lm[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) lm[nb] = -INFINITY;
#pragma unroll
    for (int j = 0; j < D; ++j) {
      const int p = p_begin + j;
      if (j >= n_pages) {  // uniform
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) sb[j][nb] = f4{-INFINITY, -INFINITY, -INFINITY, -INFINITY};
      } else if ((p + 1) * kPageSize > mask_from) {  // uniform
        mask_page<NB, HD, HPW>(sb[j], pvb[j], dbits, mask_from, p * kPageSize + 4 * g16, len);
      }
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) lm[nb] = fmaxf(lm[nb], max4(sb[j][nb]) * a.scale_log2);
    }
    raise_max<NB, HD>(st, lm);
#pragma unroll
    for (int j = 0; j < D; ++j)
      if (j < n_pages) page_pv<NB, HD, E, KV, HPW>(st, sb[j], pvb[j], upper, a.scale_log2);
  } else {
  f4 s_cur[NB];
  if constexpr (kPipelined)
    page_scores<NB, HD, E, KV, HPW>(s_cur, widen_k<E, KV, HD, HPW>(ring[0]), my_q, lane, upper);
  // 64 rows over e4m3 outside the page pairs (bf16 queries), and head dim 256:
  // the Q fragments held in AGPRs for the loop, pinned there as in the pair
  // loop (the compiler had copied them between AGPR sets every page; cfg3
  // shape: bf16 / e4m3 q16 283.7 -> 271.0 us, head dim 256 q8 680.5 -> 668.7
  // us, e4m3 324.2 -> 322.2 us).
  constexpr bool kQRegs =
      ((NB == 4 && KV::kBytes == 1) || HD == 256) && HPW == 1 && !kPipelined;
  u4 qf[kQRegs ? NB : 1][KK];
  if constexpr (kQRegs) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) qf[nb][kk] = my_q[(nb * KK + kk) * 64 + lane];
  }
  for (int i = 0; i < n_pages; i += D) {
#pragma unroll
    for (int j = 0; j < D; ++j) {
      const int ii = i + j;
      if (ii < n_pages) {
        const int p = p_begin + ii;
        const bool masked = (p + 1) * kPageSize > mask_from;
        if constexpr (kPipelined) {
          // Slot (j + 1) % D holds page ii + 1 (a zero page past the split).
          f4 s_next[NB];
          page_scores<NB, HD, E, KV, HPW>(s_next, widen_k<E, KV, HD, HPW>(ring[(j + 1) % D]),
                                          my_q, lane, upper);
          PageV<HD, HPW> pv = widen_v<E, KV, HD, HPW>(ring[j]);
          page_finish<NB, HD, E, KV, HPW>(st, s_cur, pv, upper, dbits, mask_from,
                                          p * kPageSize + 4 * g16, len, masked, a.scale_log2);
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) s_cur[nb] = s_next[nb];
        } else {
          // K and V widened together, then the scores (the order that schedules
          // best where no pipelining is done).
          const PageK<HD, HPW> kf = widen_k<E, KV, HD, HPW>(ring[j]);
          PageV<HD, HPW> pv = widen_v<E, KV, HD, HPW>(ring[j]);
          if constexpr (kQRegs) {
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
              for (int kk = 0; kk < KK; ++kk) asm volatile("" : "+a"(qf[nb][kk]));
              s_cur[nb] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
              for (int kk = 0; kk < KK; ++kk)
                s_cur[nb] = E::mma_qk(kf.k[0][kk], qf[nb][kk], s_cur[nb]);
            }
          } else {
            page_scores<NB, HD, E, KV, HPW>(s_cur, kf, my_q, lane, upper);
          }
          page_finish<NB, HD, E, KV, HPW>(st, s_cur, pv, upper, dbits, mask_from,
                                          p * kPageSize + 4 * g16, len, masked, a.scale_log2);
        }
      }
      const int pid = next_pid;
      next_pid = page_id(ii + D + 1);
      load_page(pid, p_begin + ii + D, ring[j]);
    }
  }
  }
  if (active)
    write_results<NB, HD, E>(a, st, sm_stage + wave * 16 * (HD + 4), map, direct,
                             !single && !balanced, b, slot + slot_base, slot_heads, head0);
  });
}

// The rows of one wave of the 8-wave kernel: rows base .. base + 31 of kv head
// kvh (two 16-row blocks).
struct HalfRows {
  int kvh, rows, hkv, base;
  __device__ __forceinline__ int head(int, int) const { return kvh; }
  __device__ __forceinline__ int row(int nb, int r) const { return base + 16 * nb + r; }
  __device__ __forceinline__ bool real(int nb, int r) const {
    return kvh < hkv && row(nb, r) < rows;
  }
};

// s_waitcnt vmcnt(n) with the other counters left alone (gfx9 encoding: vmcnt in
// bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt holds 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// One 16-byte non-temporal buffer load per lane straight into LDS (gfx950
// buffer_load_dwordx4 ... lds): lane l's 16 bytes land at LDS byte address
// lds + 16 l. Written as inline asm on purpose: the compiler's own wait-count
// pass, seeing such a load, waits for all vector memory (vmcnt(0)) before every
// later LDS read that might alias it, which would drain a ring of these loads at
// each step; the callers place their vmcnt waits themselves and issue no other
// vector-memory loads meanwhile. m0 (the LDS base of the load) is saved and
// restored around it.
__device__ __forceinline__ void load_to_lds(__amdgpu_buffer_rsrc_t rsrc, unsigned voffset,
                                            unsigned lds) {
  unsigned saved;
  asm volatile(
      "s_mov_b32 %[saved], m0\n\t"
      "s_mov_b32 m0, %[lds]\n\t"
      "buffer_load_dwordx4 %[off], %[rsrc], 0 offen nt lds\n\t"
      "s_mov_b32 m0, %[saved]"
      : [saved] "=&s"(saved)
      : [lds] "s"(lds), [off] "v"(voffset), [rsrc] "s"(rsrc)
      : "memory");
}

// LDS layout of one head's page slice (16 tokens x HD elements of the cache's
// type) for the 8-wave kernel, and the reads that turn it into the register
// form KV::load gives the main kernel (KV::Regs), so the math is shared.
// 16-bit caches: 16 chunks of 16 bytes per token; chunk c of token t sits at
// position 16 t + (c ^ t), so the 16 tokens an MFMA operand read takes at one
// chunk fall in 16 different bank groups.
template <typename KV>
struct LdsSlice;

template <>
struct LdsSlice<KvNative<128>> {
  static constexpr int kChunks = 16;  // 16-byte chunks per token row (256 bytes)
  __device__ __forceinline__ static int pos(int t, int c) { return 16 * t + (c ^ t); }
  __device__ __forceinline__ static int token_of(int p) { return p >> 4; }
  __device__ __forceinline__ static int chunk_of(int p) { return (p & 15) ^ (p >> 4); }
  // K fragment kk of lane (g, l16): token l16, dims 32 kk + 8 g (chunk 4 kk + g);
  // V: tokens 4 g + e, dims 8 l16 .. + 7 (chunk l16).
  __device__ __forceinline__ static void read(KvNative<128>::Regs& r, const char* ks,
                                              const char* vs, int g, int l16) {
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) r.k[kk] = *(const u4*)(ks + 16 * pos(l16, 4 * kk + g));
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const u4 x = *(const u4*)(vs + 16 * pos(4 * g + e, l16));
#pragma unroll
      for (int w = 0; w < 4; ++w) r.v[e][w] = x[w];
    }
  }
};

// 33..64 query rows per kv head (q_len 16 at GQA 4) at head dim 128. Eight
// waves per workgroup: two per kv head, each with 32 of the head's rows in two
// 16-row blocks (the 32-row math), so no wave holds the 128 accumulator
// registers of 64 rows, and two waves share each SIMD, one's MFMAs under the
// other's softmax. The two waves of a head read each page once between them:
// the workgroup's K and V of 4 heads (32 KiB a page of 16-bit K and V) arrive
// in a ring of D LDS slots by direct buffer loads
// (load_to_lds: 1 KiB of a head's page slice per wave and load, in the layout of
// LdsSlice), so the bytes in flight take no registers. Per page: wait for this
// thread's loads of the page (manual vmcnt: nothing else in the loop touches
// vector memory), one barrier (the page is in LDS, and every wave has read the
// previous page's slot, which it did before that page's math), read the wave's K
// and V into registers, refill the previous page's slot with the page D - 1
// ahead, then the math: D - 1 pages stay in flight. One barrier a page rather
// than two (read, barrier, refill this page's slot with D in flight) measured
// 0.3% faster for fp16 and 3.8% for bf16 at KV 32K x 16 sequences. Pages past the
// split load through a zero-length resource (zeros, no memory traffic), as in
// sqa_partial_kernel.
template <int D, typename E, typename KV>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(2)))
void sqa_partial_lds_kernel(PartialArgs a) {
  constexpr int HD = 128, NB = 2, KK = Dims<HD>::KK, MB = Dims<HD>::MB;
  using L = LdsSlice<KV>;
  constexpr int kHeadSlice = 16 * L::kChunks * 16;  // one head's K (or V) of a page
  constexpr int kSlot = 2 * 4 * kHeadSlice;         // K and V of 4 heads
  constexpr int kLoads = kSlot / (512 * 16);        // loads per thread and page
  constexpr int kThreads = 512;
  static_assert(HD * KV::kBytes == 16 * L::kChunks, "a token row is kChunks 16-byte chunks");
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);

  // blockIdx.x = item * head_groups + head_group; with paired items (two head
  // groups), 4k + 2 head_group + (item & 1) for item 2k + (item & 1), so both
  // workgroups of an item run on XCDs of the item's parity. wave = half * 4 +
  // head slot.
  const int head_groups = (a.hkv + 3) / 4;
  const bool pairs = a.pair_items != 0;
  const int hgrp = pairs ? (blockIdx.x & 3) >> 1 : blockIdx.x % head_groups;
  const int item = pairs ? (blockIdx.x >> 2) * 2 + (blockIdx.x & 1) : blockIdx.x / head_groups;
  const int hs = wave & 3;
  const int kvh = hgrp * 4 + hs;
  const HalfRows map{kvh, a.rows, a.hkv, 32 * (wave >> 2)};
  // Waves without rows (a head past the last, or no rows past 32) still load
  // and meet the barriers; they skip the math.
  const bool active = kvh < a.hkv && map.base < a.rows;

  const bool balanced = is_balanced(a.pages_per_split);
  const bool single = !balanced && a.num_splits == 1;
  static_assert(D + 1 <= kIdPad, "page-id table padding must cover the ring's look-ahead");
  constexpr int kIdSlots = (kMaxSplitPages + kIdPad + kThreads - 1) / kThreads;
  // The ring and, after a piece's page loop, the waves' output staging.
  __shared__ __attribute__((aligned(16))) char sm_ring[D * kSlot];
  __shared__ int sm_ids[kIdSlots * kThreads];
  // Load i of a thread fills 1 KiB piece ci = 8 i + wave of a slot: K (first
  // half of the pieces) or V, head slot (ci / parts) % 4, part ci % parts of the
  // head's slice; lane l fills position 64 part + l, i.e. chunk
  // L::chunk_of(position) of token L::token_of(position).
  constexpr int kParts = kHeadSlice / 1024;  // 1 KiB pieces per head slice
  const unsigned tok_bytes = a.token_stride;
  unsigned voff[kLoads];
#pragma unroll
  for (int i = 0; i < kLoads; ++i) {
    const int ci = 8 * i + wave;
    const int pos = 64 * (ci % kParts) + (threadIdx.x & 63);
    voff[i] = L::token_of(pos) * tok_bytes + (hgrp * 4 + (ci / kParts) % 4) * a.head_stride +
              16 * L::chunk_of(pos);
  }

  // Paired items: the page loop's time (100 MHz counter) and pages, for the
  // merge kernel's choice of the next call's item sizes under adaptive pairs
  // (zero if the item has no piece).
  float loop_ticks = 0.f;
  int loop_pages = 0;
  const bool paired_call =
      for_each_piece<D>(a, plan_view(a), item, [&](const ItemRange& it, const int (&first_id)[D]) {
  const int tid = piece_tid();
  const int lane = tid & 63;
  const int g16 = lane >> 4;
  const int l16 = lane & 15;
  const int b = max(it.b, 0);
  const int len = it.len;
  const int p_begin = it.p_begin;
  const int p_end = it.p_end;
  const int32_t* bt_row = a.block_tables + (size_t)b * a.bt_stride;
  const int shift = a.page_shift;
  const int sub_mask = (1 << shift) - 1;
  if (it.b < 0) return;  // uniform
  const bool direct = it.n_valid <= 1;
  const size_t slot = (size_t)it.slot0 + it.split;
  if (p_begin >= p_end && !single) {  // fixed plan only
    write_empty_split<NB>(a, map, slot, it.n_valid == 1 ? -1.f : 0.f);
    return;  // uniform
  }
  const int n_split = p_end > p_begin ? p_end - p_begin : 0;

  // Q fragments (kept in registers), draft bits, then the split's page ids.
  u4 qreg[NB][KK];
  unsigned long long dbits[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int r = map.row(nb, l16);
    const bool real = map.real(nb, l16);
    const int qi = real ? r / a.group : 0;
    const int gg = real ? r - qi * a.group : 0;
    const int hh = real ? kvh * a.group + gg : 0;
    const _Float16* qp = a.q + ((size_t)(b * a.q_len + qi) * a.hq + hh) * HD;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      const u4 x = *(const u4*)(qp + KV::q_dims(kk, g16));
      qreg[nb][kk] = real ? x : u4{0u, 0u, 0u, 0u};
    }
    dbits[nb] = draft_bits(a, b, qi, real);
  }
  int idreg[kIdSlots];
  const int last_id = n_split > 0 ? n_split - 1 : 0;
#pragma unroll
  for (int k = 0; k < kIdSlots; ++k) {
    const int i = tid + k * kThreads;
    const int x = bt_row[(p_begin + min(i, last_id)) >> shift];
    idreg[k] = i < n_split ? x : -1;
  }

  const size_t sub_bytes = (size_t)kPageSize * tok_bytes;
  auto issue_page = [&](int pid, int p, int j) {
    // The page is the same for the whole workgroup: its resource lives in SGPRs.
    pid = __builtin_amdgcn_readfirstlane(pid);
    const size_t off =
        pid >= 0 ? (size_t)pid * (size_t)a.page_stride + (size_t)(p & sub_mask) * sub_bytes : 0;
    const int nrec = pid >= 0 ? (int)a.page_extent : 0;
    const __amdgpu_buffer_rsrc_t kr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)((const char*)a.k + off), (short)0, nrec, kBufferFlags);
    const __amdgpu_buffer_rsrc_t vr = __builtin_amdgcn_make_buffer_rsrc(
        (void*)((const char*)a.v + off), (short)0, nrec, kBufferFlags);
#pragma unroll
    for (int i = 0; i < kLoads; ++i)
      load_to_lds(i < kLoads / 2 ? kr : vr, voff[i],
                  (unsigned)(size_t)(sm_ring + j * kSlot + (8 * i + wave) * 1024));
  };
#pragma unroll
  for (int j = 0; j < D - 1; ++j)
    issue_page(j < n_split ? clamp_page(first_id[j], a.num_pages) : -1, p_begin + j, j);
#pragma unroll
  for (int k = 0; k < kIdSlots; ++k) {
    const int i = tid + k * kThreads;
    sm_ids[i] = idreg[k] >= 0 ? clamp_page(idreg[k], a.num_pages) : -1;
  }
  const int mask_from = len - a.q_len;

  WaveState<NB, HD> st;
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    st.m[nb] = -INFINITY;
    st.l[nb] = 0.f;
    st.thr[nb] = -INFINITY;
    st.nmu[nb] = -0.f;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) st.acc[mb][nb] = f4{0.f, 0.f, 0.f, 0.f};
  }
  __syncthreads();  // sm_ids written

  const unsigned long long t_loop = it.paired ? __builtin_amdgcn_s_memrealtime() : 0;
  int next_pid = sm_ids[D - 1];
  for (int i = 0; i < n_split; i += D) {
#pragma unroll
    for (int j = 0; j < D; ++j) {
      const int ii = i + j;
      if (ii < n_split) {  // uniform over the workgroup
        wait_vmcnt<kLoads * (D - 2)>();  // this thread's loads of page ii
        __syncthreads();  // page ii is in slot j; every wave is done with page ii - 1
        const char* ks = sm_ring + j * kSlot + hs * kHeadSlice;
        typename KV::Regs raw[1];
        L::read(raw[0], ks, ks + 4 * kHeadSlice, g16, l16);
        const int pid = next_pid;
        next_pid = sm_ids[ii + D];
        issue_page(pid, p_begin + ii + D - 1, (j + D - 1) % D);
        if (active) {
          const int p = p_begin + ii;
          const bool masked = (p + 1) * kPageSize > mask_from;
          const PageK<HD, 1> kf = widen_k<E, KV, HD, 1>(raw);
          PageV<HD, 1> pv = widen_v<E, KV, HD, 1>(raw);
          f4 sc[NB];
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) {
            sc[nb] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kk = 0; kk < KK; ++kk) sc[nb] = E::mma_qk(kf.k[0][kk], qreg[nb][kk], sc[nb]);
          }
          page_finish<NB, HD, E, KV, 1>(st, sc, pv, false, dbits, mask_from,
                                        p * kPageSize + 4 * g16, len, masked, a.scale_log2);
        }
      }
    }
  }
  if (it.paired) {
    loop_ticks = (float)(__builtin_amdgcn_s_memrealtime() - t_loop);
    loop_pages = n_split;
  }
  // Loads past the piece still write (zeros) into the ring: drain them before
  // the ring becomes the output staging.
  wait_vmcnt<0>();
  __syncthreads();
  if (active)
    write_results<NB, HD, E>(a, st, (float*)sm_ring + wave * 16 * (HD + 4), map, direct,
                             !single && !balanced, b, slot, a.hkv, 0);
  });
  // An adaptive paired call (the same answer in every workgroup) leaves a record
  // from every workgroup. Whenever adaptive pairing was asked for, workgroup 0
  // stamps the call (or clears the stamp when the lengths made it fall back):
  // the merge kernel reads the records only under a stamp of this call.
  if (a.pair_items == kPairsAdaptive && threadIdx.x == 0) {
    if (paired_call)
      *(int2*)(a.tune + 4 + 2 * blockIdx.x) =
          int2{__float_as_int(loop_ticks), loop_pages | (item & 1) << 30 | 1 << 31};
    if (blockIdx.x == 0) a.tune[2] = paired_call ? __uint_as_float(kTuneStamp) : 0.f;
  }
}

// Log-sum-exp merge of split partials (reference: csrc/small_q_attention_ext.cu:339-366):
// M = max_s m_s; O = sum_s acc_s 2^(m_s - M) / sum_s l_s 2^(m_s - M); splits
// with l_s <= 0 are skipped and a row with no visible key is written as 0.
// fp16 partials hold acc_s / l_s (so acc_s = l_s times the stored row).
//
// One pass, every load of a round in flight at once: WPR waves serve one
// output row; each thread owns the 16 bytes of a partial row at dims DPT c ..
// DPT c + DPT - 1 (DPT = 8 fp16 or 4 fp32 values) and the splits g, g + SG, ...
// of its split group g, U splits per round (one round wherever the row's
// splits allow: the round trip to the partials, not their bytes, sets the
// time). Each group keeps a running max and rescales its sums when the max
// grows (as the online softmax does), so no pass over the maxima precedes the
// sums; the groups then meet by shuffles within a wave and in LDS across the
// row's waves.
// A (first slot, count) entry held to the slots that exist, whatever the table
// holds (the partial kernel writes it within them).
__device__ __forceinline__ SeqSplits in_range(SeqSplits t, int num_splits) {
  t.first = min(max(t.first, 0), num_splits - 1);
  t.count = min(max(t.count, 0), num_splits - t.first);
  return t;
}

// Paired items: the next call's delta from this call's page-loop times (one
// workgroup of 256 threads). Even items took P + d pages, odd ones P - d; with
// per-page times t_e and t_o the two end together at delta = (t_o - t_e) /
// (t_o + t_e), whatever this call's delta was. The new value moves halfway
// there (one call's times are noisy), within +-kPairDeltaMax. Only after a
// call that ran paired (its stamp in tune[2]); the stamp is cleared with the
// records, so a later call that did not pair (a length that differs) changes
// nothing.
__device__ __noinline__ void update_pair_delta(float* tune, int records) {
  __shared__ float sums[4][4];
  const int t = threadIdx.x;
  if (__float_as_uint(tune[2]) != kTuneStamp) return;  // uniform over the workgroup
  float te = 0.f, pe = 0.f, to = 0.f, po = 0.f;
  for (int i = t; i < records; i += 256) {
    const int2 r = *(const int2*)(tune + 4 + 2 * i);
    if (r.y < 0) {  // recorded by this call's partial kernel
      const float pages = (float)(r.y & 0x3fffffff);
      const float ticks = __int_as_float(r.x);
      if ((r.y >> 30) & 1) {
        to += ticks;
        po += pages;
      } else {
        te += ticks;
        pe += pages;
      }
    }
  }
  for (int o = 32; o >= 1; o >>= 1) {
    te += __shfl_xor(te, o);
    pe += __shfl_xor(pe, o);
    to += __shfl_xor(to, o);
    po += __shfl_xor(po, o);
  }
  if ((t & 63) == 0) {
    sums[t >> 6][0] = te;
    sums[t >> 6][1] = pe;
    sums[t >> 6][2] = to;
    sums[t >> 6][3] = po;
  }
  __syncthreads();
  if (t == 0) {
    te = sums[0][0] + sums[1][0] + sums[2][0] + sums[3][0];
    pe = sums[0][1] + sums[1][1] + sums[2][1] + sums[3][1];
    to = sums[0][2] + sums[1][2] + sums[2][2] + sums[3][2];
    po = sums[0][3] + sums[1][3] + sums[2][3] + sums[3][3];
    if (pe > 0.f && po > 0.f && te > 0.f && to > 0.f) {
      const float ue = te / pe, uo = to / po;
      const float target = (uo - ue) / (uo + ue);
      float old = __float_as_uint(tune[0]) == kTuneMagic ? tune[1] : 0.f;
      old = old == old ? fminf(fmaxf(old, -kPairDeltaMax), kPairDeltaMax) : 0.f;
      tune[1] = fminf(fmaxf(0.5f * (old + target), -kPairDeltaMax), kPairDeltaMax);
      tune[0] = __uint_as_float(kTuneMagic);
    }
  }
  // Records and stamp are marked as read: a later call that writes none changes
  // nothing.
  for (int i = t; i < records; i += 256) tune[4 + 2 * i + 1] = 0.f;
  if (t == 0) tune[2] = 0.f;
}

template <int WPR, int HD, typename E, int U>
__global__ __launch_bounds__(256) void sqa_merge_kernel(MergeArgs a) {
  // Each thread owns DPT dims of the row, 16 bytes of every partial row (fp16
  // partials: 8 dims; fp32: 4), and the splits g, g + SG, ... of its split
  // group g; a row's WPR waves cover SG = 64 WPR / CH splits per load
  // instruction and U SG splits per round.
  constexpr int DPT = E::kHalfPartials ? 8 : 4;
  constexpr int CH = HD / DPT;      // threads per partial row
  constexpr int TPR = 64 * WPR;     // threads per output row
  constexpr int SG = TPR / CH;      // split groups of a row
  constexpr int RPW = 256 / TPR;    // rows per workgroup
  static_assert(SG >= 1 && TPR % CH == 0 && 256 % TPR == 0, "a row's threads must cover its dims");
  const int t = threadIdx.x;
  const int tr = t % TPR;
  const int c = tr % CH;
  const int g = tr / CH;
  const int row = blockIdx.x * RPW + t / TPR;
  const int total = a.batch * a.q_len * a.hq;
  const bool live = row < total;  // uniform per row
  if (a.tune != nullptr && blockIdx.x == 0) update_pair_delta(a.tune, a.tune_records);
  const int rowc = live ? row : 0;
  const int h = rowc % a.hq;
  const int qi = (rowc / a.hq) % a.q_len;
  const int b = rowc / (a.hq * a.q_len);
  const int kvh = h / a.group;
  const int r = qi * a.group + (h - kvh * a.group);

  // Where the row's splits are. Fixed plan: all num_splits slots of the
  // sequence, no length needed (splits past its pages hold l = 0, and l = -1
  // in split 0 says the partial kernel already wrote the row). Balanced plan:
  // the (first slot, count) table the partial kernel wrote; when every
  // sequence was expected to span spec_pages pages, the layout of that case
  // (sequence b's pages from b * spec_pages on, items of spec_pps pages) is
  // assumed while the table is read, and the row is merged again from the
  // table if the two differ.
  const bool balanced = is_balanced(a.pages_per_split);
  const bool expect = balanced && a.spec_pages > 0;
  // With items per head group (hg_items) the row's head group has its own
  // region of slots (four kv heads each), table, slot count and item size.
  const bool hg_split = a.hg_items[0] > 0;
  const int grp = kvh >> 2;
  const int num_splits = hg_split ? a.hg_items[grp] + a.batch : a.num_splits;
  const SeqSplits* seq_splits = a.seq_splits + (hg_split ? grp * a.batch : 0);
  const int spec_pps = hg_split && grp ? a.hg_spec_pps1 : a.spec_pps;
  // items between consecutive splits of this row, and the row's item in split 0
  const size_t stride = (size_t)(hg_split ? 4 : a.hkv) * a.rows;
  const size_t row_item =
      hg_split ? ((size_t)(grp ? a.hg_items[0] + a.batch : 0) * 4 + (kvh & 3)) * a.rows + r
               : (size_t)kvh * a.rows + r;
  int n_valid, slot0;
  SeqSplits table = {0, 0};
  if (expect) {
    const int start = b * a.spec_pages;
    const int i0 = start / spec_pps;
    n_valid = (start + a.spec_pages - 1) / spec_pps - i0 + 1;
    slot0 = i0 + b;
  } else if (balanced) {
    table = in_range(seq_splits[b], num_splits);
    n_valid = table.count;
    slot0 = table.first;
  } else {
    n_valid = a.num_splits;
    slot0 = b * a.num_splits;
  }
  if (!live) n_valid = 0;

  float mt = -INFINITY, den = 0.f;
  float acc[DPT];
  u4 o[U];
  float m[U], l[U];
  // One round: splits sb + u * SG (u < U) of the slots [s0, s0 + nv). Loads are
  // unconditional, from an in-bounds slot (past the last split: split 0 of the
  // row again, weight 0), so rounds need no branch around their loads.
  auto load_round = [&](int s0, int nv, int sb) {
    const float* ml = a.part_ml + ((size_t)s0 * stride + row_item) * 2;
    const size_t o0 = ((size_t)s0 * stride + row_item) * HD + DPT * c;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int sp = sb + u * SG;
      const size_t it = (size_t)(sp < nv ? sp : 0) * stride;
      if constexpr (E::kHalfPartials)
        o[u] = *(const u4*)((const _Float16*)a.part_o + o0 + it * HD);
      else
        o[u] = *(const u4*)(a.part_o + o0 + it * HD);
      const float2 p = *(const float2*)(ml + it * 2);  // (max, sum) in one load
      m[u] = p.x;
      l[u] = sp < nv ? p.y : 0.f;
    }
  };
  auto add_round = [&]() {
    float cm = -INFINITY;
#pragma unroll
    for (int u = 0; u < U; ++u) cm = !(l[u] <= 0.f) ? fmaxf(cm, m[u]) : cm;
    const float nm = fmaxf(mt, cm);
    if (nm != -INFINITY) {
      const float sc = mt == -INFINITY ? 0.f : fast_exp2(mt - nm);
      den *= sc;
#pragma unroll
      for (int i = 0; i < DPT; ++i) acc[i] *= sc;
#pragma unroll
      for (int u = 0; u < U; ++u) {
        // Splits without keys (l <= 0) never touch the sums: their partial sums
        // were never written and may hold anything. A NaN sum (the split saw a
        // NaN) is used, so the row comes out NaN.
        const bool use = !(l[u] <= 0.f);
        const float w = use ? fast_exp2(m[u] - nm) : 0.f;
        den += w * l[u];
        // Normalised partials weigh in with their sum.
        const float wo = E::kHalfPartials ? w * l[u] : w;
        float x[DPT];
        if constexpr (E::kHalfPartials) {
          const h8 v = __builtin_bit_cast(h8, o[u]);
#pragma unroll
          for (int i = 0; i < 8; ++i) x[i] = (float)v[i];
        } else {
          const f4 v = __builtin_bit_cast(f4, o[u]);
#pragma unroll
          for (int i = 0; i < 4; ++i) x[i] = v[i];
        }
#pragma unroll
        for (int i = 0; i < DPT; ++i) acc[i] = use ? fmaf(wo, x[i], acc[i]) : acc[i];
      }
      mt = nm;
    }
  };
  // The first round is issued before anything else is waited for (the
  // expected layout's table read rides along with it); later rounds, rare, loop.
  auto merge_splits = [&](int s0, int nv) {
    mt = -INFINITY;
    den = 0.f;
#pragma unroll
    for (int i = 0; i < DPT; ++i) acc[i] = 0.f;
    load_round(s0, nv, g);
    if (expect) table = in_range(seq_splits[b], num_splits);
    const float first_l = l[0];  // split g (split 0 for group 0)
    add_round();
    for (int sb = g + U * SG; sb < nv; sb += U * SG) {
      load_round(s0, nv, sb);
      add_round();
    }
    return first_l;
  };
  float first_l = merge_splits(slot0, n_valid);
  if (expect && live && (table.first != slot0 || table.count != n_valid)) {
    n_valid = table.count;
    slot0 = table.first;
    first_l = merge_splits(slot0, n_valid);
  }
  // A sequence with one split was written by the partial kernel: the balanced
  // plan says so by its count, a fixed plan by l = -1 in split 0, which group 0
  // (the one that stores) reads first. A sequence with no splits (no keys at
  // all) is written here as 0.
  const bool done = balanced ? n_valid == 1 : (g == 0 && first_l < 0.f);
  const bool skip = !live || done;

  // Combine the SG groups of the row: within a wave by shuffles (lanes c,
  // c + CH, ...), then the row's waves through LDS.
  auto combine = [&](float mo, float dn, const float (&ao)[DPT]) {
    const float nm = fmaxf(mt, mo);
    if (nm == -INFINITY) return;
    const float sa = mt == -INFINITY ? 0.f : fast_exp2(mt - nm);
    const float so = mo == -INFINITY ? 0.f : fast_exp2(mo - nm);
    den = den * sa + dn * so;
#pragma unroll
    for (int i = 0; i < DPT; ++i) acc[i] = acc[i] * sa + ao[i] * so;
    mt = nm;
  };
#pragma unroll
  for (int off = CH; off < 64; off <<= 1) {
    const float mo = __shfl_xor(mt, off), dn = __shfl_xor(den, off);
    float ao[DPT];
#pragma unroll
    for (int i = 0; i < DPT; ++i) ao[i] = __shfl_xor(acc[i], off);
    combine(mo, dn, ao);
  }
  if constexpr (WPR > 1) {
    static_assert(RPW == 1, "the LDS combine serves one row per workgroup");
    __shared__ float sm_acc[WPR][CH][DPT + 1];
    __shared__ float sm_m[WPR][CH], sm_d[WPR][CH];
    if (!live || (balanced && n_valid == 1)) return;  // uniform over the workgroup (one row)
    const int wave = t >> 6;
    if ((t & 63) < CH) {
#pragma unroll
      for (int i = 0; i < DPT; ++i) sm_acc[wave][c][i] = acc[i];
      sm_m[wave][c] = mt;
      sm_d[wave][c] = den;
    }
    __syncthreads();
    if (t >= CH) return;
#pragma unroll
    for (int w = 1; w < WPR; ++w) {
      float ao[DPT];
#pragma unroll
      for (int i = 0; i < DPT; ++i) ao[i] = sm_acc[w][c][i];
      combine(sm_m[w][c], sm_d[w][c], ao);
    }
  }
  if (skip || g != 0) return;
  const float inv = !(den <= 0.f) ? a.out_scale / den : 0.f;  // 0: no key; NaN stays NaN
  if constexpr (DPT == 8) {
    // Two 8-byte stores: the output need only be 8-byte aligned.
    const float lo[4] = {acc[0] * inv, acc[1] * inv, acc[2] * inv, acc[3] * inv};
    const float hi[4] = {acc[4] * inv, acc[5] * inv, acc[6] * inv, acc[7] * inv};
    u2* op = (u2*)(a.out + (size_t)row * HD + 8 * c);
    op[0] = E::pack4(lo);
    op[1] = E::pack4(hi);
  } else {
    const float out[4] = {acc[0] * inv, acc[1] * inv, acc[2] * inv, acc[3] * inv};
    *(u2*)(a.out + (size_t)row * HD + 4 * c) = E::pack4(out);
  }
}

// Ring depth: the pages in flight per wave hold about 32 KiB of 16-bit K and
// V: 4 pages at head dim 128 (3 at 64 rows, where the registers run out), 8 at
// head dim 64 (4 at 64 rows: bf16 q16 201.5 -> 194.5 us, fp16 174.5 -> 173.9)
// and 2 at 256, which holds at most 32 rows (its accumulators double). e4m3
// caches keep the same page counts although their pages hold half the bytes,
// and at 64 rows 3 at head dim 64 and, at head dim 128, 2 under bf16 queries
// or 4 under fp16 ones (two page pairs): the widened K and V fragments take
// the registers a deeper ring would need.
// Measured at 16 sequences of 32K keys, partial kernel, e4m3 ring at twice
// these depths -> these: head dim 128 q2 / q8 170.7 / 181.4 -> 169.7 / 174.2
// us, q16 278 (6 pages) -> 261 (3) -> 251 us (2); head dim 256 q8 342.7 ->
// 325.1 us; head dim 64 q4 / q8 / q16 104.2 / 119.8 / 185 -> 100.7 / 116.6 /
// 169 us (2 pages at 64 rows there lose the pipelined loop: 154 -> 165 us).
template <int HD, typename E, typename KV>
void launch_partial_hd(const PartialArgs& a, const LaunchShape& sh, dim3 grid, dim3 block,
                       hipStream_t stream) {
  constexpr int D4 = 4 * 128 / HD, D2 = 2 * 128 / HD;
  static_assert(HD != 128 || D4 == kRingPages, "the host's ring-batch test assumes this ring");
  // e4m3 at head dim 128: 2 pages, or 4 under fp16 queries, whose pair steps
  // (pair_finish) need a second pair in flight while one is computed.
  constexpr int D3 = KV::kBytes == 1 ? (HD == 128 ? (__is_same(E, ElemF16) ? 4 : 2) : 3)
                                     : (HD == 64 ? 4 : 3 * 128 / HD);
  if (sh.hpw == 2) {
    // Two heads per wave: half the pages in flight, each twice the bytes.
    if constexpr (HD == 64) {
      if (sh.row_blocks == 1)
        hipLaunchKernelGGL((sqa_partial_kernel<1, D2, 4, 1, HD, E, KV, 2>), grid, block, 0,
                           stream, a);
      else if (sh.row_blocks == 2)
        hipLaunchKernelGGL((sqa_partial_kernel<2, D2, 4, 1, HD, E, KV, 2>), grid, block, 0,
                           stream, a);
      else
        hipLaunchKernelGGL((sqa_partial_kernel<4, D2, 4, 1, HD, E, KV, 2>), grid, block, 0,
                           stream, a);
    }
  } else if (sh.row_blocks == 1) {
    if constexpr (HD == 128 && KV::kBytes == 2) {
      if (a.ring_batch) {
        hipLaunchKernelGGL((sqa_partial_kernel<1, D4, 4, 1, HD, E, KV, 1, true>), grid, block, 0,
                           stream, a);
        return;
      }
    }
    hipLaunchKernelGGL((sqa_partial_kernel<1, D4, 4, 1, HD, E, KV, 1>), grid, block, 0, stream,
                       a);
  } else if (sh.row_blocks == 2) {
    if constexpr (HD == 128 && KV::kBytes == 2) {
      if (a.ring_batch) {
        hipLaunchKernelGGL((sqa_partial_kernel<2, D4, 4, 1, HD, E, KV, 1, true>), grid, block, 0,
                           stream, a);
        return;
      }
    }
    hipLaunchKernelGGL((sqa_partial_kernel<2, D4, 4, 1, HD, E, KV, 1>), grid, block, 0, stream,
                       a);
  } else if constexpr (HD == 128 && KV::kBytes == 2) {
    // 33..64 rows of 16-bit K and V: two waves per kv head sharing an LDS ring
    // of 128 KiB (4 pages). e4m3 caches take the one-wave-per-head kernel below:
    // it widens each page once per head where two waves would both widen it
    // (cfg3 shape q16: 256.3 -> 246.6 us; B4 KV 8K 34.8 -> 33.6 us).
    hipLaunchKernelGGL((sqa_partial_lds_kernel<4, E, KV>), grid, dim3(512), 0, stream, a);
  } else if constexpr (HD != 256) {
    hipLaunchKernelGGL((sqa_partial_kernel<4, D3, 4, 1, HD, E, KV, 1>), grid, block, 0, stream,
                       a);
  }
}

template <typename E, template <int> class KV>
void launch_partial_as(const PartialArgs& a, const LaunchShape& sh, dim3 grid, dim3 block,
                       hipStream_t stream) {
  if (a.head_dim == 64)
    launch_partial_hd<64, E, KV<64>>(a, sh, grid, block, stream);
  else if (a.head_dim == 256)
    launch_partial_hd<256, E, KV<256>>(a, sh, grid, block, stream);
  else
    launch_partial_hd<128, E, KV<128>>(a, sh, grid, block, stream);
}

template <int HD, typename E, int WPR>
void launch_merge_u(const MergeArgs& a, int u, dim3 grid, hipStream_t stream) {
  if (u <= 2)
    hipLaunchKernelGGL((sqa_merge_kernel<WPR, HD, E, 2>), grid, dim3(256), 0, stream, a);
  else if (u <= 4)
    hipLaunchKernelGGL((sqa_merge_kernel<WPR, HD, E, 4>), grid, dim3(256), 0, stream, a);
  else
    hipLaunchKernelGGL((sqa_merge_kernel<WPR, HD, E, 8>), grid, dim3(256), 0, stream, a);
}

template <int HD, typename E>
void launch_merge_hd(const MergeArgs& a, int per_row, hipStream_t stream) {
  // A row's splits in one round of loads wherever 8 per thread cover them: a
  // wave per row (4 rows per workgroup) for 1024 rows and more, where the
  // chip has rows enough; a workgroup of 4 waves per row below that, or where a
  // wave would need a second round (one sequence, KV 32K, q_len 8: 128 splits
  // per row). Each thread issues U loads of 16 bytes at once, the smallest U of
  // 2, 4, 8 that covers the row (more rounds past 8).
  constexpr int kSplitsPerWave = 64 / (HD / (E::kHalfPartials ? 8 : 4));
  const int total = a.batch * a.q_len * a.hq;
  if (total >= 1024 && per_row <= 8 * kSplitsPerWave) {
    const int u = (per_row + kSplitsPerWave - 1) / kSplitsPerWave;
    launch_merge_u<HD, E, 1>(a, u, dim3((unsigned)((total + 3) / 4)), stream);
  } else {
    const int u = (per_row + 4 * kSplitsPerWave - 1) / (4 * kSplitsPerWave);
    launch_merge_u<HD, E, 4>(a, u, dim3((unsigned)total), stream);
  }
}

template <typename E>
void launch_merge_as(const MergeArgs& a, int per_row, hipStream_t stream) {
  if (a.head_dim == 64)
    launch_merge_hd<64, E>(a, per_row, stream);
  else if (a.head_dim == 256)
    launch_merge_hd<256, E>(a, per_row, stream);
  else
    launch_merge_hd<128, E>(a, per_row, stream);
}

}  // namespace

hipError_t launch_partial(const PartialArgs& a, hipStream_t stream) {
  const LaunchShape sh = launch_shape(a.rows, a.hkv, a.head_dim);
  const int head_groups = (a.hkv + sh.heads - 1) / sh.heads;
  // Work items: fixed plan, one per slot; balanced, num_splits - batch (a
  // sequence's share of the spare slots comes from the item it ends in).
  const long long items = is_balanced(a.pages_per_split)
                              ? (long long)(a.num_splits - a.batch)
                              : (long long)a.batch * a.num_splits;
  const dim3 grid((unsigned)(items * head_groups));
  const dim3 block(sh.waves() * 64);
  if (a.bf16) {
    if (a.kv_fp8)
      launch_partial_as<ElemBF16, KvFp8>(a, sh, grid, block, stream);
    else
      launch_partial_as<ElemBF16, KvNative>(a, sh, grid, block, stream);
  } else {
    if (a.kv_fp8)
      launch_partial_as<ElemF16, KvFp8>(a, sh, grid, block, stream);
    else
      launch_partial_as<ElemF16, KvNative>(a, sh, grid, block, stream);
  }
  return hipGetLastError();
}

hipError_t launch_merge(const MergeArgs& a, hipStream_t stream) {
  // Splits per sequence, for the choice of merge variant: a fixed plan's
  // num_splits; the balanced plan's count per sequence is known only on the
  // device: the batch average, items / batch. It depends on the slot count
  // alone, so the plain balanced plan and the one with an expected page count
  // merge with the same variant (and give the same bits).
  // With items per head group, the larger group's count (a row of the other
  // group then loads a few more splits than it has, as splits past a row's
  // last do).
  const int items = a.hg_items[0] > 0 ? max(a.hg_items[0], a.hg_items[1]) : a.num_splits - a.batch;
  const int per_row = is_balanced(a.pages_per_split) ? (items + a.batch - 1) / a.batch
                                                     : a.num_splits;
  if (a.bf16)
    launch_merge_as<ElemBF16>(a, per_row, stream);
  else
    launch_merge_as<ElemF16>(a, per_row, stream);
  return hipGetLastError();
}

}  // namespace sqa
