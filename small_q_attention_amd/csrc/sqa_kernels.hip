// gfx950 kernels for paged small-q (speculative-decoding "MTP") attention.
//
// Semantics (reference: /root/reference/src/small_q_attention/reference.py:46-72,
// csrc/small_q_attention_ext.cu:37-54): query head h reads kv head h / group;
// draft row qi of sequence b sees tokens t < seq_lens[b] - q_len + qi + 1;
// token t is slot t % 16 of page block_tables[b, t / 16]; scale head_dim^-1/2;
// fp32 softmax; fp16 output.
//
// Work decomposition. One workgroup owns (sequence b, kv head, split) and holds
// every query row that reads that kv head: rows = q_len * group, row
// r = qi * group + g <-> query head kvh * group + g. Each K/V byte is loaded
// from HBM once and used by all rows, straight from registers: the four waves
// of the workgroup take interleaved pages of the split and merge their
// (max, sum, output) states through LDS at the end.
//
// Per 16-token page a wave issues 4 K and 4 V global_load_dwordx4 (1 KiB each).
//   S^T[token][row] = K . Q^T : v_mfma_f32_16x16x32_f16, A = K (lane l: token
//     l%16, 8 consecutive dims), B = Q^T (lane l: row l%16, same dims). The head
//     dimension is contracted in the order d = 32*kk + 8*(l/16) + e, which is
//     the same for A and B, so it needs no data movement.
//   O^T[d][row] += V^T . P^T : v_mfma_f32_16x16x16_f16. The S^T accumulator
//     (lane l: tokens 4*(l/16)+0..3 of row l%16) is exactly the B operand, so
//     P never leaves its registers. Lane l loads V rows 4*(l/16)+0..3, dims
//     8*(l%16)+0..7 (four full 256-byte rows per instruction) and regroups
//     them with one bit-select per half pair: output block mb covers dims
//     d = 8*m + mb, m = 0..15.
// Rows beyond q_len*group (q_len*group not a multiple of 16) carry zero Q and
// are never stored.
#include "sqa_internal.h"

#include <math.h>

namespace sqa {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef _Float16 h4 __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef unsigned u4 __attribute__((ext_vector_type(4)));
typedef unsigned u2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ float xor_max(float x) {
  x = fmaxf(x, __shfl_xor(x, 16));
  return fmaxf(x, __shfl_xor(x, 32));
}

__device__ __forceinline__ float xor_sum(float x) {
  x += __shfl_xor(x, 16);
  return x + __shfl_xor(x, 32);
}

// One page worth of registers: K (4 x 16 B) and V (4 x 16 B) per lane.
struct PageRegs {
  u4 k[4];
  u4 v[4];
};

template <int NB>
struct WaveState {
  f4 acc[8][NB];   // O^T blocks: lane l holds dims 32*(l/16)+8*r+mb of row 16*nb+l%16
  float m[NB];     // running row max (log2 units), identical in the 4 lane groups
  float l[NB];     // partial row sum over this lane's tokens
};

__device__ __forceinline__ int clamp_page(int pid, long long num_pages) {
  return (pid >= 0 && (long long)pid < num_pages) ? pid : 0;
}

template <int NB>
__device__ __forceinline__ void process_page(WaveState<NB>& st, PageRegs& pg, const h8 (&qf)[NB][4],
                                             const int (&vis)[NB], int tok0, int len, bool masked,
                                             float scale_log2) {
  // Scores S^T[token][row] for this page.
  f4 s[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    s[nb] = f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      s[nb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(h8, pg.k[kk]), qf[nb][kk],
                                                    s[nb], 0, 0, 0);
    }
    s[nb] *= scale_log2;
  }
  if (masked) {
    // tok0 = absolute index of this lane's first token (4 consecutive tokens).
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (tok0 + e >= vis[nb]) s[nb][e] = -INFINITY;
      }
    }
    // V rows past the sequence end may hold anything (even NaN); 0 * NaN would
    // poison the product, so zero them.
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      if (tok0 + e >= len) pg.v[e] = u4{0u, 0u, 0u, 0u};
    }
  }

  h4 ph[NB];
  bool rescale = false;
  float alpha[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    float pm = fmaxf(fmaxf(s[nb][0], s[nb][1]), fmaxf(s[nb][2], s[nb][3]));
    pm = xor_max(pm);
    const float mn = fmaxf(st.m[nb], pm);
    const float mu = (mn == -INFINITY) ? 0.f : mn;
    alpha[nb] = fast_exp2(st.m[nb] - mu);
    rescale |= (alpha[nb] != 1.0f);
    st.m[nb] = mn;
    float lsum = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const _Float16 p = (_Float16)fast_exp2(s[nb][e] - mu);
      ph[nb][e] = p;
      lsum += (float)p;
    }
    st.l[nb] = st.l[nb] * alpha[nb] + lsum;
  }
  if (__any(rescale)) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
      for (int mb = 0; mb < 8; ++mb) st.acc[mb][nb] *= alpha[nb];
    }
  }

  // O^T += V^T . P^T, one 16x16x16 MFMA per (dim block, row block).
#pragma unroll
  for (int mb = 0; mb < 8; ++mb) {
    const int j = mb >> 1;
    const unsigned w0 = pg.v[0][j], w1 = pg.v[1][j], w2 = pg.v[2][j], w3 = pg.v[3][j];
    u2 av;
    if ((mb & 1) == 0) {
      av = u2{(w0 & 0xffffu) | (w1 << 16), (w2 & 0xffffu) | (w3 << 16)};
    } else {
      av = u2{(w0 >> 16) | (w1 & 0xffff0000u), (w2 >> 16) | (w3 & 0xffff0000u)};
    }
    const h4 a = __builtin_bit_cast(h4, av);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      st.acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x16f16(a, ph[nb], st.acc[mb][nb], 0, 0, 0);
    }
  }
}

template <int NB, int NW>
__global__ __launch_bounds__(NW * 64) void sqa_partial_kernel(PartialArgs a) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g16 = lane >> 4;
  const int l16 = lane & 15;

  // blockIdx.x = ((b * num_splits + split) * hkv + kvh): the kv heads of one
  // page range are neighbours in dispatch order.
  int wg = blockIdx.x;
  const int kvh = wg % a.hkv;
  wg /= a.hkv;
  const int split = wg % a.num_splits;
  const int b = wg / a.num_splits;

  int len = a.seq_lens[b];
  len = len < 0 ? 0 : len;
  int pages_used = (len + kPageSize - 1) / kPageSize;
  pages_used = pages_used < a.max_pages ? pages_used : a.max_pages;
  const int p_begin = split * a.pages_per_split;
  const int p_end = min(p_begin + a.pages_per_split, pages_used);
  const bool single = a.num_splits == 1;
  if (p_begin >= p_end && !single) return;  // the merge kernel never reads this split

  // Q fragments (B operand of the score MFMA) and per-row visible length.
  h8 qf[NB][4];
  int vis[NB];
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int r = nb * 16 + l16;
    if (r < a.rows) {
      const int qi = r / a.group;
      const int gg = r - qi * a.group;
      const _Float16* qp =
          a.q + ((size_t)(b * a.q_len + qi) * a.hq + kvh * a.group + gg) * kHeadDim + 8 * g16;
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) qf[nb][kk] = *(const h8*)(qp + 32 * kk);
      vis[nb] = len - a.q_len + 1 + qi;
    } else {
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) qf[nb][kk] = h8{0, 0, 0, 0, 0, 0, 0, 0};
      vis[nb] = 0;
    }
  }
  // Pages whose last token index >= mask_from need the causal/tail mask.
  const int mask_from = len - a.q_len + 1;

  WaveState<NB> st;
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    st.m[nb] = -INFINITY;
    st.l[nb] = 0.f;
#pragma unroll
    for (int mb = 0; mb < 8; ++mb) st.acc[mb][nb] = f4{0.f, 0.f, 0.f, 0.f};
  }

  const size_t tok_stride = (size_t)a.hkv * kHeadDim;         // elements between tokens
  const size_t page_stride = (size_t)kPageSize * tok_stride;   // elements between pages
  const size_t k_lane = (size_t)l16 * tok_stride + (size_t)kvh * kHeadDim + 8 * g16;
  const size_t v_lane = (size_t)(4 * g16) * tok_stride + (size_t)kvh * kHeadDim + 8 * l16;
  const int32_t* bt_row = a.block_tables + (size_t)b * a.max_pages;

  auto load_page = [&](int p, PageRegs& pg) {
    const int pid = clamp_page(bt_row[p], a.num_pages);
    const _Float16* kb = a.k + (size_t)pid * page_stride + k_lane;
    const _Float16* vb = a.v + (size_t)pid * page_stride + v_lane;
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) pg.k[kk] = *(const u4*)(kb + 32 * kk);
#pragma unroll
    for (int e = 0; e < 4; ++e) pg.v[e] = *(const u4*)(vb + e * tok_stride);
  };

  int p = p_begin + wave;
  PageRegs cur;
  if (p < p_end) load_page(p, cur);
  for (; p < p_end; p += NW) {
    PageRegs nxt;
    const int pn = p + NW;
    if (pn < p_end) load_page(pn, nxt);
    const bool masked = (p + 1) * kPageSize > mask_from;
    process_page<NB>(st, cur, qf, vis, p * kPageSize + 4 * g16, len, masked, a.scale_log2);
    cur = nxt;
  }

  // Row sums over the four lane groups.
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) st.l[nb] = xor_sum(st.l[nb]);

  float row_m[NB], row_l[NB];
  if constexpr (NW == 1) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      row_m[nb] = st.m[nb];
      row_l[nb] = st.l[nb];
    }
  } else {
    __shared__ float sm_m[NW][NB * 16];
    __shared__ float sm_l[NW][NB * 16];
    __shared__ f4 sm_acc[8 * NB][64];
    if (g16 == 0) {
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        sm_m[wave][nb * 16 + l16] = st.m[nb];
        sm_l[wave][nb * 16 + l16] = st.l[nb];
      }
    }
    __syncthreads();
    float fac[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const int r = nb * 16 + l16;
      float mx = -INFINITY;
#pragma unroll
      for (int w = 0; w < NW; ++w) mx = fmaxf(mx, sm_m[w][r]);
      const float mu = (mx == -INFINITY) ? 0.f : mx;
      float lt = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) lt += sm_l[w][r] * fast_exp2(sm_m[w][r] - mu);
      fac[nb] = fast_exp2(st.m[nb] - mu);
      row_m[nb] = mx;
      row_l[nb] = lt;
    }
    // Deterministic serial sum of the waves' scaled accumulators.
#pragma unroll
    for (int w = NW - 1; w >= 0; --w) {
      if (wave == w) {
#pragma unroll
        for (int mb = 0; mb < 8; ++mb) {
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) {
            f4 x = st.acc[mb][nb] * fac[nb];
            if (w != NW - 1) x += sm_acc[mb * NB + nb][lane];
            if (w == 0) {
              st.acc[mb][nb] = x;
            } else {
              sm_acc[mb * NB + nb][lane] = x;
            }
          }
        }
      }
      if (w > 0) __syncthreads();
    }
    if (wave != 0) return;
  }

  // Wave 0 stores: lane l owns dims 32*g16 + 8*r + mb (r = 0..3, mb = 0..7)
  // of row 16*nb + l16.
#pragma unroll
  for (int nb = 0; nb < NB; ++nb) {
    const int r = nb * 16 + l16;
    if (r >= a.rows) continue;
    const int qi = r / a.group;
    const int gg = r - qi * a.group;
    if (single) {
      const float inv = row_l[nb] > 0.f ? 1.0f / row_l[nb] : 0.f;
      _Float16* op = a.out + ((size_t)(b * a.q_len + qi) * a.hq + kvh * a.group + gg) * kHeadDim + 32 * g16;
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        h8 o;
#pragma unroll
        for (int mb = 0; mb < 8; ++mb) o[mb] = (_Float16)(st.acc[mb][nb][rr] * inv);
        *(h8*)(op + 8 * rr) = o;
      }
    } else {
      const size_t item = ((size_t)(b * a.hkv + kvh) * a.num_splits + split) * a.rows + r;
      float* op = a.part_o + item * kHeadDim + 32 * g16;
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        f4 lo, hi;
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) {
          lo[mb] = st.acc[mb][nb][rr];
          hi[mb] = st.acc[mb + 4][nb][rr];
        }
        *(f4*)(op + 8 * rr) = lo;
        *(f4*)(op + 8 * rr + 4) = hi;
      }
      if (g16 == 0) {
        a.part_ml[item * 2 + 0] = row_m[nb];
        a.part_ml[item * 2 + 1] = row_l[nb];
      }
    }
  }
}

// Log-sum-exp merge of split partials (reference: csrc/small_q_attention_ext.cu:339-366):
// M = max_s m_s; O = sum_s acc_s 2^(m_s - M) / sum_s l_s 2^(m_s - M); splits
// with l_s <= 0 are skipped and a row with no visible key is written as 0.
// 32 lanes per output row, 4 dims each; 8 rows per 256-thread block.
__global__ __launch_bounds__(256) void sqa_merge_kernel(MergeArgs a) {
  const int row = blockIdx.x * 8 + (threadIdx.x >> 5);
  const int total = a.batch * a.q_len * a.hq;
  if (row >= total) return;
  const int d4 = (threadIdx.x & 31) * 4;
  const int h = row % a.hq;
  const int qi = (row / a.hq) % a.q_len;
  const int b = row / (a.hq * a.q_len);
  const int kvh = h / a.group;
  const int r = qi * a.group + (h - kvh * a.group);

  int len = a.seq_lens[b];
  len = len < 0 ? 0 : len;
  int pages_used = (len + kPageSize - 1) / kPageSize;
  pages_used = pages_used < a.max_pages ? pages_used : a.max_pages;
  int n_valid = (pages_used + a.pages_per_split - 1) / a.pages_per_split;
  n_valid = n_valid < a.num_splits ? n_valid : a.num_splits;

  const size_t base = (size_t)(b * a.hkv + kvh) * a.num_splits;
  float mx = -INFINITY;
  for (int s = 0; s < n_valid; ++s) mx = fmaxf(mx, a.part_ml[((base + s) * a.rows + r) * 2]);
  f4 acc = f4{0.f, 0.f, 0.f, 0.f};
  float den = 0.f;
  if (mx != -INFINITY) {
    for (int s = 0; s < n_valid; ++s) {
      const size_t item = (base + s) * a.rows + r;
      const float ls = a.part_ml[item * 2 + 1];
      if (ls <= 0.f) continue;
      const float w = fast_exp2(a.part_ml[item * 2] - mx);
      den += ls * w;
      acc += w * *(const f4*)(a.part_o + item * kHeadDim + d4);
    }
  }
  const float inv = den > 0.f ? 1.0f / den : 0.f;
  h4 o;
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = (_Float16)(acc[i] * inv);
  *(h4*)(a.out + (size_t)row * kHeadDim + d4) = o;
}

}  // namespace

hipError_t launch_partial(const PartialArgs& a, hipStream_t stream) {
  const dim3 grid((unsigned)(a.batch * a.hkv * a.num_splits));
  const dim3 block(kWaves * 64);
  switch (row_blocks(a.rows)) {
    case 1:
      hipLaunchKernelGGL((sqa_partial_kernel<1, kWaves>), grid, block, 0, stream, a);
      break;
    case 2:
      hipLaunchKernelGGL((sqa_partial_kernel<2, kWaves>), grid, block, 0, stream, a);
      break;
    default:
      hipLaunchKernelGGL((sqa_partial_kernel<4, kWaves>), grid, block, 0, stream, a);
      break;
  }
  return hipGetLastError();
}

hipError_t launch_merge(const MergeArgs& a, hipStream_t stream) {
  const int total = a.batch * a.q_len * a.hq;
  const dim3 grid((unsigned)((total + 7) / 8));
  hipLaunchKernelGGL(sqa_merge_kernel, grid, dim3(256), 0, stream, a);
  return hipGetLastError();
}

}  // namespace sqa
