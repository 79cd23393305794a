/*
 * Scalar double-precision brute force of paged small-q (MTP) attention.
 *
 * TEST INFRASTRUCTURE ONLY: loaded by oracle/cbrute.py for tests/ and the
 * bench's CPU baseline; the product library never links it.
 *
 * Mathematics of /root/reference/src/small_q_attention/reference.py:46-72:
 *   scale = D^-1/2 (:46); query head qh reads kv head qh / (Hq/Hkv) (:67);
 *   draft row qi of sequence b sees tokens t < seq_lens[b] - Q + qi + 1 (:63);
 *   token t is slot t % page of physical page block_tables[b, t / page]
 *   (:54-59); out = softmax(q . k * scale) @ v (:68-70).
 * Rows with no visible token are written as 0 (the reference raises for them,
 * reference.py:52-53; the split-KV kernels of the reference write 0,
 * csrc/small_q_attention_ext.cu:365).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

static double g_half_table[65536];
static double g_bf16_table[65536];
static double g_fp8_table[256];
static int g_table_ready = 0;

/* IEEE-754 binary16 bit pattern -> double. */
static double half_bits_to_double(uint16_t h) {
  const int sign = h >> 15;
  const int expo = (h >> 10) & 31;
  const int mant = h & 1023;
  double v;
  if (expo == 0) {
    v = ldexp((double)mant, -24);
  } else if (expo == 31) {
    v = mant ? NAN : INFINITY;
  } else {
    v = ldexp((double)(mant | 1024), expo - 25);
  }
  return sign ? -v : v;
}

/* bfloat16 bit pattern -> double: the top half of an IEEE-754 binary32. */
static double bf16_bits_to_double(uint16_t h) {
  const uint32_t w = (uint32_t)h << 16;
  float f;
  memcpy(&f, &w, sizeof(f));
  return (double)f;
}

/* OCP FP8 E4M3 ("e4m3fn") byte -> double: 1 sign, 4 exponent (bias 7) and 3
 * mantissa bits, subnormals at exponent 0, NaN at S.1111.111, no infinities. */
static double fp8_e4m3_to_double(uint8_t h) {
  const int sign = h >> 7;
  const int expo = (h >> 3) & 15;
  const int mant = h & 7;
  double v;
  if (expo == 15 && mant == 7) {
    v = NAN;
  } else if (expo == 0) {
    v = ldexp((double)mant, -9);
  } else {
    v = ldexp((double)(mant | 8), expo - 10);
  }
  return sign ? -v : v;
}

static void build_table(void) {
  if (g_table_ready) return;
  for (int i = 0; i < 65536; ++i) {
    g_half_table[i] = half_bits_to_double((uint16_t)i);
    g_bf16_table[i] = bf16_bits_to_double((uint16_t)i);
  }
  for (int i = 0; i < 256; ++i) g_fp8_table[i] = fp8_e4m3_to_double((uint8_t)i);
  g_table_ready = 1;
}

/* Element e of a K/V array of type kv_elem (0 binary16, 1 bfloat16, 2 e4m3). */
static inline double kv_value(const void* base, long long e, int kv_elem) {
  if (kv_elem == 2) return g_fp8_table[((const uint8_t*)base)[e]];
  const uint16_t bits = ((const uint16_t*)base)[e];
  return kv_elem == 1 ? g_bf16_table[bits] : g_half_table[bits];
}

double sqa_oracle_half_to_double(uint16_t bits) { return half_bits_to_double(bits); }
double sqa_oracle_bf16_to_double(uint16_t bits) { return bf16_bits_to_double(bits); }
double sqa_oracle_fp8_to_double(uint8_t bits) { return fp8_e4m3_to_double(bits); }

/*
 * q:  [B, Q, Hq, D] fp16 bits;  out: [B, Q, Hq, D] double;  bt: [B, max_pages]
 * int32;  sl: [B] int32.  K/V element d of kv head h at slot t of page p is
 * kc[p * ps + t * ts + h * hs + d] (V alike from vc; strides in elements).
 * mask: NULL (row qi sees tokens t < sl - Q + qi + 1, the reference's causal
 * draft chain, reference.py:63) or [B, Q, mask_words] uint32 words: row qi
 * sees t < sl - Q, and draft token j = t - (sl - Q) (t < sl) when bit j % 32 of
 * word j / 32 is set. Logits are scaled by `scale`, outputs by `out_scale`.
 * q holds binary16 (bf16 == 0) or bfloat16 (bf16 != 0) bit patterns; kc, vc
 * hold elements of kv_elem (0 binary16, 1 bfloat16, 2 OCP e4m3 bytes), the
 * strides counting elements.
 * Rows that see no token are 0.
 * Returns 0, or -1 if a page id read by the computation lies outside
 * [0, num_pages), or -2 if a sequence needs more than max_pages pages.
 */
int sqa_oracle_f64_ex(const uint16_t* q, const void* kc, const void* vc,
                      long long ps, long long ts, long long hs,
                      const int32_t* bt, const int32_t* sl, const uint32_t* mask, int mask_words,
                      double scale, double out_scale, int bf16, int kv_elem, double* out,
                      int B, int Q, int Hq, int Hkv, int D, int page, int max_pages,
                      long long num_pages) {
  build_table();
  const double* g_val = bf16 ? g_bf16_table : g_half_table;
  const int group = Hq / Hkv;
  const long long rows = (long long)B * Q * Hq;

  for (int b = 0; b < B; ++b) {
    const long long len = sl[b] > 0 ? sl[b] : 0;
    const long long pages_used = (len + page - 1) / page;
    if (pages_used > max_pages) return -2;
    for (long long p = 0; p < pages_used; ++p) {
      const int32_t pid = bt[(long long)b * max_pages + p];
      if (pid < 0 || pid >= num_pages) return -1;
    }
  }

#pragma omp parallel
  {
    double* logits = NULL;
    char* seen = NULL;
    long long cap = 0;
    double* qv = (double*)malloc(sizeof(double) * (size_t)D);
    double* acc = (double*)malloc(sizeof(double) * (size_t)D);
#pragma omp for schedule(dynamic, 1)
    for (long long row = 0; row < rows; ++row) {
      const int qh = (int)(row % Hq);
      const int qi = (int)((row / Hq) % Q);
      const int b = (int)(row / ((long long)Hq * Q));
      const int kvh = qh / group;
      const long long len = sl[b] > 0 ? sl[b] : 0;
      const long long draft_base = len - Q;
      double* o = out + row * D;
      if (len > cap) {
        free(logits);
        free(seen);
        cap = len;
        logits = (double*)malloc(sizeof(double) * (size_t)cap);
        seen = (char*)malloc((size_t)cap);
      }
      long long n_seen = 0;
      for (long long t = 0; t < len; ++t) {
        int vis;
        if (!mask) {
          vis = t < draft_base + qi + 1;
        } else {
          const long long j = t - draft_base;
          const uint32_t* words = mask + ((long long)b * Q + qi) * mask_words;
          vis = j < 0 || ((words[j / 32] >> (j % 32)) & 1u);
        }
        seen[t] = (char)vis;
        n_seen += vis;
      }
      if (n_seen == 0) {
        for (int d = 0; d < D; ++d) o[d] = 0.0;
        continue;
      }
      for (int d = 0; d < D; ++d) qv[d] = g_val[q[row * D + d]];
      double peak = -INFINITY;
      for (long long t = 0; t < len; ++t) {
        if (!seen[t]) continue;
        const long long pid = bt[(long long)b * max_pages + t / page];
        const long long kr = pid * ps + (t % page) * ts + (long long)kvh * hs;
        double s = 0.0;
        for (int d = 0; d < D; ++d) s += qv[d] * kv_value(kc, kr + d, kv_elem);
        s *= scale;
        logits[t] = s;
        if (s > peak) peak = s;
      }
      double denom = 0.0;
      for (int d = 0; d < D; ++d) acc[d] = 0.0;
      for (long long t = 0; t < len; ++t) {
        if (!seen[t]) continue;
        const double w = exp(logits[t] - peak);
        denom += w;
        const long long pid = bt[(long long)b * max_pages + t / page];
        const long long vr = pid * ps + (t % page) * ts + (long long)kvh * hs;
        for (int d = 0; d < D; ++d) acc[d] += w * kv_value(vc, vr + d, kv_elem);
      }
      for (int d = 0; d < D; ++d) o[d] = out_scale * acc[d] / denom;
    }
    free(logits);
    free(seen);
    free(qv);
    free(acc);
  }
  return 0;
}

/* The reference's contract: separate [num_pages, page, Hkv, D] caches, causal
 * draft chain, scale D^-1/2. */
int sqa_oracle_f64(const uint16_t* q, const uint16_t* kc, const uint16_t* vc,
                   const int32_t* bt, const int32_t* sl, double* out,
                   int B, int Q, int Hq, int Hkv, int D, int page, int max_pages,
                   long long num_pages) {
  const long long ts = (long long)Hkv * D;
  return sqa_oracle_f64_ex(q, kc, vc, (long long)page * ts, ts, D, bt, sl, NULL, 0,
                           1.0 / sqrt((double)D), 1.0, 0, 0, out, B, Q, Hq, Hkv, D, page,
                           max_pages, num_pages);
}
