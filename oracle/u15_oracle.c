/*
 * u15_oracle.c -- CPU oracle for the MoT projection GEMMs.
 *
 * TEST INFRASTRUCTURE ONLY: the checker, never the thing measured or
 * shipped.  See u15_oracle.h for the contract of each function.
 *
 * How each function is pinned (tests/test_oracle.py):
 *   u15o_f32_to_bf16      exhaustive against numpy's RNE rule over a sweep of
 *                         bit patterns + ties; against the reference's own
 *                         RNE via the compiled reference (oracle/_ref).
 *   u15o_linear(_bf16)    against the compiled reference u15::ref::linear
 *                         (oracle/_ref, built from src/u15-ref.cc) on the
 *                         reference test's own inputs (golden fixture);
 *                         closed forms: identity / permutation weights,
 *                         one-hot rows, K=1 outer product, exact small ints.
 *   u15o_mot_linear_bf16  reference linear per group; exchange control
 *                         (swapping the two weight sets changes the result).
 *   u15o_silu/swiglu      against the compiled reference u15::ref::silu;
 *                         closed forms silu(0)=0, silu(x)->x, odd symmetry
 *                         silu(x)-silu(-x)=x.
 *   u15o_quant_rows_i8    brute-force Python on tiny inputs using exact
 *                         rational arithmetic (fractions); invariants:
 *                         |q|<=127, the absmax element maps to +-127, zero
 *                         rows, ties away from zero.
 *   u15o_gemm_i8_i32      brute-force Python integer sums; the exact
 *                         row/column-sum identity; +-127 extremes.
 *   u15o_dequant_*        float32 numpy evaluation of the same expression.
 *   u15o_f16_to_bf16_n    every finite and infinite f16 pattern against
 *                         numpy's f16 -> f32 widening then torch's RNE;
 *                         NaN patterns follow the reference's bit rule
 *                         (checked on the device, not independently).
 *   u15o_attention        bit-equal to the compiled reference's
 *                         u15::ref::attention (with its block_causal_mask
 *                         or a causal mask) on packed copies of the cache;
 *                         the reference tests' controls: a wrong GQA group
 *                         differs, block-causal differs from causal on an
 *                         edit-shaped prefix and equals it on pure text.
 *   u15o_rms_norm, u15o_rope_inv_freq, u15o_rope_half
 *                         bit-equal to the compiled reference's
 *                         u15::ref::rms_norm / rope_inv_freq /
 *                         rope_half_inplace on random inputs.
 *   u15o_rope_tables      closed forms (position 0: cos 1, sin 0; the
 *                         first pair of every range has frequency 1),
 *                         the doubled halves, and ref::rope_half on the
 *                         table's angles.
 *   u15o_split_qk_norm_rope
 *                         its projection composition equals the compiled
 *                         reference's split_rope_project (u15-ref.cc:
 *                         121-175) after re-layout; the reference test's
 *                         negative controls (h/w swapped, one whole-head
 *                         norm) differ by > 1e-2; rotation preserves each
 *                         pair's norm.
 */
#include "u15_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

uint16_t
u15o_f32_to_bf16(float f)
{
  /* src/u15-weights.cc:51-64: round to nearest even on the upper half. */
  uint32_t u;
  memcpy(&u, &f, 4);
  const uint32_t r = ((u >> 16) & 1u) + 0x7fffu;
  return (uint16_t)((u + r) >> 16);
}

float
u15o_bf16_to_f32(uint16_t h)
{
  const uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

void
u15o_f32_to_bf16_n(const float* in, size_t n, uint16_t* out)
{
  for (size_t i = 0; i < n; ++i) { out[i] = u15o_f32_to_bf16(in[i]); }
}

void
u15o_bf16_to_f32_n(const uint16_t* in, size_t n, float* out)
{
  for (size_t i = 0; i < n; ++i) { out[i] = u15o_bf16_to_f32(in[i]); }
}

void
u15o_linear(const float* x, const float* w, const float* b, size_t rows,
            size_t in_dim, size_t out_dim, float* y)
{
  /* src/u15-ref.cc:33-49: one double accumulator per output, seeded with
   * the bias, summed in input-index order, narrowed to f32 once. */
  for (size_t r = 0; r < rows; ++r) {
    const float* xr = x + r * in_dim;
    float* yr = y + r * out_dim;
    for (size_t o = 0; o < out_dim; ++o) {
      const float* wr = w + o * in_dim;
      double acc = (b != NULL) ? (double)b[o] : 0.0;
      for (size_t i = 0; i < in_dim; ++i) {
        acc += (double)xr[i] * (double)wr[i];
      }
      yr[o] = (float)acc;
    }
  }
}

void
u15o_linear_bf16(const uint16_t* x, const uint16_t* w, const uint16_t* b,
                 const int32_t* row_ids, size_t rows, size_t in_dim,
                 size_t out_dim, float* y)
{
  /* Same arithmetic as u15o_linear with the operands widened exactly from
   * bf16 (the reference's upload path rounds to bf16 and the kernel widens,
   * tests/u15-kernels-test.cc:83-90). Rows are widened one at a time. */
  float* xr = (float*)malloc(in_dim * sizeof(float));
  if (xr == NULL) { return; }
  for (size_t rr = 0; rr < rows; ++rr) {
    const size_t r = row_ids ? (size_t)row_ids[rr] : rr;
    for (size_t i = 0; i < in_dim; ++i) {
      xr[i] = u15o_bf16_to_f32(x[r * in_dim + i]);
    }
    float* yr = y + rr * out_dim;
    for (size_t o = 0; o < out_dim; ++o) {
      const uint16_t* wr = w + o * in_dim;
      double acc = (b != NULL) ? (double)u15o_bf16_to_f32(b[o]) : 0.0;
      for (size_t i = 0; i < in_dim; ++i) {
        acc += (double)xr[i] * (double)u15o_bf16_to_f32(wr[i]);
      }
      yr[o] = (float)acc;
    }
  }
  free(xr);
}

void
u15o_mot_linear_bf16(const uint16_t* x, const uint16_t* w_und,
                     const uint16_t* w_gen, size_t M_und, size_t M_gen,
                     size_t K, size_t N, float* y)
{
  /* src/u15-backbone.cc:189: `w = (e == Gen) ? L.gen : L.und`, applied to
   * the und row group and the gen row group in turn. */
  u15o_linear_bf16(x, w_und, NULL, NULL, M_und, K, N, y);
  u15o_linear_bf16(x + M_und * K, w_gen, NULL, NULL, M_gen, K, N,
                   y + M_und * N);
}

void
u15o_silu(float* x, size_t n)
{
  /* src/u15-ref.cc:51-58 */
  for (size_t i = 0; i < n; ++i) {
    const double v = (double)x[i];
    x[i] = (float)(v / (1.0 + exp(-v)));
  }
}

void
u15o_swiglu_bf16(const uint16_t* g, const uint16_t* u, size_t n, float* out)
{
  /* src/u15-ref.cc:303-304: silu(gate) in place, then gate *= up. */
  for (size_t i = 0; i < n; ++i) {
    float gv = u15o_bf16_to_f32(g[i]);
    u15o_silu(&gv, 1);
    out[i] = gv * u15o_bf16_to_f32(u[i]);
  }
}

void
u15o_quant_rows_i8(const uint16_t* x, size_t rows, size_t K, int8_t* q,
                   float* s)
{
  for (size_t r = 0; r < rows; ++r) {
    const uint16_t* xr = x + r * K;
    float amax = 0.0f;
    for (size_t k = 0; k < K; ++k) {
      const float v = fabsf(u15o_bf16_to_f32(xr[k]));
      if (v > amax) { amax = v; }
    }
    const float sc = amax / 127.0f;      /* f32 division, round-to-nearest */
    s[r] = sc;
    for (size_t k = 0; k < K; ++k) {
      long c = 0;
      if (sc != 0.0f) {
        const float t = u15o_bf16_to_f32(xr[k]) / sc;
        c = lroundf(t);                  /* half away from zero */
        if (c > 127) { c = 127; }
        if (c < -127) { c = -127; }
      }
      q[r * K + k] = (int8_t)c;
    }
  }
}

int
u15o_gemm_i8_i32(const int8_t* a, const int8_t* w, const int32_t* row_ids,
                 size_t rows, size_t K, size_t N, int32_t* acc)
{
  int ok = 0;
  for (size_t rr = 0; rr < rows; ++rr) {
    const size_t r = row_ids ? (size_t)row_ids[rr] : rr;
    const int8_t* ar = a + r * K;
    for (size_t n = 0; n < N; ++n) {
      const int8_t* wr = w + n * K;
      int64_t t = 0;
      for (size_t k = 0; k < K; ++k) { t += (int32_t)ar[k] * (int32_t)wr[k]; }
      if (t > INT32_MAX || t < INT32_MIN) { ok = -1; }
      acc[rr * N + n] = (int32_t)t;
    }
  }
  return ok;
}

void
u15o_i8_product_sums(const int8_t* a, const int8_t* w, size_t rows, size_t K,
                     size_t N, int64_t* rowsum, int64_t* colsum)
{
  /* rowsum = A . (W^T 1) and colsum = (1^T A) . W^T, exact in int64. */
  int64_t* wk = (int64_t*)calloc(K, sizeof(int64_t));
  int64_t* ak = (int64_t*)calloc(K, sizeof(int64_t));
  if (!wk || !ak) { free(wk); free(ak); return; }
  for (size_t n = 0; n < N; ++n) {
    for (size_t k = 0; k < K; ++k) { wk[k] += w[n * K + k]; }
  }
  for (size_t r = 0; r < rows; ++r) {
    int64_t t = 0;
    for (size_t k = 0; k < K; ++k) {
      t += (int64_t)a[r * K + k] * wk[k];
      ak[k] += a[r * K + k];
    }
    rowsum[r] = t;
  }
  for (size_t n = 0; n < N; ++n) {
    int64_t t = 0;
    for (size_t k = 0; k < K; ++k) { t += ak[k] * (int64_t)w[n * K + k]; }
    colsum[n] = t;
  }
  free(wk);
  free(ak);
}

void
u15o_dequant_bf16(const int32_t* acc, const float* sa, const float* sw,
                  size_t rows, size_t N, uint16_t* y)
{
  for (size_t r = 0; r < rows; ++r) {
    for (size_t n = 0; n < N; ++n) {
      const float a = (float)acc[r * N + n];      /* RNE int32 -> f32 */
      const float v = (a * sa[r]) * sw[n];
      y[r * N + n] = u15o_f32_to_bf16(v);
    }
  }
}

void
u15o_dequant_f64(const int32_t* acc, const float* sa, const float* sw,
                 size_t rows, size_t N, double* y)
{
  for (size_t r = 0; r < rows; ++r) {
    for (size_t n = 0; n < N; ++n) {
      y[r * N + n] = (double)acc[r * N + n] * (double)sa[r] * (double)sw[n];
    }
  }
}

void
u15o_dequant_affine(const uint32_t* codes, const uint16_t* scales,
                     const uint16_t* biases, int bits, int group, size_t N,
                     size_t K, uint16_t* w_out)
{
  const size_t per_word = 32u / (size_t)bits;
  const uint32_t mask = (1u << bits) - 1u;
  const size_t words = K / per_word;
  const size_t groups = K / (size_t)group;
  for (size_t n = 0; n < N; ++n) {
    for (size_t k = 0; k < K; ++k) {
      const uint32_t word = codes[n * words + k / per_word];
      const uint32_t code = (word >> ((k % per_word) * (size_t)bits)) & mask;
      const float sc = u15o_bf16_to_f32(scales[n * groups + k / group]);
      const float bi = u15o_bf16_to_f32(biases[n * groups + k / group]);
      volatile float prod = sc * (float)code;   /* no fused multiply-add */
      w_out[n * K + k] = u15o_f32_to_bf16(prod + bi);
    }
  }
}

void
u15o_pack_affine(const float* w, int bits, int group, size_t N, size_t K,
                 uint32_t* codes, uint16_t* scales, uint16_t* biases,
                 float* deq)
{
  /* tests/u15-m5-test.cc:263-310, with 255 generalised to 2^bits - 1 */
  const long qmax = (1L << bits) - 1;
  const size_t per_word = 32u / (size_t)bits;
  const size_t words = K / per_word;
  const size_t groups = K / (size_t)group;
  for (size_t n = 0; n < N; ++n) {
    for (size_t w_i = 0; w_i < words; ++w_i) { codes[n * words + w_i] = 0u; }
    for (size_t g = 0; g < groups; ++g) {
      const size_t k0 = g * (size_t)group;
      float lo = w[n * K + k0], hi = lo;
      for (int i = 1; i < group; ++i) {
        const float v = w[n * K + k0 + (size_t)i];
        if (v < lo) { lo = v; }
        if (v > hi) { hi = v; }
      }
      const float sf = u15o_bf16_to_f32(u15o_f32_to_bf16((hi - lo) / (float)qmax));
      const float bf = u15o_bf16_to_f32(u15o_f32_to_bf16(lo));
      scales[n * groups + g] = u15o_f32_to_bf16(sf);
      biases[n * groups + g] = u15o_f32_to_bf16(bf);
      for (int i = 0; i < group; ++i) {
        const size_t k = k0 + (size_t)i;
        const float v = w[n * K + k];
        long c = sf > 0.0f ? lroundf((v - bf) / sf) : 0;
        if (c < 0) { c = 0; }
        if (c > qmax) { c = qmax; }
        codes[n * words + k / per_word] |=
            (uint32_t)c << ((k % per_word) * (size_t)bits);
        if (deq != NULL) { deq[n * K + k] = sf * (float)c + bf; }
      }
    }
  }
}

void
u15o_bias_add_bf16(uint16_t* y, const uint16_t* b, size_t rows, size_t N)
{
  for (size_t r = 0; r < rows; ++r) {
    for (size_t n = 0; n < N; ++n) {
      const float v = u15o_bf16_to_f32(y[r * N + n]) + u15o_bf16_to_f32(b[n]);
      y[r * N + n] = u15o_f32_to_bf16(v);
    }
  }
}

void
u15o_f16_to_bf16_n(const uint16_t* in, size_t n, uint16_t* out)
{
  /* src/u15-weights.cc:66-94: f16 -> f32 by expanding the exponent
   * (subnormals renormalised, Inf/NaN carried with the payload shifted
   * up), then the same RNE as f32_to_bf16. */
  for (size_t i = 0; i < n; ++i) {
    const uint32_t h = in[i];
    const uint32_t sign = (h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t man = h & 0x3ffu;
    uint32_t f;
    if (exp == 0) {
      if (man == 0) {
        f = sign;
      } else {
        exp = 127 - 15 + 1;
        while ((man & 0x400u) == 0) { man <<= 1; --exp; }
        man &= 0x3ffu;
        f = sign | (exp << 23) | (man << 13);
      }
    } else if (exp == 31) {
      f = sign | 0x7f800000u | (man << 13);
    } else {
      f = sign | ((exp - 15 + 127) << 23) | (man << 13);
    }
    out[i] = (uint16_t)((f + ((f >> 16) & 1u) + 0x7fffu) >> 16);
  }
}

/* ---- the step after the q/k projections: split norm + split RoPE ---- */

void
u15o_rms_norm(const float* x, const float* w, float eps, size_t rows,
              size_t dim, float* out)
{
  /* src/u15-ref.cc:12-31: double sum of squares, double inverse root,
   * each output x * inv * w narrowed once. */
  for (size_t r = 0; r < rows; ++r) {
    const float* xr = x + r * dim;
    float* o = out + r * dim;
    double acc = 0.0;
    for (size_t c = 0; c < dim; ++c) { acc += (double)xr[c] * xr[c]; }
    const double inv = 1.0 / sqrt(acc / (double)dim + (double)eps);
    for (size_t c = 0; c < dim; ++c) {
      o[c] = (float)((double)xr[c] * inv * (double)w[c]);
    }
  }
}

void
u15o_rope_inv_freq(int dim, double theta, float* inv)
{
  /* src/u15-ref.cc:77-86: inv[i] = 1 / theta^(2i/dim), narrowed to f32. */
  for (int i = 0; i < dim / 2; ++i) {
    inv[i] = (float)(1.0 / pow(theta, (double)(2 * i) / (double)dim));
  }
}

void
u15o_rope_half(float* x, const float* inv, int dim, double pos)
{
  /* src/u15-ref.cc:88-101: rotate_half over dim/2 pairs (j, j + dim/2),
   * the angle and the rotation in double. */
  const int half = dim / 2;
  for (int j = 0; j < half; ++j) {
    const double ang = pos * (double)inv[j];
    const double c = cos(ang), s = sin(ang);
    const double a = (double)x[j], b = (double)x[j + half];
    x[j] = (float)(a * c - b * s);
    x[j + half] = (float)(b * c + a * s);
  }
}

void
u15o_rope_tables(const int32_t* pos_t, const int32_t* pos_h,
                 const int32_t* pos_w, size_t T, int D, int d_t, int d_h,
                 double theta_t, double theta_hw, float* cosf, float* sinf)
{
  /* src/u15-metal-ops.cc:547-600 (build_rope_tables): per token, the three
   * ranges [0,d_t) t, [d_t,d_t+d_h) h, [d_t+d_h,D) w, each filled with its
   * own ladder inv = 1/theta^(2i/width) formed in double, the angle
   * pos*inv in double, cos/sin narrowed once, doubled cat(f, f) across the
   * range's two halves. */
  const int off[3] = {0, d_t, d_t + d_h};
  const int width[3] = {d_t, d_h, d_h};
  const double theta[3] = {theta_t, theta_hw, theta_hw};
  const int32_t* pos[3] = {pos_t, pos_h, pos_w};
  for (int r = 0; r < 3; ++r) {
    const int half = width[r] / 2;
    for (size_t t = 0; t < T; ++t) {
      for (int i = 0; i < half; ++i) {
        const double inv =
            1.0 / pow(theta[r], (double)(2 * i) / (double)width[r]);
        const double a = (double)pos[r][t] * inv;
        const float cv = (float)cos(a), sv = (float)sin(a);
        const size_t b = t * (size_t)D + (size_t)off[r];
        cosf[b + i] = cv;
        sinf[b + i] = sv;
        cosf[b + i + half] = cv;
        sinf[b + i + half] = sv;
      }
    }
  }
}

void
u15o_split_qk_norm_rope(float* x, const float* w_t, const float* w_hw,
                        const int32_t* pos_t, const int32_t* pos_h,
                        const int32_t* pos_w, size_t T, size_t H, int D,
                        int d_t, int d_h, double theta_t, double theta_hw,
                        float eps, int do_norm, int do_rope)
{
  /* The reference test's CPU path (tests/u15-kernels-test.cc:156-181),
   * the same two steps split_qk_norm and split_rope take: on each
   * (token, head) row of x [T][H*D], rms_norm of the two halves
   * [0, D/2) and [D/2, D) with their own weights, then rotate_half on the
   * three ranges with ladders 1/theta_t^(2i/d_t) and 1/theta_hw^(2i/d_h)
   * (u15-ref.cc:121-175 uses the same split). */
  const int half = D / 2;
  float inv_t[256], inv_h[256], a[512], na[512];
  u15o_rope_inv_freq(d_t, theta_t, inv_t);
  u15o_rope_inv_freq(d_h, theta_hw, inv_h);
  for (size_t t = 0; t < T; ++t) {
    for (size_t h = 0; h < H; ++h) {
      float* row = x + (t * H + h) * (size_t)D;
      if (do_norm) {
        for (int c = 0; c < half; ++c) { a[c] = row[c]; }
        u15o_rms_norm(a, w_t, eps, 1, (size_t)half, na);
        for (int c = 0; c < half; ++c) { row[c] = na[c]; }
        for (int c = 0; c < half; ++c) { a[c] = row[half + c]; }
        u15o_rms_norm(a, w_hw, eps, 1, (size_t)half, na);
        for (int c = 0; c < half; ++c) { row[half + c] = na[c]; }
      }
      if (do_rope) {
        u15o_rope_half(row, inv_t, d_t, (double)pos_t[t]);
        u15o_rope_half(row + d_t, inv_h, d_h, (double)pos_h[t]);
        u15o_rope_half(row + d_t + d_h, inv_h, d_h, (double)pos_w[t]);
      }
    }
  }
}

/* ---- attention ------------------------------------------------------ */

static int
attn_allowed(int mode, const int32_t* t_index, size_t qpos, size_t j)
{
  /* mode 0: bidirectional; 1: causal, j <= qpos; 2: block-causal
   * (src/u15-ref.cc:179-192): t[j] == t[qpos] or j <= qpos. */
  if (mode == 0) { return 1; }
  if (j <= qpos) { return 1; }
  return mode == 2 && t_index[j] == t_index[qpos];
}

void
u15o_attention(const float* q, const float* k, const float* v, int mode,
               const int32_t* t_index, size_t hq, size_t hkv, size_t tq,
               size_t tk, size_t d, size_t cap, size_t q_offset, float* out)
{
  /* src/u15-ref.cc:194-235 (attention): per query head h, its kv head
   * h / (hq/hkv); scores q.k in double scaled by 1/sqrt(d); masked keys
   * dropped (the additive -inf); softmax in double; out = sum p v.
   * Layouts as the GPU path keeps them: q and out head-major [hq][tq][d],
   * k and v a cache [hkv][cap][d] of which keys [0, tk) are in use; the
   * queries sit at key positions q_offset + i. */
  const double scale = 1.0 / sqrt((double)d);
  const size_t group = hq / hkv;
  double* row = (double*)malloc(sizeof(double) * (tk > 0 ? tk : 1));
  for (size_t h = 0; h < hq; ++h) {
    const size_t hk = h / group;
    for (size_t i = 0; i < tq; ++i) {
      const float* qi = q + (h * tq + i) * d;
      const size_t qpos = q_offset + i;
      double mx = -INFINITY;
      for (size_t j = 0; j < tk; ++j) {
        if (!attn_allowed(mode, t_index, qpos, j)) { row[j] = -INFINITY; continue; }
        const float* kj = k + (hk * cap + j) * d;
        double acc = 0.0;
        for (size_t c = 0; c < d; ++c) { acc += (double)qi[c] * (double)kj[c]; }
        row[j] = acc * scale;
        if (row[j] > mx) { mx = row[j]; }
      }
      double sum = 0.0;
      for (size_t j = 0; j < tk; ++j) {
        row[j] = isinf(row[j]) && row[j] < 0 ? 0.0 : exp(row[j] - mx);
        sum += row[j];
      }
      const double inv = sum > 0.0 ? 1.0 / sum : 0.0;
      float* o = out + (h * tq + i) * d;
      for (size_t c = 0; c < d; ++c) {
        double acc = 0.0;
        for (size_t j = 0; j < tk; ++j) {
          acc += row[j] * inv * (double)v[(hk * cap + j) * d + c];
        }
        o[c] = (float)acc;
      }
    }
  }
  free(row);
}

double
u15o_rel_l2(const float* a, const float* b, size_t n)
{
  /* tests/u15-kernels-test.cc:95-105 */
  double num = 0.0, den = 0.0;
  for (size_t i = 0; i < n; ++i) {
    const double d = (double)a[i] - (double)b[i];
    num += d * d;
    den += (double)b[i] * (double)b[i];
  }
  return den > 0.0 ? sqrt(num / den) : sqrt(num);
}

double
u15o_max_rel(const float* a, const float* b, size_t n)
{
  double md = 0.0, mb = 0.0;
  for (size_t i = 0; i < n; ++i) {
    const double d = fabs((double)a[i] - (double)b[i]);
    if (d > md) { md = d; }
    if (fabs((double)b[i]) > mb) { mb = fabs((double)b[i]); }
  }
  return mb > 0.0 ? md / mb : md;
}
