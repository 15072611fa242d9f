/*
 * u15_oracle.h -- CPU oracle for the MoT projection GEMMs.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker the GPU path is
 * compared against.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it; the product library never links it and has
 * no CPU fallback.
 *
 * Each function restates the reference's algorithm and cites the
 * reference file:line it follows (tgo-app-dev/vpipe-sensenova-u1.5).
 * Everything is single-threaded, like the reference's CPU path.
 *
 * Pinning (what checks each function against something other than itself)
 * is listed in the header comment of u15_oracle.c.
 */
#ifndef U15_ORACLE_H
#define U15_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* bf16 <-> f32.  to: round-to-nearest-even as src/u15-weights.cc:51-64
 * (and the tests' to_bf16, tests/u15-kernels-test.cc:65-73); from: a
 * 16-bit shift, tests/u15-kernels-test.cc:75-81. */
uint16_t u15o_f32_to_bf16(float f);
float    u15o_bf16_to_f32(uint16_t h);
void     u15o_f32_to_bf16_n(const float* in, size_t n, uint16_t* out);
void     u15o_bf16_to_f32_n(const uint16_t* in, size_t n, float* out);

/* y[r][o] = sum_i x[r][i]*w[o][i] (+ b[o]): f32 operands, DOUBLE
 * accumulation in index order, f32 result.  src/u15-ref.cc:33-49. */
void u15o_linear(const float* x, const float* w, const float* b,
                 size_t rows, size_t in_dim, size_t out_dim, float* y);

/* The same on bf16 operands (widened exactly), f32 result (not rounded).
 * `row_ids` selects which rows of x to compute (NULL = all `rows`);
 * y has one row per computed row. */
void u15o_linear_bf16(const uint16_t* x, const uint16_t* w,
                      const uint16_t* b, const int32_t* row_ids,
                      size_t rows, size_t in_dim, size_t out_dim, float* y);

/* The two-group MoT linear: rows [0,M_und) with w_und, rows
 * [M_und, M_und+M_gen) with w_gen -- row-wise the reference's
 * per-pass expert selection, src/u15-backbone.cc:189. */
void u15o_mot_linear_bf16(const uint16_t* x, const uint16_t* w_und,
                          const uint16_t* w_gen, size_t M_und, size_t M_gen,
                          size_t K, size_t N, float* y);

/* silu in double, src/u15-ref.cc:51-58; swiglu = silu(g)*u,
 * src/u15-ref.cc:303-304.  The bf16 variant takes bf16 gate/up (the
 * GEMMs' rounded outputs) and returns f32. */
void u15o_silu(float* x, size_t n);
void u15o_swiglu_bf16(const uint16_t* g, const uint16_t* u, size_t n,
                      float* out);

/* Symmetric per-row int8 quantisation (BASELINE numerics; rounding rule of
 * the reference's only quantisation fixture, std::lround,
 * tests/u15-m5-test.cc:295):
 *   s = absmax/127 (f32, correctly rounded), q = clamp(lround(x/s),-127,127)
 *   s == 0  ->  q = 0. */
void u15o_quant_rows_i8(const uint16_t* x, size_t rows, size_t K, int8_t* q,
                        float* s);

/* Exact int8 GEMM: acc[r][n] = sum_k a[r][k]*w[n][k] in int64, stored int32
 * (checked to fit).  row_ids as u15o_linear_bf16.  Returns 0, or -1 if an
 * accumulator does not fit in int32. */
int u15o_gemm_i8_i32(const int8_t* a, const int8_t* w, const int32_t* row_ids,
                     size_t rows, size_t K, size_t N, int32_t* acc);

/* Exact row / column sums of the int8 product, computed WITHOUT forming
 * it: rowsum[r] = sum_k a[r][k] * (sum_n w[n][k]),
 *         colsum[n] = sum_k (sum_r a[r][k]) * w[n][k]   (int64). */
void u15o_i8_product_sums(const int8_t* a, const int8_t* w, size_t rows,
                          size_t K, size_t N, int64_t* rowsum,
                          int64_t* colsum);

/* Dequant epilogue: y = bf16_rne(((float)acc * sa[r]) * sw[n]). */
void u15o_dequant_bf16(const int32_t* acc, const float* sa, const float* sw,
                       size_t rows, size_t N, uint16_t* y);
/* The same in double without rounding (the "exact" dequantised value). */
void u15o_dequant_f64(const int32_t* acc, const float* sa, const float* sw,
                      size_t rows, size_t N, double* y);

/* Affine-quantized weight packs (the reference's QWeight, u15-metal-ops.h:
 * 39-57; shape rules u15-weights.cc:248-325): codes u32 [N][K*bits/32],
 * scales and biases bf16 [N][K/group]; element k of row n is
 *   w = scale[n][k/group] * code + bias[n][k/group]
 * in f32 (a multiply, then an add), code k sitting at bits
 * [bits*(k % (32/bits)), +bits) of word k / (32/bits) -- the w8 order of the
 * reference's own pack fixture (tests/u15-m5-test.cc:300-306), w4 by the
 * same low-bits-first rule.  dequant writes bf16 (RNE), the expansion the
 * reference's dequant-once route feeds to the dense GEMM
 * (u15-metal-ops.cc:359-400). */
void u15o_dequant_affine(const uint32_t* codes, const uint16_t* scales,
                         const uint16_t* biases, int bits, int group,
                         size_t N, size_t K, uint16_t* w_out);
/* Builds a pack from f32 weights the way the reference's fixture does
 * (tests/u15-m5-test.cc:263-310): per group, scale = bf16((hi-lo)/(2^bits-1)),
 * bias = bf16(lo), code = clamp(lround((w - bias)/scale), 0, 2^bits-1)
 * (0 when scale is 0); `deq` (optional) receives scale*code+bias in f32. */
void u15o_pack_affine(const float* w, int bits, int group, size_t N, size_t K,
                      uint32_t* codes, uint16_t* scales, uint16_t* biases,
                      float* deq);

/* y[r][n] = bf16(y[r][n] + b[n]) (f32 add), the reference's bias_add
 * (u15-metal-ops.cc:435-446). */
void u15o_bias_add_bf16(uint16_t* y, const uint16_t* b, size_t rows, size_t N);

/* f16 -> bf16 the loader's way (src/u15-weights.cc:66-94): widen to f32
 * exactly, then RNE. */
void u15o_f16_to_bf16_n(const uint16_t* in, size_t n, uint16_t* out);

/* The step after the q/k projections (src/u15-ref.h:25-95):
 *   rms_norm      y = x * 1/sqrt(mean(x^2) + eps) * w, double arithmetic
 *   rope_inv_freq inv[i] = 1/theta^(2i/dim), i < dim/2
 *   rope_half     rotate_half on pairs (j, j + dim/2) at one position
 *   rope_tables   the packed [T][D] f32 cos/sin of build_rope_tables
 *                 (src/u15-metal-ops.cc:547-600)
 *   split_qk_norm_rope  on x [T][H*D] in place: the two half norms, then
 *                 the three-way rope [t | h | w] (D/2, D/4, D/4). */
void u15o_rms_norm(const float* x, const float* w, float eps, size_t rows,
                   size_t dim, float* out);
void u15o_rope_inv_freq(int dim, double theta, float* inv);
void u15o_rope_half(float* x, const float* inv, int dim, double pos);
void u15o_rope_tables(const int32_t* pos_t, const int32_t* pos_h,
                      const int32_t* pos_w, size_t T, int D, int d_t, int d_h,
                      double theta_t, double theta_hw, float* cosf,
                      float* sinf);
void u15o_split_qk_norm_rope(float* x, const float* w_t, const float* w_hw,
                             const int32_t* pos_t, const int32_t* pos_h,
                             const int32_t* pos_w, size_t T, size_t H, int D,
                             int d_t, int d_h, double theta_t,
                             double theta_hw, float eps, int do_norm,
                             int do_rope);

/* Grouped-query attention (src/u15-ref.cc:194-235), double arithmetic.
 * q, out head-major [hq][tq][d]; k, v caches [hkv][cap][d], keys [0, tk)
 * in use; query i sits at key position q_offset + i.  mode 0 bidirectional,
 * 1 causal (j <= pos), 2 block-causal (t_index[j] == t_index[pos] or
 * j <= pos; src/u15-ref.cc:179-192). */
void u15o_attention(const float* q, const float* k, const float* v, int mode,
                    const int32_t* t_index, size_t hq, size_t hkv, size_t tq,
                    size_t tk, size_t d, size_t cap, size_t q_offset,
                    float* out);

/* rel-L2 = sqrt(sum (a-b)^2 / sum b^2), tests/u15-kernels-test.cc:95-105;
 * max-rel = max|a-b| / max|b|. */
double u15o_rel_l2(const float* a, const float* b, size_t n);
double u15o_max_rel(const float* a, const float* b, size_t n);

/* The reference tests' input generator: std::mt19937(seed) with
 * std::normal_distribution<float>(0, stddev) from this toolchain's
 * libstdc++ (tests/u15-kernels-test.cc:110-118,
 * tests/u15-m5-test.cc:87-94).  Lets a fixture be regenerated exactly. */
void u15o_randn_mt(uint32_t seed, float stddev, size_t n, float* out);

#ifdef __cplusplus
}
#endif

#endif
