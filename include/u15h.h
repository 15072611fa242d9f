/*
 * u15h.h -- C ABI for the SenseNova-U1.5 Mixture-of-Transformers projection
 * GEMMs on AMD MI355X (gfx950).
 *
 * This is the drop-in boundary for the GEMM half of the reference's op
 * vocabulary, `u15::MetalOps` (src/u15-metal-ops.h:59-531 in
 * tgo-app-dev/vpipe-sensenova-u1.5). Every entry point below names the
 * reference interface it replaces.
 *
 * Conventions (the reference's, src/u15-metal-ops.h:102-103 and
 * src/u15-ref.h:13-17):
 *   activations  x [M][K]  row-major (token-major), bf16
 *   weights      w [N][K]  row-major ([out][in], as torch stores them), bf16
 *   output       y [M][N]  row-major, bf16
 *   y[m][n] = sum_k x[m][k] * w[n][k]  (+ bias[n]),  fp32 accumulation
 *
 * Mixture-of-Transformers routing: every projection exists twice, the base
 * ("und") weight set used by understanding tokens and the `_mot_gen` ("gen")
 * set used by generated-image tokens (reference src/u15-backbone.cc:189,
 * src/u15-weights.h:97-117).  In the grouped entry points the activation
 * rows are split in two contiguous groups: rows [0, M_und) use the und
 * weights and rows [M_und, M_und + M_gen) use the gen weights.  Both groups
 * run in ONE kernel launch.  u15h_route_rows() builds the gather/scatter
 * row map for the case where token types are interleaved.
 *
 * Memory: the caller owns every pointer passed in; all are device pointers
 * (hipMalloc / torch) unless stated.  The context owns only its scratch.
 * Alignment: every pointer must be 16-byte aligned.
 *
 * Ordering: every call enqueues on the caller's hipStream_t and returns
 * without synchronising.  A context is not thread-safe: use one per host
 * thread, or serialise.  A context owns scratch memory that its GEMM calls
 * write and read on the device (the split-K partial sums, the int8 route's
 * codes and scales, the dequant expansion), so ALL calls on one context
 * must be ordered on ONE stream (or otherwise ordered by the caller, e.g.
 * with events): two calls on one context queued on unordered streams race
 * on that scratch.  Use one context per stream for concurrent work.
 *
 * Errors: every call returns a u15h_status.  On any non-OK status from a
 * shape / argument check NOTHING has been launched (the reference's
 * "encoder untouched on a decline", src/u15-metal-ops.cc:297-299).
 * u15h_last_error() gives a human-readable reason.
 */
#ifndef U15H_H
#define U15H_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct u15h_ctx u15h_ctx;
typedef void*           u15h_stream;   /* a hipStream_t; NULL = the null stream */
typedef uint16_t        u15h_bf16;     /* bf16 bit pattern */

typedef enum {
  U15H_OK      = 0,
  U15H_EINVAL  = 1, /* bad shape, alignment, null pointer, or limit exceeded */
  U15H_ENODEV  = 2, /* no usable gfx950 device / kernels not loadable        */
  U15H_ELAUNCH = 3, /* the HIP runtime rejected a launch                     */
  U15H_ENOMEM  = 4  /* scratch allocation failed                             */
} u15h_status;

#define U15H_ABI_VERSION 1
/* Grouped entry points take at most this many projections per launch. */
#define U15H_MAX_PROJ 4

/* ------------------------------------------------------------------ */
/* context                                                             */
/* ------------------------------------------------------------------ */

/* Replaces MetalOps::init (src/u15-metal-ops.cc:39-245): binds a device,
 * checks that it is gfx950 and that every kernel of this library is
 * loadable, and refuses otherwise (ENODEV) instead of running a silent
 * no-op.  `device` is a HIP device ordinal. */
u15h_status u15h_create(int device, u15h_ctx** out);
void        u15h_destroy(u15h_ctx* ctx);
int         u15h_abi_version(void);
const char* u15h_status_str(u15h_status s);
/* Reason for the last non-OK status on this context ("" if none). */
const char* u15h_last_error(const u15h_ctx* ctx);

/* ------------------------------------------------------------------ */
/* dense bf16 GEMM                                                     */
/* ------------------------------------------------------------------ */

/* Replaces MetalOps::linear(enc, x, w, bias, y, M, K, N)
 * (src/u15-metal-ops.h:102-109, src/u15-metal-ops.cc:327-346) and its
 * BN=64 twin MetalOps::linear_wide (src/u15-metal-ops.h:111-119).
 * y[M][N] = x[M][K] . w[N][K]^T (+ bias[N]).  bias may be NULL.
 * If the int8 tier is on (u15h_enable_i8_gemm) and the shape qualifies
 * (M >= the tier's row floor, K % 128 == 0) the call is served by the int8
 * path with per-call quantisation of both operands -- the interception
 * MetalOps::linear_mma_ makes (src/u15-metal-ops.cc:283-306).  The K rule
 * differs from the reference's on purpose: its tier quantises per 512-wide
 * group of K and so takes only K % 512 == 0 (src/u15-metal-ops.h:76-83);
 * this tier's scales are per token and per output channel (no K groups),
 * so any K its 128-byte LDS stages divide qualifies.  Every projection of
 * the model (K = 4096, 12288) passes both rules.  At most 128
 * rows with K % 64 == 0 run a weight-streaming kernel (16 or 64 output
 * columns per workgroup) instead of the 256 x 256 tiles.
 * Limits: M >= 0, N > 0, K > 0, K % 8 == 0, N % 8 == 0. */
u15h_status u15h_linear(u15h_ctx* ctx, u15h_stream stream,
                        const u15h_bf16* x, const u15h_bf16* w,
                        const u15h_bf16* bias, u15h_bf16* y,
                        int M, int K, int N);

/* One projection of a MoT layer: both weight sets and its output. */
typedef struct {
  const u15h_bf16* w_und;    /* [N][K] base weights (understanding rows)  */
  const u15h_bf16* w_gen;    /* [N][K] _mot_gen weights (generated rows)  */
  const u15h_bf16* bias_und; /* [N] or NULL                               */
  const u15h_bf16* bias_gen; /* [N] or NULL                               */
  u15h_bf16*       y;        /* [M_und + M_gen][N]                        */
  int              N;
} u15h_mot_proj;

/* The two-group grouped GEMM: for each of `nproj` projections sharing the
 * same input x (e.g. q, k and v; or gate and up), rows [0, M_und) of x are
 * multiplied by w_und and rows [M_und, M_und+M_gen) by w_gen, all in one
 * launch.  Row-wise this equals MetalOps::linear with that row's expert's
 * weights (src/u15-backbone.cc:189 selects `L.gen : L.und` per pass; this
 * call does the selection per row group instead of per pass).
 * Limits: 1 <= nproj <= U15H_MAX_PROJ, K % 8 == 0, every N % 8 == 0. */
u15h_status u15h_mot_linear(u15h_ctx* ctx, u15h_stream stream,
                            const u15h_bf16* x, int M_und, int M_gen, int K,
                            const u15h_mot_proj* proj, int nproj);

/* u15h_mot_linear without any device allocation.  No counterpart in the
 * reference; it is for callers that cannot call hipMalloc: code under HIP
 * graph capture, tight serving loops, harnesses that forbid allocation.
 * Same arguments, kernels and results (bit for bit) as u15h_mot_linear,
 * but the split-K partial sums go to a static device array of the
 * library (64 MiB per GPU, one 256x256 tile of 4-byte sums for each of up
 * to 256 compute units; every GPU the library runs on holds it until the
 * process ends) instead of the context's workspace.  Nothing in it needs
 * clearing between calls.  EINVAL if a launch would need more partial sums
 * than the array holds (a GPU with more than 256 CUs); ENODEV if the
 * array's address could not be looked up at u15h_create.  All calls of
 * this entry point on one GPU share the one array -- from any context and
 * any stream -- so calls that can overlap on one GPU race: order them
 * (one stream, or events). */
u15h_status u15h_mot_linear_noalloc(u15h_ctx* ctx, u15h_stream stream,
                                    const u15h_bf16* x, int M_und, int M_gen,
                                    int K, const u15h_mot_proj* proj,
                                    int nproj);

/* Affine-quantized weight pack: the reference's QWeight
 * (src/u15-metal-ops.h:39-57; shape rules src/u15-weights.cc:248-325).
 *   codes  uint32 [N][K*bits/32], code k of a row at bits
 *          [bits*(k % (32/bits)), +bits) of word k / (32/bits)
 *   scales bf16 [N][K/group],  biases bf16 [N][K/group]
 *   w[n][k] = scale * code + bias   (f32 multiply then add, then bf16 RNE)
 * bits 4 or 8, group 32 or 64. */
typedef struct {
  const uint32_t*  codes;
  const u15h_bf16* scales;
  const u15h_bf16* biases;
  int              bits;
  int              group;
} u15h_qweight;

/* Expands a pack to a dense bf16 weight w_out[N][K]: the dequant-once step
 * of MetalOps::linear_mma_q_ (src/u15-metal-ops.cc:359-400). */
u15h_status u15h_dequant_affine(u15h_ctx* ctx, u15h_stream stream,
                                const u15h_qweight* w, int N, int K,
                                u15h_bf16* w_out);

/* Replaces MetalOps::linear(enc, x, QWeight, bias, y, M, K, N) for a
 * quantized pack (src/u15-metal-ops.cc:359-433).  Below the row floor (M <
 * 96, the reference's _mma_q_min_m, src/u15-metal-ops.h:502; env
 * U15H_Q_MIN_M) the pack is read directly, as the reference's steel qmm
 * does (src/u15-metal-ops.cc:402-431): each weight is dequantised in
 * registers to the expansion's bf16 value, so the result equals
 * u15h_linear on the expansion bit for bit (K % 64 == 0; other K take the
 * expansion).  From the floor on: dequant once into the context's
 * grow-only scratch, then u15h_linear's route on the expansion --
 * including its int8 interception when the tier is on and the shape
 * qualifies (the reference's linear_mma_q_ re-enters linear_mma_,
 * src/u15-metal-ops.cc:291-300, 393-399). */
u15h_status u15h_linear_q(u15h_ctx* ctx, u15h_stream stream,
                          const u15h_bf16* x, const u15h_qweight* w,
                          const u15h_bf16* bias, u15h_bf16* y,
                          int M, int K, int N);

/* Replaces MetalOps::bias_add(enc, y, bias, M, N) (src/u15-metal-ops.cc:
 * 435-446): y[m][n] = bf16(y[m][n] + bias[n]), f32 add.  N % 8 == 0. */
u15h_status u15h_bias_add(u15h_ctx* ctx, u15h_stream stream, u15h_bf16* y,
                          const u15h_bf16* bias, int M, int N);

/* f16 -> bf16 on the device: the weight loader's f16_to_bf16_
 * (src/u15-weights.cc:66-94; the pack's scales and biases ship F16): widen
 * to f32 exactly, then RNE.  src holds f16 bit patterns; n % 4 == 0, both
 * pointers 8-byte aligned. */
u15h_status u15h_f16_to_bf16(u15h_ctx* ctx, u15h_stream stream,
                             const uint16_t* src, int64_t n, u15h_bf16* dst);

/* The quantized-pack shape rule of bind_matrix_ (src/u15-weights.cc:
 * 247-325), host only: from K and the column counts of `.scales` and
 * `.weight` (u32 codes), group = K / scales_cols and bits = codes_cols *
 * 32 / K.  U15H_EINVAL unless both close exactly on bits 4/8, group 32/64. */
u15h_status u15h_qweight_geometry(int K, int64_t scales_cols,
                                  int64_t codes_cols, int* bits, int* group);

/* Affine pack -> per-output-channel symmetric int8, the int8 tier's weight
 * format: the pack is expanded to bf16 (as u15h_dequant_affine, into the
 * context's dequant scratch) and each row quantised as
 * u15h_quant_rows_i8: sw[n] = absmax/127, wq[n][k] = clamp(round(w/sw)).
 * No reference counterpart (the reference's int8 tier quantises its
 * weights inside the un-vendored I8GemmContext); this is the repack the
 * scope table names for feeding the int8 GEMM from a quantized checkpoint. */
u15h_status u15h_repack_affine_i8(u15h_ctx* ctx, u15h_stream stream,
                                  const u15h_qweight* w, int N, int K,
                                  int8_t* wq, float* sw);

/* f32 -> bf16 round-to-nearest-even on the device: the weight loader's
 * conversion (src/u15-weights.cc:51-64).  n % 4 == 0. */
u15h_status u15h_f32_to_bf16(u15h_ctx* ctx, u15h_stream stream,
                             const float* src, int64_t n, u15h_bf16* dst);

/* ------------------------------------------------------------------ */
/* The step after the q/k projections: split norm and split RoPE       */
/* ------------------------------------------------------------------ */

/* Replaces MetalOps::split_qk_norm(enc, x, w_t, w_hw, heads, tokens,
 * head_dim, eps) (src/u15-metal-ops.h:169-173, .cc:508-524;
 * kernel u15_split_qk_norm, src/u15-kernels.metal:50-90).  x [tokens]
 * [heads*head_dim] bf16 in place; per (token, head) the halves [0, D/2)
 * and [D/2, D) are normalised separately:
 *   y = x * rsqrt(mean(half^2) + eps) * w   (w_t / w_hw bf16 [D/2], f32)
 * head_dim even, <= 512. */
u15h_status u15h_split_qk_norm(u15h_ctx* ctx, u15h_stream stream,
                               u15h_bf16* x, const u15h_bf16* w_t,
                               const u15h_bf16* w_hw, int heads, int tokens,
                               int head_dim, float eps);

/* Replaces MetalOps::split_rope(enc, x, cos, sin, heads, tokens, head_dim,
 * d_t, d_h) (src/u15-metal-ops.h:177-181, .cc:526-545; kernel
 * u15_split_rope, src/u15-kernels.metal:92-157): rotate_half on the ranges
 * [0,d_t) t, [d_t,d_t+d_h) h, [d_t+d_h,head_dim) w of every head, with the
 * f32 tables cos/sin [tokens][head_dim] from u15h_build_rope_tables (device
 * memory).  d_t + 2*d_h == head_dim, both even. */
u15h_status u15h_split_rope(u15h_ctx* ctx, u15h_stream stream, u15h_bf16* x,
                            const float* cos_tab, const float* sin_tab,
                            int heads, int tokens, int head_dim, int d_t,
                            int d_h);

/* Both in one pass over x (no reference counterpart; the backbone issues
 * them back to back, src/u15-backbone.cc:203-206): the normalised row
 * stays in f32 between the norm and the rotation. */
u15h_status u15h_split_qk_norm_rope(u15h_ctx* ctx, u15h_stream stream,
                                    u15h_bf16* x, const u15h_bf16* w_t,
                                    const u15h_bf16* w_hw,
                                    const float* cos_tab,
                                    const float* sin_tab, int heads,
                                    int tokens, int head_dim, int d_t,
                                    int d_h, float eps);

/* One expert's q and k norm weights (ExpertLayer's q_norm, q_norm_hw,
 * k_norm, k_norm_hw; src/u15-weights.h:97-117), each [head_dim / 2]. */
typedef struct {
  const u15h_bf16* q_t;
  const u15h_bf16* q_hw;
  const u15h_bf16* k_t;
  const u15h_bf16* k_hw;
} u15h_qk_norm;

/* The attention prologue of a two-group pass in ONE launch.  It replaces
 * the calls between the q/k/v projections and attention in
 * U15Backbone::layer_step_ (src/u15-backbone.cc:203-216: split_qk_norm on
 * q and k, split_rope on q and k, transpose_into_cache of k and v), with
 * rows [0, M_und) taking `und`'s norm weights and the next M_gen rows
 * `gen`'s, as the grouped projections do.  For token t and head h:
 *   q[t][h]                    <- rope(norm(q[t][h]))   in place
 *   k_cache[h][offset + t][:]  <- rope(norm(k[t][h]))
 *   v_cache[h][offset + t][:]  <- v[t][h]
 * q is [T][hq*head_dim], k and v [T][hkv*head_dim] (T = M_und + M_gen),
 * caches [hkv][cap][head_dim].  k and v are only read.  Bits equal
 * u15h_split_qk_norm_rope on q and k per expert group, then
 * u15h_transpose_into_cache of k and v.  No reference counterpart as one
 * call.  Limits: head_dim a power of two in [16, 512], d_t / 16 and
 * d_h / 16 powers of two with d_h dividing d_t (the model's 64 | 32 | 32),
 * every pointer 16-byte aligned, offset + T <= cap; other shapes take the
 * separate calls. */
u15h_status u15h_mot_attention_prologue(
    u15h_ctx* ctx, u15h_stream stream, u15h_bf16* q, const u15h_bf16* k,
    const u15h_bf16* v, const u15h_qk_norm* und, const u15h_qk_norm* gen,
    const float* cos_tab, const float* sin_tab, int M_und, int M_gen, int hq,
    int hkv, int head_dim, int d_t, int d_h, float eps, u15h_bf16* k_cache,
    u15h_bf16* v_cache, int cap, int offset);

/* Replaces MetalOps::build_rope_tables(pos_t, pos_h, pos_w, head_dim, d_t,
 * d_h, theta_t, theta_hw) (src/u15-metal-ops.h:186-195, .cc:547-600).  HOST
 * function, no context: fills host arrays cos_tab/sin_tab [tokens]
 * [head_dim]; per range the ladder 1/theta^(2i/width) and the angle
 * pos*inv are formed in double and narrowed once, each range's second half
 * repeating its first.  The caller copies the tables to the device. */
u15h_status u15h_build_rope_tables(const int32_t* pos_t, const int32_t* pos_h,
                                   const int32_t* pos_w, int tokens,
                                   int head_dim, int d_t, int d_h,
                                   double theta_t, double theta_hw,
                                   float* cos_tab, float* sin_tab);

/* ------------------------------------------------------------------ */
/* Attention over the K/V cache                                        */
/* ------------------------------------------------------------------ */

/* Replaces MetalOps::sdpa(enc, q, k, v, out, hq, hkv, tq, tk, d, cap,
 * causal, q_offset) (src/u15-metal-ops.h:226-232, .cc:648-676) and, with
 * causal = 0, sdpa_steel (h:289-295, the bidirectional flash path the
 * backbone uses for generation, src/u15-backbone.cc:225-232).
 *   q, out  HEAD-major [hq][tq][d] bf16
 *   k, v    caches [hkv][cap][d] bf16; keys [0, tk) in use, so the stride
 *           between kv heads is the CAPACITY cap, not tk
 *   query head h reads kv head h / (hq / hkv)  (the GQA group size)
 *   softmax(q.k / sqrt(d)) . v, f32 accumulation; causal: key j attends
 *   iff j <= q_offset + i (queries sit at q_offset within the keys).
 * d in {32, 64, 128}; hq % hkv == 0; tk <= cap. */
u15h_status u15h_sdpa(u15h_ctx* ctx, u15h_stream stream, const u15h_bf16* q,
                      const u15h_bf16* k, const u15h_bf16* v, u15h_bf16* out,
                      int hq, int hkv, int tq, int tk, int d, int cap,
                      int causal, int q_offset);

/* Replaces MetalOps::sdpa_block_causal (src/u15-metal-ops.h:330-337;
 * kernel src/u15-kernels.metal:186-255): key j attends to query i iff
 * t_index[j] == t_index[q_offset + i] or j <= q_offset + i (causal across
 * t blocks, bidirectional within one; src/u15-ref.cc:179-192).  t_index is
 * device int32 covering positions [0, max(tk, q_offset + tq)). */
u15h_status u15h_sdpa_block_causal(u15h_ctx* ctx, u15h_stream stream,
                                   const u15h_bf16* q, const u15h_bf16* k,
                                   const u15h_bf16* v, u15h_bf16* out,
                                   const int32_t* t_index, int hq, int hkv,
                                   int tq, int tk, int d, int cap,
                                   int q_offset);

/* The same attention reading q and writing out TOKEN-major [tq][hq*d] (the
 * layout the projections produce and o_proj consumes), which folds away the
 * transpose_thd before and the transpose_htd after the reference's head-
 * major kernels (src/u15-backbone.cc:208, 241).  No reference counterpart.
 * mode 0 bidirectional, 1 causal, 2 block-causal (t_index as above). */
u15h_status u15h_attention_token_major(u15h_ctx* ctx, u15h_stream stream,
                                       const u15h_bf16* q, const u15h_bf16* k,
                                       const u15h_bf16* v, u15h_bf16* out,
                                       const int32_t* t_index, int hq,
                                       int hkv, int tq, int tk, int d,
                                       int cap, int q_offset, int mode);

/* Replace MetalOps::transpose_thd / transpose_htd / transpose_into_cache
 * (src/u15-metal-ops.h:339-355): [T][H][D] <-> [H][T][D], and [T][H*D]
 * into a cache [H][cap][D] at token offset `offset`.  D % 8 == 0. */
u15h_status u15h_transpose_thd(u15h_ctx* ctx, u15h_stream stream,
                               const u15h_bf16* in, u15h_bf16* out, int T,
                               int H, int D);
u15h_status u15h_transpose_htd(u15h_ctx* ctx, u15h_stream stream,
                               const u15h_bf16* in, u15h_bf16* out, int T,
                               int H, int D);
u15h_status u15h_transpose_into_cache(u15h_ctx* ctx, u15h_stream stream,
                                      const u15h_bf16* in, u15h_bf16* cache,
                                      int T, int H, int D, int cap,
                                      int offset);

/* ------------------------------------------------------------------ */
/* The layer norms and the residual add (either side of the projections) */
/* ------------------------------------------------------------------ */

/* Replaces MetalOps::rms_norm(enc, x, w, y, rows, dim, eps)
 * (src/u15-metal-ops.h:158-166, .cc:494-505), the whole-row RMSNorm with
 * gain that feeds q|k|v (input_layernorm) and gate|up
 * (post_attention_layernorm) in U15Backbone::layer_step_
 * (src/u15-backbone.cc:196, 249): y = bf16((x * inv) * w) with inv =
 * 1/sqrt(mean(x^2) + eps), the sum in f32 (the reference's CPU form,
 * src/u15-ref.cc:15-31, accumulates in double).  x, y [rows][dim], w [dim],
 * bf16.  The reference's `fast` flag picks between two reductions of its
 * library with one contract; there is one here.  Limits: dim % 8 == 0,
 * dim <= 16384, 16-byte aligned operands, eps >= 0; y may equal x. */
u15h_status u15h_rms_norm(u15h_ctx* ctx, u15h_stream stream,
                          const u15h_bf16* x, const u15h_bf16* w,
                          u15h_bf16* y, int rows, int dim, float eps);

/* The int8 tier's input in the same pass: the norm above, then the row's
 * bf16 results quantised per token (u15h_quant_rows_i8's scale and codes,
 * bit for bit, as if it ran on y).  q [rows][dim] int8, s [rows] f32; y
 * [rows][dim] is written only when not NULL.  No reference counterpart:
 * it saves the quantiser's separate read of the normed rows.  Limits as
 * u15h_rms_norm's. */
u15h_status u15h_rms_norm_quant_i8(u15h_ctx* ctx, u15h_stream stream,
                                   const u15h_bf16* x, const u15h_bf16* w,
                                   int rows, int dim, float eps,
                                   u15h_bf16* y, int8_t* q, float* s);

/* The norms of a two-group pass in one launch, with the residual add
 * before them.  No reference counterpart as one call: U15Backbone::
 * layer_step_ issues add(x, proj) and then rms_norm(x, post_ln)
 * (src/u15-backbone.cc:245-249), and, across layers, the last add then
 * the next layer's input norm (:256, :196), one expert per pass.  For rows
 * [0, M_und) with w_und and the next M_gen rows with w_gen:
 *   if delta: x <- bf16(x + delta)                 (the residual stream)
 *   y <- bf16((x * inv) * w)  as u15h_rms_norm     (when y is not NULL)
 *   q, s <- the per-token int8 codes of those bf16 values, as
 *           u15h_rms_norm_quant_i8                 (when q is not NULL)
 * Bits equal u15h_add, then u15h_rms_norm per group (and
 * u15h_quant_rows_i8).  x, delta, y [M_und + M_gen][dim] bf16; q int8,
 * s [rows] f32 (both or neither); at least one of y, q.  y must not be x
 * when delta is given.  Limits as u15h_rms_norm's. */
u15h_status u15h_mot_rms_norm(u15h_ctx* ctx, u15h_stream stream,
                              u15h_bf16* x, const u15h_bf16* delta, int M_und,
                              int M_gen, int dim, const u15h_bf16* w_und,
                              const u15h_bf16* w_gen, float eps, u15h_bf16* y,
                              int8_t* q, float* s);

/* Replaces MetalOps::add(enc, dst, src, n) (src/u15-metal-ops.h:361-363,
 * .cc:974-982; kernel u15_add, src/u15-kernels.metal:496-504), the
 * residual add of layer_step_ (src/u15-backbone.cc:245, 256):
 * dst[i] = bf16(f32(dst[i]) + f32(src[i])).  Any n and alignment. */
u15h_status u15h_add(u15h_ctx* ctx, u15h_stream stream, u15h_bf16* dst,
                     const u15h_bf16* src, int64_t n);

/* ------------------------------------------------------------------ */
/* SwiGLU                                                              */
/* ------------------------------------------------------------------ */

/* Replaces MetalOps::swiglu (src/u15-metal-ops.cc:634-646):
 * out[i] = silu(gate[i]) * up[i], bf16 in/out, fp32 math
 * (reference formula: src/u15-ref.cc:51-58 and :303-304). */
u15h_status u15h_swiglu(u15h_ctx* ctx, u15h_stream stream,
                        const u15h_bf16* gate, const u15h_bf16* up,
                        u15h_bf16* out, int64_t n);

/* The int8 tier's input to the down projection in one pass: h =
 * swiglu(gate, up) as u15h_swiglu, then its per-token int8 codes q
 * [rows][inter] and scales s [rows] as u15h_quant_rows_i8 on h (bit for
 * bit).  h [rows][inter] is written only when not NULL.  No reference
 * counterpart: it saves writing h and reading it back.  Limits: inter %
 * 8 == 0, inter <= 16384, 16-byte aligned operands. */
u15h_status u15h_swiglu_quant_i8(u15h_ctx* ctx, u15h_stream stream,
                                 const u15h_bf16* gate, const u15h_bf16* up,
                                 int rows, int inter, u15h_bf16* h, int8_t* q,
                                 float* s);

/* Replaces MetalOps::swiglu_fused(enc, x, w_fused, y, M, K, inter)
 * (src/u15-metal-ops.h:121-135, src/u15-metal-ops.cc:470-491) with the
 * reference's weight layout: w_fused[2*inter][K] ROW-INTERLEAVED, row 2i =
 * gate row i, row 2i+1 = up row i.  y[M][inter] = silu(x.gate^T) *
 * (x.up^T), gate and up rounded to bf16 before the product.
 * Limits: K % 8 == 0, inter % 8 == 0. */
u15h_status u15h_swiglu_fused(u15h_ctx* ctx, u15h_stream stream,
                              const u15h_bf16* x, const u15h_bf16* w_fused,
                              u15h_bf16* y, int M, int K, int inter);

/* The same product in grouped form: one launch computes, for
 * each row group, h[M][I] = silu(x.Wg^T) * (x.Wu^T) with the gate and up
 * weights given SEPARATELY (no interleaved repack needed: each output tile
 * reads the matching gate and up rows).  Rounding follows the unfused
 * reference sequence: gate and up are rounded to bf16 first, then the
 * silu-product is computed in fp32 and rounded to bf16.
 * Limits: K % 8 == 0, I % 8 == 0. */
u15h_status u15h_mot_gate_up_swiglu(u15h_ctx* ctx, u15h_stream stream,
                                    const u15h_bf16* x, int M_und, int M_gen,
                                    int K, const u15h_bf16* wg_und,
                                    const u15h_bf16* wu_und,
                                    const u15h_bf16* wg_gen,
                                    const u15h_bf16* wu_gen, u15h_bf16* h,
                                    int I);

/* ------------------------------------------------------------------ */
/* int8 tier                                                           */
/* ------------------------------------------------------------------ */

/* Replaces MetalOps::enable_i8_gemm(bool want) (src/u15-metal-ops.h:71-92,
 * src/u15-metal-ops.cc:262-275).  Returns whether the tier is ON afterwards,
 * which is not the same as `want`: the environment variable U15H_I8_GEMM
 * ("0"/"1") overrides either way.  When on, u15h_linear() routes qualifying
 * shapes through the int8 path. */
int  u15h_enable_i8_gemm(u15h_ctx* ctx, int want);
/* Replaces MetalOps::release_i8_scratch (src/u15-metal-ops.h:94-98). */
void u15h_release_i8_scratch(u15h_ctx* ctx);
/* Row floor of the int8 route of u15h_linear (default 1024, env
 * U15H_I8_MIN_M); the reference's tier declines below ~1k rows
 * (src/u15-metal-ops.h:71-83). */
int  u15h_i8_min_m(const u15h_ctx* ctx);

/* Symmetric per-row int8 quantisation of a bf16 matrix [rows][K]:
 *   s[r] = max_k |x[r][k]| / 127            (fp32, correctly rounded)
 *   q[r][k] = clamp(round_half_away(x[r][k] / s[r]), -127, 127)
 *   (s[r] == 0 gives q = 0)
 * Used both for per-token activations and for per-output-channel weights
 * (a weight [N][K] quantised per row is quantised per output channel).
 * No reference counterpart computes these numerics (the reference's int8
 * tier uses per-512-group scales inside an unvendored library); the
 * rounding rule is the one the reference's quantisation fixture uses
 * (std::lround, tests/u15-m5-test.cc:295). */
u15h_status u15h_quant_rows_i8(u15h_ctx* ctx, u15h_stream stream,
                               const u15h_bf16* x, int rows, int K,
                               int8_t* q, float* s);

/* One int8 projection: quantised weights of both sets, their per-channel
 * scales, and the output.  `y` is int32 [M][N] for u15h_mot_gemm_i8_i32
 * and bf16 [M][N] for u15h_mot_gemm_i8. */
typedef struct {
  const int8_t* wq_und;  /* [N][K] */
  const float*  sw_und;  /* [N]    */
  const int8_t* wq_gen;  /* [N][K] */
  const float*  sw_gen;  /* [N]    */
  void*         y;
  int           N;
} u15h_mot_proj_i8;

/* int8 x int8 -> raw int32 accumulators, grouped like u15h_mot_linear.
 * Exact: |acc| <= 127*127*K < 2^31 for K <= 133143.  Scales are ignored.
 * Limits: K % 128 == 0, K <= 131072, N % 8 == 0. */
u15h_status u15h_mot_gemm_i8_i32(u15h_ctx* ctx, u15h_stream stream,
                                 const int8_t* xq, int M_und, int M_gen,
                                 int K, const u15h_mot_proj_i8* proj,
                                 int nproj);

/* int8 GEMM with the fused dequant epilogue:
 *   y[m][n] = bf16_rne( ((float)acc[m][n] * sx[m]) * sw[n] )
 * (int32 -> fp32 conversion round-to-nearest-even, two fp32 multiplies in
 * that order, then round-to-nearest-even to bf16).
 * Replaces the int8 route of MetalOps::linear_mma_
 * (src/u15-metal-ops.cc:300-306) with BASELINE numerics: per-token
 * activation scales, per-output-channel weight scales.
 * Limits as u15h_mot_gemm_i8_i32. */
u15h_status u15h_mot_gemm_i8(u15h_ctx* ctx, u15h_stream stream,
                             const int8_t* xq, const float* sx, int M_und,
                             int M_gen, int K, const u15h_mot_proj_i8* proj,
                             int nproj);

/* ------------------------------------------------------------------ */
/* The resident MoT layer stack                                        */
/* ------------------------------------------------------------------ */

/* The seven projections of an expert layer, in the order
 * U15Backbone::layer_step_ issues them (src/u15-backbone.cc:197-254), and
 * the two experts of a MotLayer (src/u15-weights.h:113-116). */
typedef enum {
  U15H_PROJ_Q = 0, U15H_PROJ_K = 1, U15H_PROJ_V = 2, U15H_PROJ_O = 3,
  U15H_PROJ_GATE = 4, U15H_PROJ_UP = 5, U15H_PROJ_DOWN = 6, U15H_NPROJ = 7
} u15h_proj_id;
typedef enum { U15H_UND = 0, U15H_GEN = 1 } u15h_expert;

/* A host-side table of device pointers: n_layers MotLayers, each with the
 * seven projection matrices of both experts (the reference's
 * MotLayer{und, gen} of ExpertLayer, src/u15-weights.h:97-117), bf16
 * [N][K] and optionally their int8-tier copies (per-output-channel codes
 * [N][K] + f32 scales [N], as u15h_quant_rows_i8 makes them).  The
 * caller owns the weight memory and keeps it resident; the stack holds
 * pointers only.  Shapes follow LlmConfig (src/u15-config.h:40-63):
 * q [heads*head_dim][hidden], k/v [kv_heads*head_dim][hidden],
 * o [hidden][heads*head_dim], gate/up [inter][hidden], down [hidden][inter]. */
typedef struct u15h_stack u15h_stack;

u15h_status u15h_stack_create(int n_layers, int hidden, int heads,
                              int kv_heads, int head_dim, int inter,
                              u15h_stack** out);
void        u15h_stack_destroy(u15h_stack* st);

/* Maps one of the reference's tensor names to its slot, by the rule of
 * U15Weights' layer binder (src/u15-weights.cc:539-578):
 *   language_model.model.layers.<i>.self_attn.{q,k,v,o}_proj[_mot_gen]
 *   language_model.model.layers.<i>.mlp[_mot_gen].{gate,up,down}_proj
 * each optionally followed by ".weight".  The attention matrices suffix
 * the TENSOR (q_proj_mot_gen), the MLP suffixes the MODULE
 * (mlp_mot_gen.gate_proj).  Host only.  EINVAL for any other name (norms,
 * embeddings, a malformed layer index). */
u15h_status u15h_weight_slot(const char* name, int* layer, int* expert,
                             int* proj);

/* Binds a bf16 matrix [N][K] (device memory, 16-byte aligned) to the slot
 * a reference tensor name maps to.  EINVAL for an unknown name or a layer
 * index outside the stack. */
u15h_status u15h_stack_bind(u15h_stack* st, const char* name,
                            const u15h_bf16* w);
/* Binds the int8-tier copy of a slot: wq [N][K] int8, sw [N] f32. */
u15h_status u15h_stack_bind_i8(u15h_stack* st, const char* name,
                               const int8_t* wq, const float* sw);
/* The same two bindings by index (either pointer group may be NULL to
 * leave it unchanged). */
u15h_status u15h_stack_set(u15h_stack* st, int layer, int expert, int proj,
                           const u15h_bf16* w, const int8_t* wq,
                           const float* sw);

/* The matrices a pass needs are bound (the projection half of
 * ExpertLayer::complete, src/u15-weights.cc:333-339): every layer's seven
 * matrices of the und expert (need_und) and/or the gen expert (need_gen),
 * bf16 (tier 0) or int8 (tier 1).  On EINVAL, `missing` (if not NULL)
 * receives the reference name of the first unbound matrix, or, for the
 * int8 tier, why the stack's widths do not fit it (every projection's K
 * must be a multiple of 128 and at most 131072). */
u15h_status u15h_stack_check(const u15h_stack* st, int need_und,
                             int need_gen, int tier, char* missing,
                             size_t missing_cap);

/* The activations of one layer's projections: the reference's layer
 * scratch (_normed, _q, _k, _v, _attn_t, _gate, _up, _ff, _proj;
 * src/u15-backbone.cc:197-254), rows [0, M_und) und, then M_gen gen. */
typedef struct {
  const u15h_bf16* x;     /* [M][hidden]          q|k|v input            */
  u15h_bf16*       q;     /* [M][heads*head_dim]                         */
  u15h_bf16*       k;     /* [M][kv_heads*head_dim]                      */
  u15h_bf16*       v;     /* [M][kv_heads*head_dim]                      */
  const u15h_bf16* attn;  /* [M][heads*head_dim]  o input                */
  u15h_bf16*       o;     /* [M][hidden]                                 */
  const u15h_bf16* x2;    /* [M][hidden]          gate|up input          */
  u15h_bf16*       gate;  /* [M][inter] (unused with U15H_FUSED_SWIGLU)  */
  u15h_bf16*       up;    /* [M][inter] (unused with U15H_FUSED_SWIGLU)  */
  u15h_bf16*       h;     /* [M][inter] down input; written by the fused
                             gate|up step                                */
  u15h_bf16*       down;  /* [M][hidden]                                 */
  int8_t*          xq;    /* int8 tier: [M][max(hidden, heads*head_dim,
                             inter)] activation codes (caller scratch)   */
  float*           sx;    /* int8 tier: [M] per-token scales            */
} u15h_layer_io;

/* Steps of a layer (bit mask) and options. */
#define U15H_STEP_QKV      1   /* q|k|v = x . {Wq|Wk|Wv}^T, one launch  */
#define U15H_STEP_O        2   /* o = attn . Wo^T                        */
#define U15H_STEP_GATE_UP  4   /* gate|up = x2 . {Wg|Wu}^T, one launch   */
#define U15H_STEP_DOWN     8   /* down = h . Wd^T                        */
#define U15H_STEP_ALL     15
#define U15H_TIER_BF16     0
#define U15H_TIER_I8       1   /* per-token quantisation of each step's
                                  input into xq/sx, then the int8 GEMM
                                  with the fused dequant                 */
#define U15H_FUSED_SWIGLU  1   /* flag: the gate|up step writes h =
                                  silu(gate) * up (fused epilogue; bf16
                                  tier) instead of gate and up           */

/* One layer's projection steps, both experts per launch: the projection
 * half of U15Backbone::layer_step_ (src/u15-backbone.cc:174-257), whose
 * norms, attention and residual adds stay with the caller between the
 * steps.  Each step is one grouped launch over both weight sets. */
u15h_status u15h_stack_layer(u15h_ctx* ctx, u15h_stream stream,
                             const u15h_stack* st, int layer,
                             const u15h_layer_io* io, int M_und, int M_gen,
                             int steps, int tier, int flags);

/* Every layer's projection steps in order, layer after layer, on the
 * same io buffers: forward_many's layer loop (src/u15-backbone.cc:
 * 386-426) with the non-projection ops of layer_step_ left out.  There is
 * no stop hook between layers: the reference's cooperative per-layer stop
 * (src/u15-backbone.cc:394-397) belongs to a caller that loops
 * u15h_stack_layer itself and checks its flag between the calls.  Only
 * the last layer's outputs survive in io. */
u15h_status u15h_stack_forward(u15h_ctx* ctx, u15h_stream stream,
                               const u15h_stack* st, const u15h_layer_io* io,
                               int M_und, int M_gen, int tier, int flags);

/* ---- the whole layer ------------------------------------------------ */

/* The six norm vectors of an expert layer (ExpertLayer's input_ln,
 * post_ln, q_norm, k_norm, q_norm_hw, k_norm_hw; src/u15-weights.h:97-110):
 * input_ln and post_ln [hidden], the head norms [head_dim / 2]. */
typedef enum {
  U15H_NORM_INPUT = 0, U15H_NORM_POST = 1, U15H_NORM_Q = 2, U15H_NORM_K = 3,
  U15H_NORM_Q_HW = 4, U15H_NORM_K_HW = 5, U15H_NNORM = 6
} u15h_norm_id;

/* Maps a reference norm name to its slot, by the layer binder's rule
 * (src/u15-weights.cc:549-566):
 *   language_model.model.layers.<i>.input_layernorm[_mot_gen]
 *   language_model.model.layers.<i>.post_attention_layernorm[_mot_gen]
 *   language_model.model.layers.<i>.self_attn.{q,k}_norm[_hw][_mot_gen]
 * each optionally followed by ".weight" (the layernorms suffix the
 * MODULE, the head norms the TENSOR).  Host only; EINVAL for any other
 * name. */
u15h_status u15h_norm_slot(const char* name, int* layer, int* expert,
                           int* which);
/* Binds a bf16 norm vector (device memory, 16-byte aligned) by name or by
 * index. */
u15h_status u15h_stack_bind_norm(u15h_stack* st, const char* name,
                                 const u15h_bf16* w);
u15h_status u15h_stack_set_norm(u15h_stack* st, int layer, int expert,
                                int which, const u15h_bf16* w);
/* ExpertLayer::complete (src/u15-weights.cc:333-339) in full: the seven
 * matrices (bf16, or the int8 copies for tier 1) and the six norm vectors
 * of every layer, for the und and/or gen expert.  On EINVAL `missing`
 * receives the first missing reference name. */
u15h_status u15h_stack_check_full(const u15h_stack* st, int need_und,
                                  int need_gen, int tier, char* missing,
                                  size_t missing_cap);

/* The buffers of one whole layer: the residual stream, the reference's
 * layer scratch, and the layer's K/V cache with the pass's position in it
 * (the state U15Backbone::layer_step_ reads, src/u15-backbone.cc:174-257).
 * Rows [0, M_und) und, then M_gen gen; M = M_und + M_gen. */
typedef struct {
  u15h_bf16*     x;        /* [M][hidden] the layer's input; on return
                              its output (x + attention + MLP)          */
  u15h_bf16*     normed;   /* [M][hidden] scratch (bf16 tier)            */
  u15h_bf16*     q;        /* [M][heads*head_dim] scratch                */
  u15h_bf16*     k;        /* [M][kv_heads*head_dim] scratch             */
  u15h_bf16*     v;        /* [M][kv_heads*head_dim] scratch             */
  u15h_bf16*     attn;     /* [M][heads*head_dim] scratch                */
  u15h_bf16*     proj;     /* [M][hidden] scratch (o, then down)         */
  u15h_bf16*     h;        /* [M][inter] scratch: SwiGLU output (bf16
                              tier); the gate output (int8 tier)         */
  u15h_bf16*     up;       /* [M][inter] scratch: the up output (int8
                              tier only)                                 */
  int8_t*        xq;       /* int8 tier: [M][max(hidden, heads*head_dim,
                              inter)] activation codes                   */
  float*         sx;       /* int8 tier: [M] per-token scales            */
  u15h_bf16*     k_cache;  /* this layer's [kv_heads][cap][head_dim]     */
  u15h_bf16*     v_cache;
  int            cap;      /* cache capacity in tokens                   */
  int            kv_off;   /* the pass's first position in the cache     */
  int            kv_len;   /* keys attended, kv_off + M <= kv_len <= cap */
  int            mode;     /* attention mask: 0 bidirectional, 1 causal,
                              2 block-causal                             */
  const int32_t* t_index;  /* block-causal: [max(kv_len, kv_off + M)]    */
  const float*   cos_tab;  /* [M][head_dim] f32, u15h_build_rope_tables  */
  const float*   sin_tab;
  int            d_t, d_h; /* the RoPE ranges [t | h | w]                */
  float          eps;      /* the norms' epsilon                         */
} u15h_layer_full_io;

/* One whole decoder layer, both experts per launch: U15Backbone::
 * layer_step_ (src/u15-backbone.cc:174-257) for a pass of M_und und and
 * M_gen gen tokens.  The steps, in launches:
 *   normed = rms_norm(x) (each group its input_ln)    u15h_mot_rms_norm
 *   q | k | v                                         u15h_mot_linear
 *   q, k norm + RoPE; k, v into the cache at kv_off   u15h_mot_attention_prologue
 *   attn = attention(q, cache[0, kv_len))             u15h_attention_token_major
 *   proj = o(attn)                                    u15h_mot_linear
 *   x += proj; normed = rms_norm(x) (post_ln)         u15h_mot_rms_norm
 *   h = silu(gate) * up                               u15h_mot_gate_up_swiglu
 *   proj = down(h); x += proj                         u15h_mot_linear, u15h_add
 * Tier 1 (int8): the norms write the activation codes (u15h_mot_rms_norm
 * with codes), attn is quantised, gate|up write gate and up, and SwiGLU
 * writes the down projection's codes (u15h_swiglu_quant_i8); every
 * projection is u15h_mot_gemm_i8.  Requires the one-launch prologue's
 * shapes (u15h_mot_attention_prologue) and the stack complete for the
 * experts with rows (u15h_stack_check_full).  Every argument is checked
 * before the first launch.  No reference counterpart as one call; the
 * layer loop with its per-layer stop stays with the caller. */
u15h_status u15h_stack_layer_full(u15h_ctx* ctx, u15h_stream stream,
                                  const u15h_stack* st, int layer,
                                  const u15h_layer_full_io* io, int M_und,
                                  int M_gen, int tier);

/* Whole layers [first, first + count) in order, one pass through each:
 * forward_many's layer loop (src/u15-backbone.cc:386-426) over
 * u15h_stack_layer_full, on one io.  Layer first + i attends its own cache,
 * k_caches[i] / v_caches[i] ([kv_heads][cap][head_dim] each; the io's
 * k_cache and v_cache are not read); cap, kv_off, kv_len, mode and the
 * RoPE tables are the pass's, the same for every layer.  Between two
 * layers, the first's residual add and the second's input norm run as one
 * pass (u15h_mot_rms_norm with the down output as the residual), which
 * gives the same bits as count calls of u15h_stack_layer_full.  Every
 * layer's arguments are checked before the first launch.  There is no
 * stop hook between layers: a caller that needs the reference's
 * cooperative per-layer stop (src/u15-backbone.cc:394-397) loops
 * u15h_stack_layer_full itself. */
u15h_status u15h_stack_forward_full(u15h_ctx* ctx, u15h_stream stream,
                                    const u15h_stack* st, int first, int count,
                                    const u15h_layer_full_io* io,
                                    u15h_bf16* const* k_caches,
                                    u15h_bf16* const* v_caches, int M_und,
                                    int M_gen, int tier);

/* ------------------------------------------------------------------ */
/* profiling                                                           */
/* ------------------------------------------------------------------ */

/* Profiling hook; no counterpart in the reference (whose perf test times
 * whole command buffers, tests/u15-perf-test.cc:63-110).  `event` is a
 * hipEvent_t: the next GEMM launched through this context completes it
 * with the GEMM kernel's own end timestamp (the event is bound to the
 * kernel's dispatch, hipExtLaunchKernel; no extra packet on the stream),
 * before any split-K reduction kernel, then forgets it.  NULL cancels. */
u15h_status u15h_profile_next_gemm(u15h_ctx* ctx, void* event);
/* The same with a second event taking the next GEMM kernel's START
 * timestamp (after any quantisation the same call launches first), so the
 * pair times exactly that kernel's execution, as a kernel trace does.
 * Either may be NULL.  No reference counterpart. */
u15h_status u15h_profile_bracket_next_gemm(u15h_ctx* ctx, void* before,
                                           void* after);
/* The general form (hipEvent_t pairs, each bound to one kernel's start and
 * end timestamps): the next quantiser launched through this context
 * (u15h_quant_rows_i8, as the stack's int8 steps call it), the next GEMM
 * kernel, and that GEMM call's reduction kernel (split-K tail or skinny
 * K shares).  A pair whose kernel does not run in that call is never
 * recorded.  Every pending pair is dropped once the next GEMM call has
 * launched.  Any may be NULL.  No reference counterpart: it lets a caller
 * sum exactly the kernel time of its own timed steps. */
u15h_status u15h_profile_next_kernels(u15h_ctx* ctx, void* quant_start,
                                      void* quant_end, void* gemm_start,
                                      void* gemm_end, void* reduce_start,
                                      void* reduce_end);

/* ------------------------------------------------------------------ */
/* per-token routing                                                   */
/* ------------------------------------------------------------------ */

/* Per-token expert routing for interleaved token types (the grouped entry
 * points above assume und rows first, then gen rows).  Given
 * expert[M] (0 = und / base weights, 1 = gen / _mot_gen weights; host
 * memory), writes perm[M] (host memory) such that rows perm[0..M_und) are
 * the und tokens and perm[M_und..M) the gen tokens, each in their original
 * order (a stable partition), and returns the counts.  The reference makes
 * this split by pass (src/u15-generator.cc:379 prefill = und,
 * :548 denoise = gen); this is the row-level equivalent. */
u15h_status u15h_route_rows(const uint8_t* expert, int M, int32_t* perm,
                            int* M_und, int* M_gen);

/* Gather rows into expert order: dst[i][:] = src[perm[i]][:]
 * (bf16, row length `cols`, perm in device memory). */
u15h_status u15h_gather_rows(u15h_ctx* ctx, u15h_stream stream,
                             const u15h_bf16* src, const int32_t* perm,
                             int M, int cols, u15h_bf16* dst);
/* Scatter rows back to token order: dst[perm[i]][:] = src[i][:]. */
u15h_status u15h_scatter_rows(u15h_ctx* ctx, u15h_stream stream,
                              const u15h_bf16* src, const int32_t* perm,
                              int M, int cols, u15h_bf16* dst);

#ifdef __cplusplus
}  /* extern "C" */
#endif

#endif /* U15H_H */
