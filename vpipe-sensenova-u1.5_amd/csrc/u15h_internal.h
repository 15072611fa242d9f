// u15h_internal.h -- shared definitions between the C-ABI layer and the
// gfx950 kernels.  Not installed; the public surface is include/u15h.h.
#ifndef U15H_INTERNAL_H
#define U15H_INTERNAL_H

#include <hip/hip_runtime_api.h>
#include <stdint.h>

#include "u15h.h"

namespace u15h {

// Output tile of one workgroup and the K bytes staged per LDS stage.
// 128 bytes of K is 64 bf16 or 128 int8: both element types share one
// LDS byte layout and one load schedule; only the MFMA differs.
constexpr int kBM = 256;          // activation rows per tile
constexpr int kBN = 256;          // weight rows (output columns) per tile
constexpr int kKB = 128;          // bytes of K per stage
constexpr int kMaxProb = 8;       // problems (weight sets x projections) per launch

// What the epilogue does with the fp32 / int32 accumulators.
enum class Epi : int {
  kBf16 = 0,         // y = bf16_rne(acc (+ bias))                 [bf16 GEMM]
  kI32 = 1,          // y = acc (int32)                            [int8 GEMM]
  kDequantBf16 = 2,  // y = bf16_rne((float(acc)*sa[m])*sw[n] (+ bias))
  kSwiglu = 3,       // y = bf16(silu(bf16(g)) * bf16(u)), gate/up tile pairs
};

// One GEMM of a batch: y[rows][n] = a[rows][K] . w[n][K]^T.
struct GemmProblem {
  const void*     a;      // activation rows [rows][K]
  const void*     w;      // weight rows [n][K]  (gate rows for kSwiglu)
  const void*     w2;     // up rows [n][K] for kSwiglu, else unused
  void*           y;      // output rows, ldy elements apart
  const uint16_t* bias;   // bf16 [n] or null
  const float*    sa;     // per-row scale [rows] (kDequantBf16)
  const float*    sw;     // per-column scale [n] (kDequantBf16)
  int rows;               // activation rows of this problem
  int n;                  // output columns of this problem
  int wld;                // bytes between consecutive weight rows
  int ldy;                // output row pitch in elements
  int tiles_m;            // ceil(rows / kBM)
  int tiles_n;            // ceil(n / tile columns)
  int tile_begin;         // first linear tile index of this problem
};

// A batch of problems run by one launch.  Tiles are numbered problem by
// problem.  Tiles [split_begin, total_tiles) -- the ones that would
// otherwise leave most of the GPU idle in a last, partial round -- run as
// `split` workgroups each, every one covering a contiguous share of the K
// stages and writing its raw accumulators to `ws`; a second, small kernel
// sums the shares and applies the epilogue.
struct GemmBatch {
  GemmProblem p[kMaxProb];
  int nprob;
  int kbytes;             // bytes per activation / weight row (K * elem size)
  int total_tiles;
  int split_begin;        // == total_tiles when nothing is split
  int split;              // K shares per split tile (1 = no split)
  void* ws;               // [(tile - split_begin) * split + share][kBM][kBN]
};

// Workgroups a batch launches.
__host__ __device__ inline int grid_blocks(const GemmBatch& b)
{
  return b.split_begin + (b.total_tiles - b.split_begin) * b.split;
}
// Bytes of partial-sum workspace a batch needs.
inline size_t split_ws_bytes(const GemmBatch& b)
{
  return (size_t)(b.total_tiles - b.split_begin) * b.split * kBM * kBN * 4;
}

// Kernel launchers (u15h_kernels.hip).  All are asynchronous on `s`.
// How the GEMM kernel is launched: `waves` is the workgroup shape, 4 (one
// wave per SIMD, 128x128 per wave) or 8 (two per SIMD, 128x64 per wave);
// `cus` > 0 caps the grid at that many workgroups (persistent: one per CU),
// 0 launches one workgroup per work item.
struct GemmShape {
  int waves;
  int cus;
  // 8-wave workgroup MFMA shape: 1 = 16x16 for both types (the measured
  // best, the default), 0 = 32x32 for both, -1 = 16x16 for int8 and 32x32
  // for bf16.  The 4-wave workgroup always runs 16x16.
  int mfma16;
};

// Profiling events bound to kernel dispatches (hipExtLaunchKernel: each
// takes its kernel's start or end timestamp; no packet of its own).  Null
// members are not recorded.
struct GemmEvents {
  hipEvent_t before = nullptr;        // GEMM kernel start
  hipEvent_t after = nullptr;         // GEMM kernel end
  hipEvent_t red_before = nullptr;    // split-K / skinny reduction start
  hipEvent_t red_after = nullptr;     // its end
};
hipError_t launch_gemm_bf16(const GemmBatch& b, Epi epi, const GemmShape& g,
                            hipStream_t s, const GemmEvents& ev);

// The skinny bf16 GEMM for problems of at most kSkinnyMaxRows rows: one
// workgroup per column block (skinny_cols(max_rows, qbits) output columns:
// 16 up to 16 rows, 64 above; or twice that where skinny_wide_ok, 32 per
// wave) and K share.  Problem p's column blocks are
// [cb_begin, cb_begin + ceil(n / cols)); with S > 1 the shares' fp32
// partial sums go to ws + ws_off as [S][rows][n] and a second kernel adds
// them in share order, the bias, and rounds to bf16.
constexpr int kSkinnyMaxRows = 128;
constexpr int skinny_cols(int max_rows, int) { return max_rows <= 16 ? 16 : 64; }
constexpr bool skinny_wide_ok(int max_rows, int qbits) { return qbits == 0 && max_rows > 64; }
struct SkinnyProblem {
  const void*     a;      // activation rows [rows][K] (bf16)
  const void*     w;      // weight rows [n][K] (bf16), or the pack's codes
  const uint16_t* qs;     // affine pack: scales bf16 [n][K / group]
  const uint16_t* qb;     // affine pack: biases bf16 [n][K / group]
  void*           y;      // output rows [rows][ldy] (bf16)
  const uint16_t* bias;   // bf16 [n] or null
  int rows;
  int n;
  int ldy;
  int cb_begin;           // first column block of this problem
  size_t ws_off;          // floats from ws to this problem's partial sums
};
struct SkinnyBatch {
  SkinnyProblem p[kMaxProb];
  int nprob;
  int kbytes;             // bytes per row of K (K * 2; a multiple of 128)
  int split;              // K shares per column block (S)
  int cols;               // output columns per block (skinny_cols)
  int total_cb;           // column blocks over all problems
  int max_rows;           // largest problem (picks the kernel build)
  int qbits;              // 0: bf16 weights; 4 or 8: affine-quantized pack
  int qgroup;             // the pack's group (32 or 64)
  float* ws;              // partial sums when split > 1
};
// Floats of partial-sum workspace a skinny batch needs.
inline size_t skinny_ws_floats(const SkinnyBatch& b)
{
  if (b.split <= 1) { return 0; }
  size_t f = 0;
  for (int i = 0; i < b.nprob; ++i) {
    f += (size_t)b.split * b.p[i].rows * b.p[i].n;
  }
  return f;
}
// The skinny kernels: bf16 weights, or (qbits 4 / 8) an affine-quantized
// pack dequantised in registers to the expansion's bf16 weights.
hipError_t launch_skinny_bf16(const SkinnyBatch& b, hipStream_t s,
                              const GemmEvents& ev);
hipError_t launch_gemm_i8(const GemmBatch& b, Epi epi, const GemmShape& g,
                          hipStream_t s, const GemmEvents& ev);
hipError_t launch_quant_rows_i8(const uint16_t* x, int rows, int K,
                                int8_t* q, float* sc, hipStream_t s,
                                hipEvent_t start = nullptr,
                                hipEvent_t end = nullptr);
// Whole-row RMSNorm with gain, dim <= 16384, dim % 8 == 0, operands
// 16-byte aligned: with d not null x = bf16(x + d) first (stored back);
// y = bf16((x * inv) * w), w = w_und for rows below m_und, else w_gen.
// With q not null it also quantises the row's bf16 results to int8 codes q
// and scale sc (y then optional), equal to launch_quant_rows_i8 on y.
hipError_t launch_rms_norm(uint16_t* x, const uint16_t* d, const uint16_t* w_und,
                           const uint16_t* w_gen, int m_und, int rows, int dim,
                           float eps, uint16_t* y, int8_t* q, float* sc,
                           hipStream_t s);
// h = swiglu(gate, up) rows [rows][dim] and their per-token int8 codes q,
// scale sc (equal to launch_swiglu then launch_quant_rows_i8); h optional.
// dim % 8 == 0, dim <= 16384, operands 16-byte aligned.
hipError_t launch_swiglu_quant(const uint16_t* gate, const uint16_t* up, int rows,
                               int dim, uint16_t* h, int8_t* q, float* sc,
                               hipStream_t s);
// dst[i] = bf16(f32(dst[i]) + f32(src[i])), any n and alignment.
hipError_t launch_add_bf16(uint16_t* dst, const uint16_t* src, int64_t n,
                           hipStream_t s);
hipError_t launch_swiglu(const uint16_t* g, const uint16_t* u, uint16_t* o,
                         int64_t n, hipStream_t s);
hipError_t launch_dequant_affine(const uint32_t* codes, const uint16_t* sc,
                                 const uint16_t* bi, int bits, int group, int N,
                                 int K, uint16_t* w, hipStream_t s);
hipError_t launch_split_norm_rope(uint16_t* x, const uint16_t* w_t,
                                  const uint16_t* w_hw, const float* cosf,
                                  const float* sinf, int rows, int H, int D,
                                  int d_t, int d_h, float eps, bool norm,
                                  bool rope, hipStream_t s);
// Attention operands.  q and out are addressed as q[h * q_head + t * q_tok
// + c] (head-major: q_head = tq*d, q_tok = d; token-major: q_head = d,
// q_tok = hq*d); k and v are caches [hkv][cap][d].  mode 0 bidirectional,
// 1 causal, 2 block-causal (t_index).
struct AttnArgs {
  const uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* out;
  const int32_t* t_index;
  long long q_head, q_tok, o_head, o_tok;
  int hq, hkv, tq, tk, cap, q_offset, d, mode;
};
hipError_t launch_attention(const AttnArgs& a, hipStream_t s);
// The attention prologue of a two-group pass in one launch: q normed and
// rotated in place, k normed and rotated into its cache, v copied into its
// cache.  Shapes as split_norm_rope_vec_kernel's (d a power of two in
// [16, 512], d_t / 16 and d_h / 16 powers of two, d_h dividing d_t), every
// pointer 16-byte aligned.  Expert e's norm weights are w[e][0..3] = q_t,
// q_hw, k_t, k_hw; rows [0, m_und) take e = 0.
struct PrologueArgs {
  uint16_t* q;
  const uint16_t* k;
  const uint16_t* v;
  uint16_t* k_cache;
  uint16_t* v_cache;
  const uint16_t* w[2][4];
  const float* cosf;
  const float* sinf;
  int tokens, m_und, hq, hkv, d, d_t, d_h, cap, offset;
  float eps;
};
// Up to max_rpt (1, 2 or 4) heads of a token per thread.
hipError_t launch_attention_prologue(const PrologueArgs& a, hipStream_t s,
                                     int max_rpt);
hipError_t launch_transpose_rows(const uint16_t* src, uint16_t* dst, int T,
                                 int H, int D, long long src_t, long long src_h,
                                 long long dst_t, long long dst_h,
                                 hipStream_t s);
hipError_t launch_f16_to_bf16(const uint16_t* src, int64_t n, uint16_t* dst,
                              hipStream_t s);
hipError_t launch_bias_add(uint16_t* y, const uint16_t* b, int M, int N,
                           hipStream_t s);
hipError_t launch_f32_to_bf16(const float* src, int64_t n, uint16_t* dst,
                              hipStream_t s);
hipError_t launch_gather_rows(const uint16_t* src, const int32_t* perm,
                              int M, int cols, uint16_t* dst, bool scatter,
                              hipStream_t s);
// Forces every kernel's code object to load; false if any cannot.
bool kernels_loadable();

// The allocation-free entry point's split-K scratch: a static device array
// of this many bytes (one 256 x 256 tile of 4-byte sums per CU, up to 256
// CUs), looked up per device (at most kMaxScratchDevices of them).
constexpr size_t kNoAllocScratchBytes = (size_t)256 * kBM * kBN * 4;
constexpr int kMaxScratchDevices = 64;
// Device address of that array on `device`, which must be current on the
// first call for it; the result is kept per device.
hipError_t noalloc_scratch(int device, void** out);

// Sets the context's last-error text (u15h_last_error) and returns `st`;
// for host code of the library outside u15h_api.cc.
u15h_status set_error(u15h_ctx* ctx, u15h_status st, const char* msg);

// Tile columns per tile for an epilogue (kSwiglu tiles produce half).
constexpr int tile_cols(Epi e) { return e == Epi::kSwiglu ? kBN / 2 : kBN; }

}  // namespace u15h

#endif
