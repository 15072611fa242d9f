// u15h_kernels.hip -- gfx950 (CDNA4) kernels for the MoT projection GEMMs.
//
// The GEMM (mot_gemm_kernel) computes y = a . w^T for a batch of up to
// kMaxProb problems in ONE launch: the two MoT weight sets of a projection
// (und rows / gen rows) and several projections sharing an input (q, k, v;
// gate, up) all become entries of the batch's problem table, which rides in
// the kernel arguments.  Row-wise every problem is the reference's
// MetalOps::linear (src/u15-metal-ops.cc:327-346) with one weight set.
//
// Tile: 256 activation rows x 256 weight rows.  The default workgroup has
// 8 waves (2 per SIMD) in a 2x4 grid, each owning 128 activation rows x 64
// weight rows (wave w: rows 128*(w/4).., weight rows 64*(w%4)..; the two
// waves of a SIMD own the two row halves); the 4-wave workgroup owns
// 128x128 per wave, its 256 accumulator registers pinned in AGPRs by
// inline-asm MFMAs whose source order is the loop's schedule.  K is staged
// through LDS 128 bytes at a time (64 bf16 or 128 int8): both element types
// share one byte layout, one load schedule and one swizzle.  The MFMA is a
// trait (Mma*): by default the 16x16 shapes, v_mfma_f32_16x16x32_bf16 and
// v_mfma_i32_16x16x64_i8 (the 32x32 ones as an option), each taking 16
// bytes of K per lane.
//
// Operand order: the WEIGHT fragment is the MFMA's first operand, so the
// accumulator's rows are output columns.  A lane then holds groups of four
// consecutive output columns of one activation row, which the epilogue
// stores as one 8-byte (bf16) or 16-byte (int32) write.
//
// LDS: two stages of [256 weight rows | 256 activation rows] x 128 bytes.
// Row r's 16-byte chunk c sits at chunk position c ^ ((r >> 1) & 7), so
// the 16 rows a fragment read touches at one k-chunk land in 16 different
// bank groups, and the 8 lanes that write one row write all eight
// positions.
//
// Global loads use buffer resources sized to the tile's valid rows, so rows
// past M or N read as zero in hardware; a K tail (K not a multiple of the
// stage) is zero-filled by pushing the invalid chunks' offsets out of range.
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <mutex>
#include <type_traits>

#include "u15h_internal.h"

namespace u15h {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef unsigned u32x2_t __attribute__((ext_vector_type(2)));
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kStage = (kBM + kBN) * kKB;   // 64 KiB per LDS stage
constexpr int kRsrcWord3 = 0x00020000;      // raw buffer, 32-bit data format
constexpr int kOobOffset = 0x40000000;      // any offset past every resource
constexpr int kNonTemporal = 2;             // buffer cache policy: nt

// A buffer resource whose base and size are made explicitly wave-uniform,
// so it lives in SGPRs: a resource the compiler cannot prove uniform turns
// every buffer access into a readfirstlane loop over the lanes.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t
make_rsrc(const void* base, int bytes)
{
  const uint64_t p = reinterpret_cast<uint64_t>(base);
  const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)p);
  const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(p >> 32));
  const int n = __builtin_amdgcn_readfirstlane(bytes);
  return __builtin_amdgcn_make_buffer_rsrc(
      reinterpret_cast<void*>(((uint64_t)hi << 32) | lo), 0, n, kRsrcWord3);
}

__device__ __forceinline__ uint32_t
bf16_bits(float f)
{
  // Round to nearest even; the same rule the oracle and the reference's
  // weight loader use (finite values).
  const uint32_t u = __builtin_bit_cast(uint32_t, f);
  return (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
}

// Two floats as packed bf16 (lo in the low half) in one v_cvt_pk_bf16_f32:
// round to nearest even, the same result as bf16_bits for finite values.
__device__ __forceinline__ uint32_t
pack_bf16x2(float lo, float hi)
{
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  typedef float f32x2_t __attribute__((ext_vector_type(2)));
  return __builtin_bit_cast(uint32_t,
                            __builtin_convertvector((f32x2_t){lo, hi}, bf16x2_t));
}

// Bit reinterpretation through a by-value copy: __builtin_bit_cast applied
// directly to an element of an ext_vector_type accumulator reads the
// vector's first element, not the indexed one.
template <class To, class From>
__device__ __forceinline__ To
bits_as(From v)
{
  return __builtin_bit_cast(To, v);
}

__device__ __forceinline__ float
bf16_to_f32(uint32_t h)
{
  return __builtin_bit_cast(float, h << 16);
}

// MFMA flavours of the GEMM.  A fragment is kF x kF of D (weight rows x
// activation rows); one MFMA consumes kKBytes bytes of K per row, which
// lane l reads as 16 bytes at chunk l / kF of row l % kF (kG = 64 / kF
// chunks).  Lane l holds D column l % kF (an activation row) and, for
// accumulator element r, D row (r / 4) * 4 kG + 4 (l / kF) + r % 4: groups
// of four consecutive output columns, kE / 4 of them per fragment.
// The 16x16 shapes sustain ~15% more MFMA throughput than the 32x32 ones
// under the power cap with random operands (2089 vs 1716-1836 TFLOP/s
// bf16, 4404 vs 3750 TOPS int8, measured); they need twice the fragment
// registers for the same wave tile.
struct MmaBf16x16;
struct MmaI8x16;

struct MmaBf16 {                 // v_mfma_f32_32x32x16_bf16
  using acc_t = f32x16_t;
  using x16 = MmaBf16x16;
  static constexpr int kF = 32, kKBytes = 32, kE = 16;
  static constexpr bool kInt = false;
  __device__ static __forceinline__ acc_t run(i32x4_t a, i32x4_t b, acc_t c)
  {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(
        __builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
        0, 0, 0);
  }
};

struct MmaI8 {                   // v_mfma_i32_32x32x32_i8
  using acc_t = i32x16_t;
  using x16 = MmaI8x16;
  static constexpr int kF = 32, kKBytes = 32, kE = 16;
  static constexpr bool kInt = true;
  __device__ static __forceinline__ acc_t run(i32x4_t a, i32x4_t b, acc_t c)
  {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
  }
};

struct MmaBf16x16 {              // v_mfma_f32_16x16x32_bf16
  using acc_t = f32x4_t;
  static constexpr int kF = 16, kKBytes = 64, kE = 4;
  static constexpr bool kInt = false;
  __device__ static __forceinline__ acc_t run(i32x4_t a, i32x4_t b, acc_t c)
  {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(
        __builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b), c,
        0, 0, 0);
  }
};

struct MmaI8x16 {                // v_mfma_i32_16x16x64_i8
  using acc_t = i32x4_t;
  static constexpr int kF = 16, kKBytes = 64, kE = 4;
  static constexpr bool kInt = true;
  __device__ static __forceinline__ acc_t run(i32x4_t a, i32x4_t b, acc_t c)
  {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
  }
};

// A 16x16 MFMA whose accumulator input and result are one AGPR tuple ("+a").
// The 4-wave workgroup holds 256 accumulator registers per lane; with the
// builtins the compiler gives the 16x16 MFMAs (which, unlike the 32x32 ones,
// have no tied-accumulator form) a different result tuple than input and
// shuffles the accumulators through VGPRs every stage.  Volatile, so these
// MFMAs keep their source order relative to each other and to the fragment
// reads and loads written between them: the source order is the schedule.
// The compiler's hazard tracking does not see inside the asm, so callers
// cover the two hazards it would: a VALU write of an accumulator (the
// zeroing) followed by the MFMA's read, and the MFMA's write followed by a
// VALU read (the epilogue's v_accvgpr_read), each with s_nop wait states.
template <class Mma>
__device__ __forceinline__ void
mfma_pinned(typename Mma::acc_t& c, i32x4_t a, i32x4_t b)
{
  static_assert(Mma::kF == 16, "pinned MFMAs are the 16x16 shapes");
  if constexpr (Mma::kInt) {
    asm volatile("v_mfma_i32_16x16x64_i8 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
  } else {
    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
  }
}

// The accumulators of one wave: weight fragments x activation fragments
// (the wave covers kBN / WN weight rows and 128 activation rows).
template <class Mma, int WN>
using acc_array_t = typename Mma::acc_t[kBN / WN / Mma::kF][128 / Mma::kF];

// ---- epilogue stores (shared by the GEMM and the split-K reduction) ------
// Four consecutive output columns n..n+3 of activation row m of problem P.
__device__ __forceinline__ void
store_bf16x4(const GemmProblem& P, int m, int n, float v0, float v1, float v2,
             float v3)
{
  if (P.bias != nullptr) {
    const uint2 bb = *reinterpret_cast<const uint2*>(P.bias + n);
    v0 += bf16_to_f32(bb.x & 0xffffu);
    v1 += bf16_to_f32(bb.x >> 16);
    v2 += bf16_to_f32(bb.y & 0xffffu);
    v3 += bf16_to_f32(bb.y >> 16);
  }
  uint2 o;
  o.x = bf16_bits(v0) | (bf16_bits(v1) << 16);
  o.y = bf16_bits(v2) | (bf16_bits(v3) << 16);
  *reinterpret_cast<uint2*>(static_cast<uint16_t*>(P.y) + (size_t)m * P.ldy +
                            n) = o;
}

__device__ __forceinline__ void
store_i32x4(const GemmProblem& P, int m, int n, int v0, int v1, int v2, int v3)
{
  *reinterpret_cast<int4*>(static_cast<int32_t*>(P.y) + (size_t)m * P.ldy +
                           n) = make_int4(v0, v1, v2, v3);
}

// Fused dequant: bf16_rne((float(acc) * sa[m]) * sw[n] (+ bias)).
__device__ __forceinline__ void
store_dequant4(const GemmProblem& P, int m, int n, int a0, int a1, int a2,
               int a3)
{
  const float sam = P.sa[m];
  const float4 swn = *reinterpret_cast<const float4*>(P.sw + n);
  store_bf16x4(P, m, n, ((float)a0 * sam) * swn.x, ((float)a1 * sam) * swn.y,
               ((float)a2 * sam) * swn.z, ((float)a3 * sam) * swn.w);
}

// SwiGLU: gate and up are rounded to bf16 first (the unfused GEMMs' output
// precision), then silu(gate) * up in fp32, rounded to bf16.
// silu(g) = g / (1 + e^-g) as g * rcp(1 + 2^(-g log2 e)) with the hardware
// exp2 and reciprocal (v_exp_f32, v_rcp_f32, ~1 ulp each): 6 VALU
// operations instead of the ~25 of libm's expf and an IEEE division.  The
// result is rounded to bf16 (8 significant bits) afterwards.  Every SwiGLU
// here (the elementwise kernel, the fused epilogue, the split reduction)
// uses this one helper, so they agree bit for bit.
__device__ __forceinline__ float
swiglu_f(float g, float u)
{
  // both rounded by one v_cvt_pk_bf16_f32 (RNE, as bf16_round for finite
  // values): three VALU operations instead of eight
  const uint32_t p = pack_bf16x2(g, u);
  const float gv = __uint_as_float(p << 16);
  const float uv = __uint_as_float(p & 0xffff0000u);
  const float e = __builtin_amdgcn_exp2f(gv * -1.4426950408889634f);
  return (gv * __builtin_amdgcn_rcpf(1.0f + e)) * uv;
}

__device__ __forceinline__ uint32_t
swiglu1(float g, float u)
{
  return bf16_bits(swiglu_f(g, u));
}

__device__ __forceinline__ void
store_swiglu4(const GemmProblem& P, int m, int n, const float g[4],
              const float u[4])
{
  uint2 o;
  o.x = swiglu1(g[0], u[0]) | (swiglu1(g[1], u[1]) << 16);
  o.y = swiglu1(g[2], u[2]) | (swiglu1(g[3], u[3]) << 16);
  *reinterpret_cast<uint2*>(static_cast<uint16_t*>(P.y) + (size_t)m * P.ldy +
                            n) = o;
}


// Which problem a linear tile index belongs to (uniform over the block).
__device__ __forceinline__ int
find_problem(const GemmBatch& B, int tile)
{
  int p = 0;
#pragma unroll
  for (int q = 1; q < kMaxProb; ++q) {
    if (q < B.nprob && tile >= B.p[q].tile_begin) { p = q; }
  }
  return p;
}

// Tile origin (first activation row, first output column) of a tile of P.
// Grouped raster: bands of 4 row-tiles, walked column by column, so the
// tiles that run together share activation and weight rows in L2.
template <Epi E>
__device__ __forceinline__ void
tile_origin(const GemmProblem& P, int tile, int* row0, int* col0)
{
  constexpr int GM = 4;
  const int t = tile - P.tile_begin;
  const int per_band = GM * P.tiles_n;
  const int band = t / per_band;
  const int first_m = band * GM;
  const int gm = min(P.tiles_m - first_m, GM);
  const int tin = t - band * per_band;
  *row0 = (first_m + tin % gm) * kBM;
  *col0 = (tin / gm) * tile_cols(E);
}

// Which tile and which share of K a workgroup computes.
struct TileWork {
  int tile;
  int share;
  bool is_split;
  int prob;     // problem index in the batch
  int row0;     // first activation row of the tile (within the problem)
  int col0;     // first output column of the tile
  int kbeg;     // first K stage of this workgroup
  int nst;      // K stages of this workgroup
};

// Work item w: whole tiles first, then the split tiles, `split`
// consecutive items per tile, each a contiguous share of the `nk` K stages.
template <Epi E>
__device__ __forceinline__ TileWork
tile_work(const GemmBatch& B, int nk, int w)
{
  TileWork t;
  const int SB = B.split_begin;
  t.is_split = w >= SB;
  t.share = 0;
  if (!t.is_split) {
    t.tile = w;
  } else {
    t.tile = SB + (w - SB) / B.split;
    t.share = (w - SB) % B.split;
  }
  t.prob = find_problem(B, t.tile);
  tile_origin<E>(B.p[t.prob], t.tile, &t.row0, &t.col0);
  t.kbeg = t.is_split ? (t.share * nk) / B.split : 0;
  const int kend = t.is_split ? ((t.share + 1) * nk) / B.split : nk;
  t.nst = kend - t.kbeg;
  return t;
}

// Scheduling masks of __builtin_amdgcn_sched_group_barrier.
constexpr int kSchedMfma = 0x008, kSchedVmem = 0x010, kSchedDsRead = 0x100;

// Where the fragment reads of a sub-step go.  When a sub-step has at least
// twice as many MFMAs as reads (the 16x16 builds: 32 MFMAs, 12 reads), read
// r goes after MFMA r * kMfmas / kReads + 1, spread over the whole
// sub-step: measured +4.6% (bf16) and +1.8% (int8) on the kernel against
// one read after each of the first 12 MFMAs, and +1.6% (bf16) against one
// after every second MFMA.  Otherwise (the 32x32 builds: 8 MFMAs, 6
// reads) one read after each of the first MFMAs.
template <int kMfmas, int kReads>
__device__ __forceinline__ bool
read_after(int k)
{
  if constexpr (kMfmas >= 2 * kReads) {
#pragma unroll
    for (int r = 0; r < kReads; ++r) {
      if (k == r * kMfmas / kReads + 1) { return true; }
    }
    return false;
  } else {
    return k < kReads;
  }
}

// `reads` fragment reads spread over `mfmas` MFMAs.
template <int kMfmas, int kReads>
__device__ __forceinline__ void
interleave_reads()
{
#pragma unroll
  for (int k = 0; k < kMfmas; ++k) {
    __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
    if (read_after<kMfmas, kReads>(k)) {
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
    }
  }
}

// `loads` direct loads and `reads` fragment reads spread over `mfmas` MFMAs.
// With at least two MFMAs per load (the 16x16 builds: 8 loads, 32 MFMAs) a
// load goes after every second MFMA from the first: int8 +0.8%, bf16 the
// same, against one load after each of the first MFMAs.
template <int kMfmas, int kLoads, int kReads>
__device__ __forceinline__ void
interleave_loads_reads()
{
  constexpr int kLoadsPerMfma = (kLoads + kMfmas - 1) / kMfmas;
  constexpr int kLoadEvery = kMfmas >= 2 * kLoads ? 2 : 1;
#pragma unroll
  for (int k = 0; k < kMfmas; ++k) {
    __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
    if constexpr (kLoadEvery == 2) {
      if (k % 2 == 0 && k / 2 < kLoads) {
        __builtin_amdgcn_sched_group_barrier(kSchedVmem, 1, 0);
      }
    } else {
#pragma unroll
      for (int l = 0; l < kLoadsPerMfma; ++l) {
        if (k * kLoadsPerMfma + l < kLoads) {
          __builtin_amdgcn_sched_group_barrier(kSchedVmem, 1, 0);
        }
      }
    }
    if (read_after<kMfmas, kReads>(k)) {
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
    }
  }
}

// Workgroup barrier for LDS hand-offs: waits for this wave's LDS accesses
// but not for its global loads and stores (__syncthreads' fence waits for
// all of them).  The memory clobber keeps the compiler from moving memory
// accesses across it.
__device__ __forceinline__ void
lds_barrier()
{
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// bf16 epilogue of a whole tile through LDS.  The MFMA layout gives each
// lane 4 consecutive output columns of one row per store, so direct stores
// write every 128-byte output line in 16-byte pieces from 8 instructions.
// Instead each wave writes its bf16 results (bias, dequant or SwiGLU
// applied) into a [256][TC] tile in the two stage buffers (rows 0..127 in
// ring[0], 128..255 in ring[1]; the main loop is done with them), then the
// tile is read back row-wise and 32 (or 16) lanes store one row's
// 512 (256) contiguous bytes.  Row r's 16-byte chunk c sits at chunk
// c ^ (r % CH) of its staged row, which spreads both the column writes (32
// rows, one chunk) and the row reads over the bank groups.
template <class Mma, Epi E, int WN>
__device__ __forceinline__ void
gemm_epilogue_staged(const GemmProblem& P, const TileWork& t, int wm, int wn,
                     int lane, const acc_array_t<Mma, WN>& acc,
                     char* const (&ring)[2], const float* scl)
{
  constexpr int NW = kBN / WN;
  constexpr int kF = Mma::kF;
  constexpr int FI = NW / kF;
  constexpr int FJ = 128 / kF;
  constexpr int kGr = Mma::kE / 4;            // 4-column groups per fragment
  constexpr int kGs = 4 * (64 / kF);          // column stride of the groups
  constexpr int TC = tile_cols(E);            // output columns per tile
  constexpr int RB = TC * 2;                  // staged bytes per row
  constexpr int CH = RB / 16;                 // 16-byte chunks per row
  const int lr = lane % kF;
  const int lh = lane / kF;
  // Scales and bias of every row and column group this lane writes, loaded
  // together before any is used (inside the per-fragment conditionals each
  // load would be waited for on its own).  Indices past the problem are
  // clamped to a valid element; those outputs are staged but never stored.
  constexpr bool kScaled = E == Epi::kDequantBf16;
  constexpr int kCols = E == Epi::kSwiglu ? 1 : FI * kGr;   // column groups
  float sam[kScaled ? FJ : 1];
  float4 swn[kScaled ? kCols : 1];
  uint2 bia[E == Epi::kSwiglu ? 1 : kCols];
  const bool has_bias = E != Epi::kSwiglu && P.bias != nullptr;
  if constexpr (E != Epi::kSwiglu) {
#pragma unroll
    for (int c = 0; c < kCols; ++c) {
      const int i = c / kGr, g = c % kGr;
      const int n = min(t.col0 + wn * NW + i * kF + g * kGs + lh * 4, P.n - 4);
      if constexpr (kScaled) {
        swn[c] = *reinterpret_cast<const float4*>(scl + kBM + wn * NW + i * kF + g * kGs +
                                                  lh * 4);
      }
      bia[c] = has_bias ? *reinterpret_cast<const uint2*>(P.bias + n) : uint2{0u, 0u};
    }
  }
  if constexpr (kScaled) {
#pragma unroll
    for (int j = 0; j < FJ; ++j) {
      sam[j] = scl[wm * 128 + j * kF + lr];
    }
  }
  // The tile's results in bf16 (bias or SwiGLU applied) are computed
  // before the barrier: a wave that leaves the main loop early converts
  // while its partner still issues MFMAs, and only the LDS writes wait
  // (bf16 step 0.35% faster, interleaved, one box).  There the bias test
  // is taken once, outside the loops: inside them its branches split the
  // code into blocks the held results spill across.
  constexpr int KC = E == Epi::kSwiglu ? (FI / 2) * kGr : FI * kGr;
  u32x2_t pk[kScaled ? 1 : FJ][KC];
  // bias: 0 none, 1 added, 2 tested per group (the dequant epilogue's
  // original form, whose registers fit only that way)
  auto convert = [&](auto bias_mode, auto&& emit) {
    constexpr int kBias = decltype(bias_mode)::value;
#pragma unroll
    for (int j = 0; j < FJ; ++j) {
      if constexpr (E == Epi::kSwiglu) {
#pragma unroll
        for (int i = 0; i < FI / 2; ++i) {
#pragma unroll
          for (int g = 0; g < kGr; ++g) {
            const auto& ga = acc[i][j];
            const auto& ua = acc[i + FI / 2][j];
            emit(j, i * kGr + g, u32x2_t{
                pack_bf16x2(swiglu_f(ga[g * 4 + 0], ua[g * 4 + 0]),
                            swiglu_f(ga[g * 4 + 1], ua[g * 4 + 1])),
                pack_bf16x2(swiglu_f(ga[g * 4 + 2], ua[g * 4 + 2]),
                            swiglu_f(ga[g * 4 + 3], ua[g * 4 + 3]))});
          }
        }
      } else {
#pragma unroll
        for (int i = 0; i < FI; ++i) {
#pragma unroll
          for (int g = 0; g < kGr; ++g) {
            const int c = i * kGr + g;
            const auto& a = acc[i][j];
            float v[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              if constexpr (kScaled) {
                v[e] = (float)bits_as<int>(a[g * 4 + e]);
              } else {
                v[e] = a[g * 4 + e];
              }
            }
            if constexpr (kScaled) {
              v[0] = (v[0] * sam[j]) * swn[c].x;
              v[1] = (v[1] * sam[j]) * swn[c].y;
              v[2] = (v[2] * sam[j]) * swn[c].z;
              v[3] = (v[3] * sam[j]) * swn[c].w;
            }
            if (kBias == 1 || (kBias == 2 && has_bias)) {
              v[0] += bf16_to_f32(bia[c].x & 0xffffu);
              v[1] += bf16_to_f32(bia[c].x >> 16);
              v[2] += bf16_to_f32(bia[c].y & 0xffffu);
              v[3] += bf16_to_f32(bia[c].y >> 16);
            }
            emit(j, c, u32x2_t{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])});
          }
        }
      }
    }
  };
  // The dequant epilogue converts after the barrier, writing each group
  // as it goes: held until then, its packed results beside its scales
  // overflow the registers.
  char* const half = wm ? ring[1] : ring[0];
  // LDS address of the 4 output columns from `col` of row `row` (within
  // the half)
  auto put_at = [&](int row, int col) {
    const int c = col >> 3;
    return half + row * RB + ((c ^ (row % CH)) << 4) + ((col & 7) << 1);
  };
  auto col_of = [&](int cg) {
    const int i = cg / kGr, g = cg % kGr;
    return (E == Epi::kSwiglu ? wn * (NW / 2) : wn * NW) + i * kF + g * kGs + lh * 4;
  };
  if constexpr (kScaled) {
    __syncthreads();
    convert(std::integral_constant<int, 2>{}, [&](int j, int cg, u32x2_t v) {
      *reinterpret_cast<u32x2_t*>(put_at(j * kF + lr, col_of(cg))) = v;
    });
  } else {
    auto hold = [&](int j, int cg, u32x2_t v) { pk[j][cg] = v; };
    if (has_bias) {
      convert(std::integral_constant<int, 1>{}, hold);
    } else {
      convert(std::integral_constant<int, 0>{}, hold);
    }
    // Every wave is past its last fragment read of the main loop.
    __syncthreads();
#pragma unroll
    for (int j = 0; j < FJ; ++j) {
#pragma unroll
      for (int cg = 0; cg < KC; ++cg) {
        *reinterpret_cast<u32x2_t*>(put_at(j * kF + lr, col_of(cg))) = pk[j][cg];
      }
    }
  }
  __syncthreads();
  // Read back: wave w stores tile rows [RW w, RW w + RW) (RW = 256 / waves);
  // 64 / CH rows per instruction, CH lanes per row.
  constexpr int RW = kBM / (2 * WN);
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  constexpr int kRowsPerRead = 64 / CH;
  // The read-back addresses depend on the lane only; computed from an
  // opaque copy of it they stay here instead of being hoisted out of the
  // tile loop, where they would be spilled across the main loop and each
  // reload would wait for every store in flight.
  int lane_o = lane;
  asm volatile("" : "+v"(lane_o));
  const int first = wave * RW;                          // first tile row
  const char* const src = first >= 128 ? ring[1] : ring[0];
  // Whole 128-byte output lines go out as non-temporal stores, so the
  // output bypasses allocation in L2 instead of evicting the activation and
  // weight rows that the tiles still running on the XCD stream through it.
  // Buffer stores over the tile's valid rows: rows past the problem fall
  // outside the resource and are dropped, columns past it get an
  // out-of-range offset (the host bounds ldy so that 256 rows of it stay
  // below kOobOffset).
  const __amdgpu_buffer_rsrc_t yr =
      make_rsrc(static_cast<uint16_t*>(P.y) + (size_t)t.row0 * P.ldy,
                min(kBM, P.rows - t.row0) * P.ldy * 2);
  const int c = lane_o % CH;
  const int n = t.col0 + c * 8;
  int voff = n < P.n ? ((first + lane_o / CH) * P.ldy + n) * 2 : kOobOffset;
  const int rstep = kRowsPerRead * P.ldy * 2;
#pragma unroll
  for (int r = 0; r < RW; r += kRowsPerRead) {
    const int hrow = first % 128 + r + lane_o / CH;     // row within the half
    const u32x4_t v = *reinterpret_cast<const u32x4_t*>(
        src + hrow * RB + ((c ^ (hrow % CH)) << 4));
    __builtin_amdgcn_raw_buffer_store_b128(v, yr, voff, 0, kNonTemporal);
    voff += rstep;
  }
  // The next tile's loads refill these buffers once every wave's reads of
  // them are done; the stores drain meanwhile.
  lds_barrier();
}

// Epilogue of a tile.  acc[i][j][r] holds tile column (weight row within
// the tile) wn*NW + i*32 + (r>>2)*8 + lh*4 + (r&3) and tile row wm*128 +
// j*32 + lr.  A K share writes its raw accumulators to the workspace
// [kBM][kBN] (rows past the problem are never read back); a whole tile
// applies the epilogue E.
template <class Mma, Epi E, int WN>
__device__ __forceinline__ void
gemm_epilogue(const GemmBatch& B, const GemmProblem& P, const TileWork& t,
              int wm, int wn, int lane, const acc_array_t<Mma, WN>& acc,
              char* const (&ring)[2], const float* scl)
{
  constexpr int NW = kBN / WN;
  constexpr int kF = Mma::kF;
  constexpr int FI = NW / kF;
  constexpr int FJ = 128 / kF;
  constexpr int kGr = Mma::kE / 4;
  constexpr int kGs = 4 * (64 / kF);
  // Lane-derived offsets from an opaque copy of the lane: computed here,
  // per tile, instead of being hoisted to the kernel's start and spilled
  // across the main loop (a reload waits for every store in flight).
  int lane_e = lane;
  asm volatile("" : "+v"(lane_e));
  const int lr = lane_e % kF;
  const int lh = lane_e / kF;
  if (t.is_split) {
    int32_t* wsb = static_cast<int32_t*>(B.ws) +
                   (size_t)((t.tile - B.split_begin) * B.split + t.share) *
                       (kBM * kBN);
#pragma unroll
    for (int j = 0; j < FJ; ++j) {
      const int ml = wm * 128 + j * kF + lr;
      if (t.row0 + ml >= P.rows) { continue; }
#pragma unroll
      for (int i = 0; i < FI; ++i) {
#pragma unroll
        for (int g = 0; g < kGr; ++g) {
          const int nl = wn * NW + i * kF + g * kGs + lh * 4;
          const auto& a = acc[i][j];
          *reinterpret_cast<int4*>(wsb + ml * kBN + nl) = make_int4(
              bits_as<int>(a[g * 4 + 0]), bits_as<int>(a[g * 4 + 1]),
              bits_as<int>(a[g * 4 + 2]), bits_as<int>(a[g * 4 + 3]));
        }
      }
    }
    return;
  }
  if constexpr (E != Epi::kI32) {
    gemm_epilogue_staged<Mma, E, WN>(P, t, wm, wn, lane_e, acc, ring, scl);
    return;
  }
#pragma unroll
  for (int j = 0; j < FJ; ++j) {
    const int m = t.row0 + wm * 128 + j * kF + lr;
    if (m >= P.rows) { continue; }
    if constexpr (E == Epi::kSwiglu) {
#pragma unroll
      for (int i = 0; i < FI / 2; ++i) {
#pragma unroll
        for (int g = 0; g < kGr; ++g) {
          const int n = t.col0 + wn * (NW / 2) + i * kF + g * kGs + lh * 4;
          if (n >= P.n) { continue; }
          float gv[4], uv[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            gv[e] = acc[i][j][g * 4 + e];
            uv[e] = acc[i + FI / 2][j][g * 4 + e];
          }
          store_swiglu4(P, m, n, gv, uv);
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < FI; ++i) {
#pragma unroll
        for (int g = 0; g < kGr; ++g) {
          const int n = t.col0 + wn * NW + i * kF + g * kGs + lh * 4;
          if (n >= P.n) { continue; }
          const auto& a = acc[i][j];
          if constexpr (E == Epi::kI32) {
            store_i32x4(P, m, n, a[g * 4], a[g * 4 + 1], a[g * 4 + 2],
                        a[g * 4 + 3]);
          } else if constexpr (E == Epi::kDequantBf16) {
            store_dequant4(P, m, n, a[g * 4], a[g * 4 + 1], a[g * 4 + 2],
                           a[g * 4 + 3]);
          } else {
            store_bf16x4(P, m, n, a[g * 4], a[g * 4 + 1], a[g * 4 + 2],
                         a[g * 4 + 3]);
          }
        }
      }
    }
  }
}

// The GEMM main loop, parametrised by the LDS pipeline:
//   KB     bytes of K per stage per row (128: 64 bf16 / 128 int8; or 64)
//   RING   LDS stages in the ring (2 with KB=128, 4 with KB=64: 128 KiB)
// A ring stage is (kBM + kBN) rows x KB bytes: weight rows 0..255, then
// activation rows.  Loads for stage k+RING are issued once stage k's
// buffer is free, so a load has RING-1 stages to land.
//
// WN = waves along the tile's N (weight-row) extent; 2 waves along M.
//   WN = 2: 4 waves, each 128 x 128 (8 x 8 accumulators of 16 x 16,
//           pinned in AGPRs)
//   WN = 4: 8 waves, two per SIMD, each 128 x 64 (4 x 8 accumulators of
//           16 x 16, or 2 x 4 of 32 x 32); a
//           wave waiting on LDS, memory or the barrier leaves the matrix
//           core to the other wave of its SIMD.
//
// LDS layout.  Row r's logical 16-byte chunk c sits at position
// c ^ key(r).  LDS serves 16 lanes of a 16-byte read per cycle over 64
// four-byte banks (16 bank groups of 16 bytes); a fragment read touches 16
// consecutive rows at one logical chunk, so key(r) is chosen to put those
// 16 reads in 16 different bank groups:
//   KB = 128 (8 chunks/row, 2 rows per 256 B): key(r) = (r >> 1) & 7
//   KB =  64 (4 chunks/row, 4 rows per 256 B): key(r) = (r >> 2) & 3
//
// Direct-to-LDS loads.  One buffer_load ... lds instruction writes a 1 KiB
// block, lane l landing at byte 16*l (KB/16 chunks per row, 1024/KB rows
// per block).  The swizzle is applied on the global side: lane l fetches
// the logical chunk that belongs at its landing position.  Wave w fills
// stage rows [w * R, (w+1) * R) with R = 512 / waves (waves 0..WN-1 the
// weight rows, exactly the rows wave column w computes with; the others
// the activation rows).  SwiGLU tiles: wave column wn owns NW/2 output
// columns; its NW weight rows are NW/2 gate rows then the NW/2 matching up
// rows, so a lane's gate and up accumulators cover the same outputs.
//
// Buffer resources span only the tile's valid rows, so rows past M or N
// read as zero in hardware; the K tail and the stages past this
// workgroup's K range are zero-filled by pushing their offsets out of
// range.  The range check applies to the per-lane (VGPR) offset, so every
// row offset is carried there; only the stage's K offset, common to all
// rows, rides in the SGPR.
template <class Mma, Epi E, int WN, int KB, int RING>
__device__ __forceinline__ void
gemm_tile(const GemmBatch& B, char* const (&ring)[RING], float* scl, int item)
{
  constexpr int kWaves = 2 * WN;
  constexpr int NW = kBN / WN;               // weight rows per wave
  constexpr int FI = NW / Mma::kF;           // weight fragments per sub-step
  constexpr int FJ = 128 / Mma::kF;          // activation fragments
  constexpr int kStageBytes = (kBM + kBN) * KB;
  constexpr int kRowsPerBlock = 1024 / KB;   // rows one load instruction fills
  constexpr int kChunks = KB / 16;           // 16-byte chunks per row
  constexpr int LB = kStageBytes / 1024 / kWaves;   // load blocks per wave
  constexpr int kSub = KB / Mma::kKBytes;    // MFMA sub-steps per stage
  constexpr int kGroups = 64 / Mma::kF;      // 16-byte chunks per sub-step
  constexpr int kRowsPerWave = (kBM + kBN) / kWaves;

  const int kbytes = B.kbytes;
  const int nk = (kbytes + KB - 1) / KB;
  const TileWork t = tile_work<E>(B, nk, item);
  const GemmProblem& P = B.p[t.prob];
  constexpr int TC = tile_cols(E);

  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // Wave w computes tile rows wm*128.. and weight rows wn*NW..; waves w and
  // w + 4 share a SIMD, so each SIMD holds one upper and one lower half.
  const int wm = wave / WN;
  const int wn = wave % WN;

  // ---- operand extents and per-wave load parameters (wave-uniform) ------
  // Weight rows are wld bytes apart (kbytes for a plain [N][K] matrix, 2K
  // for the reference's row-interleaved gate/up weight).
  const int wld = P.wld;
  const char* a_base = static_cast<const char*>(P.a) + (size_t)t.row0 * kbytes;
  const int a_bytes = min(kBM, P.rows - t.row0) * kbytes;
  const char* w_base = static_cast<const char*>(P.w) + (size_t)t.col0 * wld;
  const int w_bytes = min(E == Epi::kSwiglu ? TC : kBN, P.n - t.col0) * wld;
  const char* u_base = E == Epi::kSwiglu
                           ? static_cast<const char*>(P.w2) + (size_t)t.col0 * wld
                           : w_base;
  const bool loads_w = wave < WN;
  const int pitch = loads_w ? wld : kbytes;
  const __amdgpu_buffer_rsrc_t r_lo =
      make_rsrc(loads_w ? w_base : a_base, loads_w ? w_bytes : a_bytes);
  const __amdgpu_buffer_rsrc_t r_hi =
      make_rsrc(loads_w ? u_base : a_base, loads_w ? w_bytes : a_bytes);
  // First operand row and block mask: blocks [0, LB/2) use r_lo and
  // [LB/2, LB) r_hi (SwiGLU weights: gate then up).
  const int row_base =
      loads_w ? (E == Epi::kSwiglu ? wave * (kRowsPerWave / 2) : wave * kRowsPerWave)
              : (wave - WN) * kRowsPerWave;
  const int bmask = (loads_w && E == Epi::kSwiglu) ? (LB / 2 - 1) : (LB - 1);

  // Lane landing position -> logical chunk.  Blocks start at rows that are
  // multiples of kRowsPerBlock, so the key depends on the block only through
  // its parity when KB = 128 (8 rows per block) and not at all when KB = 64.
  const int lrow = lane / kChunks;                  // row within the block
  const int lpos = lane % kChunks;                  // landing position
  auto key_of = [&](int blk_row) {
    if constexpr (KB == 128) { return ((blk_row + lrow) >> 1) & 7; }
    else { return ((blk_row + lrow) >> 2) & 3; }
  };
  const int chunk_even = lpos ^ key_of(0);
  const int chunk_odd = lpos ^ key_of(kRowsPerBlock);
  const int lane_even = lrow * pitch + (chunk_even << 4);
  const int lane_odd = lrow * pitch + (chunk_odd << 4);
  const int tail_even =
      ((nk - 1) * KB + (chunk_even << 4) < kbytes) ? 0 : kOobOffset;
  const int tail_odd =
      ((nk - 1) * KB + (chunk_odd << 4) < kbytes) ? 0 : kOobOffset;

  // A stage's loads: per-stage offsets, then LB blocks of 1 KiB each.
  struct LoadArgs { int ko, ve, vo; };
  auto load_args = [&](int ktl) {
    const int kt = t.kbeg + ktl;
    const bool last = kt == nk - 1;
    const int oob = ktl >= t.nst ? kOobOffset : 0;
    LoadArgs a;
    a.ko = __builtin_amdgcn_readfirstlane(min(kt, nk - 1) * KB);
    a.ve = lane_even + row_base * pitch + (last ? tail_even : 0) + oob;
    a.vo = lane_odd + row_base * pitch + (last ? tail_odd : 0) + oob;
    return a;
  };
  auto load_block = [&](const LoadArgs& a, char* stage_base, int b) {
    char* dst = stage_base + wave * (kRowsPerWave * KB);
    const int orow = (b & bmask) * kRowsPerBlock;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        b < LB / 2 ? r_lo : r_hi,
        (__attribute__((address_space(3))) void*)(dst + b * 1024), 16,
        ((b & 1) ? a.vo : a.ve) + orow * pitch, a.ko, 0, 0);
  };
  auto issue_loads = [&](char* stage_base, int ktl) {
    const LoadArgs a = load_args(ktl);
#pragma unroll
    for (int b = 0; b < LB; ++b) { load_block(a, stage_base, b); }
  };

  // ---- MFMA fragments ---------------------------------------------------
  // Lane l reads row l % kF of a fragment (fragments start at multiples
  // of kF >= 16 rows, so the swizzle key of the row is that of l % kF) at
  // chunk kGroups * s + l / kF.
  const int lr = lane % Mma::kF;
  const int lh = lane / Mma::kF;
  int rd[kSub];
#pragma unroll
  for (int s = 0; s < kSub; ++s) {
    const int key = KB == 128 ? ((lr >> 1) & 7) : ((lr >> 2) & 3);
    rd[s] = lr * KB + (((kGroups * s + lh) ^ key) << 4);
  }
  const int wbase = wn * NW * KB;
  const int abase = kBN * KB + wm * 128 * KB;

  typename Mma::acc_t acc[FI][FJ];
#pragma unroll
  for (int i = 0; i < FI; ++i) {
#pragma unroll
    for (int j = 0; j < FJ; ++j) { acc[i][j] = typename Mma::acc_t{}; }
  }
  // The 4-wave workgroup runs the pinned MFMAs.  The empty asm statements
  // order the zeroing (VALU writes of the AGPRs) before the s_nop, which
  // gives the first MFMAs' accumulator reads their wait states.
  constexpr bool kPin = WN == 2;
  if constexpr (kPin) {
#pragma unroll
    for (int i = 0; i < FI; ++i) {
#pragma unroll
      for (int j = 0; j < FJ; ++j) { asm volatile("" : "+a"(acc[i][j])); }
    }
    asm volatile("s_nop 4");
  }

  i32x4_t fa[2][FI], fb[2][FJ];
  auto read_frags = [&](const char* base, int s, int buf) {
#pragma unroll
    for (int i = 0; i < FI; ++i) {
      fa[buf][i] = *reinterpret_cast<const i32x4_t*>(base + wbase + i * Mma::kF * KB +
                                                     rd[s]);
    }
#pragma unroll
    for (int j = 0; j < FJ; ++j) {
      fb[buf][j] = *reinterpret_cast<const i32x4_t*>(base + abase + j * Mma::kF * KB +
                                                     rd[s]);
    }
  };
  auto mma_step = [&](int buf) {
#pragma unroll
    for (int i = 0; i < FI; ++i) {
#pragma unroll
      for (int j = 0; j < FJ; ++j) {
        acc[i][j] = Mma::run(fa[buf][i], fb[buf][j], acc[i][j]);
      }
    }
  };
  constexpr int kMfmaPerStep = FI * FJ;
  constexpr int kReadsPerStep = FI + FJ;

  // Pinned schedule (4 waves): fragment read r of a sub-step, in the order
  // the next sub-step first uses them (a0, b0..b7, a1..a7), so its first
  // MFMAs wait for two reads, not nine.
  auto read_one = [&](const char* base, int s, int buf, int r) {
    const int q = r == 0 ? 0 : (r <= FJ ? FI + r - 1 : r - FJ);
    if (q < FI) {
      fa[buf][q] = *reinterpret_cast<const i32x4_t*>(base + wbase + q * Mma::kF * KB +
                                                     rd[s]);
    } else {
      fb[buf][q - FI] = *reinterpret_cast<const i32x4_t*>(
          base + abase + (q - FI) * Mma::kF * KB + rd[s]);
    }
  };
  // One sub-step's MFMAs with `between(k)` after MFMA k: that is where the
  // reads and loads issue (the MFMAs are volatile asm, so they stay put).
  auto pinned_step = [&](int buf, auto&& between) {
#pragma unroll
    for (int i = 0; i < FI; ++i) {
#pragma unroll
      for (int j = 0; j < FJ; ++j) {
        mfma_pinned<Mma>(acc[i][j], fa[buf][i], fb[buf][j]);
        between(i * FJ + j);
      }
    }
  };

  // One K stage in ring buffer `cur`; `nxt` holds the next stage.  On entry
  // the fragments of sub-step 0 are in fa/fb[0]; the fragments of sub-step
  // s+1 are read while the MFMAs of sub-step s run.  Before the last
  // sub-step the stage's buffer is handed back: once every wave has its
  // last fragments in registers and its loads of the next stage have
  // landed (at most the loads of the RING-2 stages after it may still be
  // in flight; loads complete in issue order), one barrier lets the loads
  // of stage k+RING refill `cur` and the first fragments of the next stage
  // be read while the last MFMAs run.  The body is branch-free, which keeps
  // the accumulators in registers across the whole loop; past the last
  // stage the extra loads fetch nothing and the extra reads are unused.
  // A wave whose 128 rows all lie past the problem (the lower half of a
  // 128-row und tile) runs the same loads, waits and barriers without the
  // fragment reads and MFMAs (`act` false), leaving its SIMD's matrix core
  // to the partner wave; its accumulators stay zero and are never stored.
  auto stage = [&](auto act, char* cur, const char* nxt, int ktl) {
    constexpr bool kAct = decltype(act)::value;
    if constexpr (kPin) {
      // The same hand-off, scheduled in source: one read after every 4th
      // MFMA (from MFMA 1 in the first sub-step, from MFMA 2 in the last),
      // and in the last sub-step one 1 KiB load after every 4th MFMA from
      // MFMA 0 -- spread loads issue without stalling the MFMA stream.
      static_assert(kSub == 2 && kMfmaPerStep == 4 * kReadsPerStep &&
                    LB == kReadsPerStep, "pinned schedule: 64 MFMAs, 16 reads, 16 loads");
      if constexpr (kAct) {
        pinned_step(0, [&](int k) {
          if (k % 4 == 1) { read_one(cur, 1, 1, k / 4); }
        });
      }
      asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
      __syncthreads();
      if constexpr (kAct) {
        const LoadArgs la = load_args(ktl + RING);
        pinned_step(1, [&](int k) {
          if (k % 4 == 0) { load_block(la, cur, k / 4); }
          if (k % 4 == 2) { read_one(nxt, 0, 0, k / 4); }
        });
      } else {
        issue_loads(cur, ktl + RING);
      }
      return;
    }
    if constexpr (kAct) {
#pragma unroll
      for (int s = 0; s + 1 < kSub; ++s) {
        read_frags(cur, s + 1, (s + 1) & 1);
        mma_step(s & 1);
        interleave_reads<kMfmaPerStep, kReadsPerStep>();
      }
    }
    if constexpr (RING == 2) {
      asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
    } else if constexpr (LB == 4) {
      asm volatile("s_waitcnt vmcnt(8) lgkmcnt(0)" ::: "memory");
    } else {
      asm volatile("s_waitcnt vmcnt(16) lgkmcnt(0)" ::: "memory");
    }
    __syncthreads();
    issue_loads(cur, ktl + RING);
    if constexpr (kAct) {
      read_frags(nxt, 0, 0);
      mma_step((kSub - 1) & 1);
      interleave_loads_reads<kMfmaPerStep, LB, kReadsPerStep>();
    }
  };

  // ---- main loop: a multiple of RING stages; a padding stage (K past the
  // range) reads as zeros and adds exactly 0 to every accumulator --------
  const int nst_pad = (t.nst + RING - 1) / RING * RING;
  // The dequant epilogue's scales, fetched ahead into LDS: the tile's 256
  // row scales (wave 0) and 256 column scales (wave 1), 4 bytes per lane
  // and instruction; entries past the problem read as zeros and scale
  // outputs that are never stored.  Issued before the stage loads, they
  // land before stage 0 (loads complete in issue order).
  if constexpr (E == Epi::kDequantBf16) {
    if (!t.is_split && wave < 2) {
      const float* src = wave == 0 ? P.sa + t.row0 : P.sw + t.col0;
      const int n = wave == 0 ? min(kBM, P.rows - t.row0) : min(kBN, P.n - t.col0);
      const __amdgpu_buffer_rsrc_t rs = make_rsrc(src, n * 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rs, (__attribute__((address_space(3))) void*)(scl + wave * kBM + i * 64), 4,
            (i * 64 + lane) * 4, 0, 0, 0);
      }
    }
  }
#pragma unroll
  for (int r = 0; r < RING; ++r) { issue_loads(ring[r], r); }
  // Stage 0 has landed once at most the later stages' loads are in flight
  // (loads complete in issue order; the previous tile's output stores may
  // still be draining, which only makes the wait longer).
  if constexpr (RING == 2) {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(LB) : "memory");
  } else {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(3 * LB) : "memory");
  }
  lds_barrier();
  auto main_loop = [&](auto act) {
    if constexpr (decltype(act)::value) {
      if constexpr (kPin) {
        // In the loop's read order (the scheduling barriers keep it), so
        // the loop's waits are the same from either predecessor.
#pragma unroll
        for (int r = 0; r < kReadsPerStep; ++r) {
          read_one(ring[0], 0, 0, r);
          __builtin_amdgcn_sched_barrier(0);
        }
      } else {
        read_frags(ring[0], 0, 0);
      }
    }
    for (int ktl = 0; ktl < nst_pad; ktl += RING) {
#pragma unroll
      for (int r = 0; r < RING; ++r) {
        stage(act, ring[r], ring[(r + 1) % RING], ktl + r);
      }
    }
  };
  if (t.row0 + wm * 128 < P.rows) {
    main_loop(std::true_type{});
  } else {
    main_loop(std::false_type{});
  }
  // No load may still be writing LDS when the workgroup retires.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  if constexpr (kPin) {
    // 32 wait states between the last MFMA's result and the epilogue's
    // reads of the AGPRs (more than the 16x16 shapes' pass count needs);
    // the empty asm statements order those reads after them.
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7");
#pragma unroll
    for (int i = 0; i < FI; ++i) {
#pragma unroll
      for (int j = 0; j < FJ; ++j) { asm volatile("" : "+a"(acc[i][j])); }
    }
  }

  gemm_epilogue<Mma, E, WN>(B, P, t, wm, wn, lane, acc, ring, scl);
}

// Two 64 KiB stages of 128 bytes of K per row.
//
// Work items are dealt in rounds of gridDim.x.  Launched with one workgroup
// per CU the kernel is persistent; launched with one workgroup per item it
// is a single round.  Workgroups b, b+8, ... run on XCD b % 8; each round's
// R items are cut into 8 contiguous runs of R/8, one per XCD, so the tiles
// that run together on an XCD share operand rows in its L2 and a partial
// last round still spreads over all eight XCDs.
template <class Mma, Epi E, int WN>
__global__ __launch_bounds__(128 * WN, 1) void
mot_gemm_kernel(const GemmBatch B)
{
  // Stages as separate objects, so the compiler can tell the fragment
  // reads of one stage from the direct-to-LDS loads filling another.
  __shared__ __attribute__((aligned(1024))) char lds0[kStage];
  __shared__ __attribute__((aligned(1024))) char lds1[kStage];
  char* const ring[2] = {lds0, lds1};
  // the dequant epilogue's row and column scales of the current tile
  __shared__ __attribute__((aligned(16))) float scl[E == Epi::kDequantBf16 ? kBM + kBN : 4];
  const int items = grid_blocks(B);
  const int G = gridDim.x;
  const int b = blockIdx.x;
  for (int base = 0; base < items; base += G) {
    const int R = min(G, items - base);
    int w = base + b;
    if (G % 8 == 0) {
      const int x = b % 8, i = b / 8;
      const int lo = x * R / 8, hi = (x + 1) * R / 8;
      if (i >= hi - lo) { break; }
      w = base + lo + i;
    } else if (b >= R) {
      break;
    }
    gemm_tile<Mma, E, WN, kKB, 2>(B, ring, scl, w);
  }
}

// ---- split-K reduction --------------------------------------------------
// One workgroup per 8 rows of a split tile: sums the tile's K shares in
// share order (fp32 adds for bf16 GEMMs, exact int32 adds for int8) and
// applies the same epilogue as mot_gemm_kernel.  Eight rows (not 16) put
// a 16-tile tail's reduction on all CUs: 4.6 us less per config-2 step.
constexpr int kReduceRowsPerThread = 2;

template <bool kInt, Epi E, int WN>
__global__ __launch_bounds__(256) void
split_reduce_kernel(const GemmBatch B)
{
  constexpr int NW = kBN / WN;
  constexpr int RPT = kReduceRowsPerThread;
  constexpr int kRowsPerBlock = 4 * RPT;
  const int ts = blockIdx.x / (kBM / kRowsPerBlock);
  const int tile = B.split_begin + ts;
  const GemmProblem& P = B.p[find_problem(B, tile)];
  int row0, col0;
  tile_origin<E>(P, tile, &row0, &col0);
  const int32_t* wsb =
      static_cast<const int32_t*>(B.ws) + (size_t)ts * B.split * (kBM * kBN);
  // Thread: column quad q of the tile, rows r and r+4 of the block.  The
  // two rows of a share are loaded together (rows past the problem read
  // stale slot values that are never stored), and the share loop is
  // unrolled, so many loads are in flight; each sum still runs in share
  // order.
  const int q = threadIdx.x & 63;
  const int block_row = (blockIdx.x % (kBM / kRowsPerBlock)) * kRowsPerBlock;
  // A block whose rows all lie past the problem (the lower half of a
  // 128-row und tile) has nothing to store; its loads would only cost
  // bandwidth.
  if (row0 + block_row >= P.rows) { return; }
  const int mlb = block_row + (threadIdx.x >> 6);
  const int nl = q * 4;
  constexpr int kCols = E == Epi::kSwiglu ? 2 : 1;   // gate (+ up) columns
  int col[kCols];
  col[0] = nl;
  if constexpr (E == Epi::kSwiglu) {
    // Gate columns sit at tile columns wn*NW + [0, NW/2), their up
    // partners NW/2 further on; the output column is col0 + wn*NW/2 +
    // that offset.
    if ((nl % NW) >= NW / 2) { return; }
    col[1] = nl + NW / 2;
  }
  float4 f[kCols][RPT];
  int4 r[kCols][RPT];
#pragma unroll
  for (int c = 0; c < kCols; ++c) {
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
      f[c][k] = make_float4(0.f, 0.f, 0.f, 0.f);
      r[c][k] = make_int4(0, 0, 0, 0);
    }
  }
#pragma unroll 8
  for (int sh = 0; sh < B.split; ++sh) {
    const int32_t* base = wsb + (size_t)sh * (kBM * kBN);
    int4 v[kCols][RPT];
#pragma unroll
    for (int c = 0; c < kCols; ++c) {
#pragma unroll
      for (int k = 0; k < RPT; ++k) {
        v[c][k] = *reinterpret_cast<const int4*>(base + (mlb + 4 * k) * kBN + col[c]);
      }
    }
#pragma unroll
    for (int c = 0; c < kCols; ++c) {
#pragma unroll
      for (int k = 0; k < RPT; ++k) {
        if constexpr (kInt) {
          r[c][k].x += v[c][k].x; r[c][k].y += v[c][k].y;
          r[c][k].z += v[c][k].z; r[c][k].w += v[c][k].w;
        } else {
          f[c][k].x += bits_as<float>(v[c][k].x);
          f[c][k].y += bits_as<float>(v[c][k].y);
          f[c][k].z += bits_as<float>(v[c][k].z);
          f[c][k].w += bits_as<float>(v[c][k].w);
        }
      }
    }
  }
#pragma unroll
  for (int k = 0; k < RPT; ++k) {
    const int m = row0 + mlb + 4 * k;
    if (m >= P.rows) { break; }
    if constexpr (E == Epi::kSwiglu) {
      const int n = col0 + (nl / NW) * (NW / 2) + (nl % NW);
      if (n >= P.n) { continue; }
      const float gv[4] = {f[0][k].x, f[0][k].y, f[0][k].z, f[0][k].w};
      const float uv[4] = {f[1][k].x, f[1][k].y, f[1][k].z, f[1][k].w};
      store_swiglu4(P, m, n, gv, uv);
    } else {
      const int n = col0 + nl;
      if (n >= P.n) { continue; }
      if constexpr (E == Epi::kI32) {
        store_i32x4(P, m, n, r[0][k].x, r[0][k].y, r[0][k].z, r[0][k].w);
      } else if constexpr (E == Epi::kDequantBf16) {
        store_dequant4(P, m, n, r[0][k].x, r[0][k].y, r[0][k].z, r[0][k].w);
      } else {
        store_bf16x4(P, m, n, f[0][k].x, f[0][k].y, f[0][k].z, f[0][k].w);
      }
    }
  }
}

// ---- per-row symmetric int8 quantisation ------------------------------
// One workgroup per row: absmax over the row (bf16 widened exactly), then
// q = clamp(round_half_away(x / s), -127, 127) with s = absmax / 127 (fp32
// division, correctly rounded).  The row is read once: each thread keeps
// its CPT 16-byte chunks in registers across the block reduction
// (CPT * 8 * 256 >= K); rows longer than that take a second read.
//
// The per-element quotient is not divided.  u = fma(x, inv, 128) with
// inv = 1/s correctly rounded once per row is the biased code before
// rounding: it lies within 2.3e-5 of the exact x/s + 128 (inv's error on
// |x/s| <= 127.00001, plus the fma's half ulp at 255), and the correctly
// rounded x/s within 3.8e-6 of the exact quotient, so rint(u) - 128 and
// round_half_away(x/s) agree unless u is within 2.7e-5 of a half-integer.
// A chunk with any element within 5e-5 of one is redone with the
// division.  |x/s| < 127.5, so the fast path needs no clamp; the bytes are
// packed biased (v_cvt_pk_u8_f32) and unbiased by flipping bit 7.  The
// codes are the division's, bit for bit.
//
// The bound needs inv to be a finite, correctly rounded reciprocal.  For a
// row whose absmax is below ~127 * 2^-128 (3.7e-37), s is so small that
// 1/s overflows to +inf; the caller then passes fast = false and every
// chunk of the row takes the division.  The redo test is written so that
// a NaN deviation (an inf or NaN product) also selects the division:
// fmaxf would drop a NaN, and `dev > limit` is false for one.
__device__ __forceinline__ uint2
quant8(const uint4 v, float s, float inv, bool fast)
{
  if (s == 0.0f) { return make_uint2(0u, 0u); }       // row of zeros
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
  float x[8];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    x[2 * e] = __uint_as_float(w[e] << 16);
    x[2 * e + 1] = __uint_as_float(w[e] & 0xffff0000u);
  }
  uint32_t packed[2] = {0u, 0u};
  bool redo = !fast;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float u = fmaf(x[e], inv, 128.0f);
    const float n = rintf(u);
    redo |= !(fabsf(u - n) <= 0.5f - 5e-5f);
    packed[e >> 2] = __builtin_amdgcn_cvt_pk_u8_f32(n, e & 3, packed[e >> 2]);
  }
  if (redo) {
    packed[0] = packed[1] = 0u;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float n = fminf(127.0f, fmaxf(-127.0f, roundf(x[e] / s)));
      packed[e >> 2] |= ((uint32_t)((int)n + 128)) << ((e & 3) * 8);
    }
  }
  return make_uint2(packed[0] ^ 0x80808080u, packed[1] ^ 0x80808080u);
}

__device__ __forceinline__ float
absmax8(const uint4 v, float amax)
{
  const uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    amax = fmaxf(amax, fabsf(bf16_to_f32(w[e] & 0xffffu)));
    amax = fmaxf(amax, fabsf(bf16_to_f32(w[e] >> 16)));
  }
  return amax;
}

template <int CPT>
__global__ __launch_bounds__(256) void
quant_rows_i8_kernel(const uint16_t* __restrict__ x, int K,
                     int8_t* __restrict__ q, float* __restrict__ sc)
{
  __shared__ float red[4];
  const int r = blockIdx.x;
  const uint4* xr = reinterpret_cast<const uint4*>(x + (size_t)r * K);
  const int nchunk = K / 8;
  uint4 v[CPT];
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = threadIdx.x + i * 256;
    v[i] = c < nchunk ? xr[c] : make_uint4(0u, 0u, 0u, 0u);
    amax = absmax8(v[i], amax);
  }
  for (int c = threadIdx.x + CPT * 256; c < nchunk; c += 256) {
    amax = absmax8(xr[c], amax);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) { amax = fmaxf(amax, __shfl_xor(amax, o)); }
  if ((threadIdx.x & 63) == 0) { red[threadIdx.x >> 6] = amax; }
  __syncthreads();
  amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float s = amax / 127.0f;
  const float inv = s != 0.0f ? 1.0f / s : 0.0f;
  // 1/s overflows for rows with absmax below ~3.7e-37: division only.
  const bool fast = inv <= 3.4028234663852886e38f;
  if (threadIdx.x == 0) { sc[r] = s; }
  uint2* qr = reinterpret_cast<uint2*>(q + (size_t)r * K);
#pragma unroll
  for (int i = 0; i < CPT; ++i) {
    const int c = threadIdx.x + i * 256;
    if (c < nchunk) { qr[c] = quant8(v[i], s, inv, fast); }
  }
  for (int c = threadIdx.x + CPT * 256; c < nchunk; c += 256) {
    qr[c] = quant8(xr[c], s, inv, fast);
  }
}

// Long rows (8192 < K <= 16384, K % 16 == 0): the same arithmetic with a
// 512-thread workgroup per row, each thread holding two adjacent 16-byte
// chunk pairs (chunks 2p, 2p + 1 of pairs p and p + 512) and writing each
// pair's 16 codes in one 16-byte store.  Measured at K = 12288, 4224 rows:
// 25.8 us (6.0 TB/s) against 31.2 us for the 256-thread form, whose
// 8-byte stores and six chunks per thread leave it latency bound.
__global__ __launch_bounds__(512) void
quant_rows_i8_wide_kernel(const uint16_t* __restrict__ x, int K,
                          int8_t* __restrict__ q, float* __restrict__ sc)
{
  __shared__ float red[8];
  const int r = blockIdx.x;
  const uint4* xr = reinterpret_cast<const uint4*>(x + (size_t)r * K);
  const int npair = K / 16;
  uint4 v[4];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int p = threadIdx.x + i * 512;
    if (p < npair) {
      v[2 * i] = xr[2 * p];
      v[2 * i + 1] = xr[2 * p + 1];
    } else {
      v[2 * i] = v[2 * i + 1] = make_uint4(0u, 0u, 0u, 0u);
    }
  }
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) { amax = absmax8(v[i], amax); }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) { amax = fmaxf(amax, __shfl_xor(amax, o)); }
  if ((threadIdx.x & 63) == 0) { red[threadIdx.x >> 6] = amax; }
  __syncthreads();
  amax = red[0];
#pragma unroll
  for (int w = 1; w < 8; ++w) { amax = fmaxf(amax, red[w]); }
  const float s = amax / 127.0f;
  const float inv = s != 0.0f ? 1.0f / s : 0.0f;
  const bool fast = inv <= 3.4028234663852886e38f;
  if (threadIdx.x == 0) { sc[r] = s; }
  uint4* qr = reinterpret_cast<uint4*>(q + (size_t)r * K);
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int p = threadIdx.x + i * 512;
    if (p < npair) {
      const uint2 a = quant8(v[2 * i], s, inv, fast);
      const uint2 b = quant8(v[2 * i + 1], s, inv, fast);
      qr[p] = make_uint4(a.x, a.y, b.x, b.y);
    }
  }
}

// Rows quantised by whole waves: WPR waves per row, RPB rows per
// workgroup, each lane holding CPL 16-byte chunks of its row in registers
// (row length K <= 512 * WPR * CPL).  Chunk i of wave part p, lane l is
// chunk i * 64 * WPR + p * 64 + l, so every load instruction reads 1 KiB
// of contiguous row and every store writes 512 contiguous bytes.  All of
// a lane's loads issue before the first use; loads past the row (or of a
// row past `rows`) read zeros through the buffer resource's range, and
// their stores are dropped the same way, so the body has no branches.
// With WPR == 1 the absmax is a wave reduction only (no LDS, no barrier).
template <int WPR, int CPL, int RPB>
__global__ __launch_bounds__(64 * WPR * RPB) void
quant_rows_i8_waves_kernel(const uint16_t* __restrict__ x, int rows, int K,
                           int8_t* __restrict__ q, float* __restrict__ sc)
{
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int rib = wave / WPR;                  // row in block
  const int part = wave % WPR;
  const int r = blockIdx.x * RPB + rib;
  const bool valid = r < rows;
  const int rr = valid ? r : 0;
  const __amdgpu_buffer_rsrc_t src =
      make_rsrc(x + (size_t)rr * K, valid ? K * 2 : 0);
  const __amdgpu_buffer_rsrc_t dst = make_rsrc(q + (size_t)rr * K, valid ? K : 0);
  u32x4_t v[CPL];
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = i * 64 * WPR + part * 64 + lane;
    v[i] = __builtin_amdgcn_raw_buffer_load_b128(src, c * 16, 0, 0);
  }
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    amax = absmax8(make_uint4(v[i].x, v[i].y, v[i].z, v[i].w), amax);
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) { amax = fmaxf(amax, __shfl_xor(amax, o)); }
  if constexpr (WPR > 1) {
    __shared__ float red[RPB][WPR];
    if (lane == 0) { red[rib][part] = amax; }
    __syncthreads();
    amax = red[rib][0];
#pragma unroll
    for (int w = 1; w < WPR; ++w) { amax = fmaxf(amax, red[rib][w]); }
  }
  const float s = amax / 127.0f;
  const float inv = s != 0.0f ? 1.0f / s : 0.0f;
  // 1/s overflows for rows with absmax below ~3.7e-37: division only.
  const bool fast = inv <= 3.4028234663852886e38f;
  if (valid && part == 0 && lane == 0) { sc[r] = s; }
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = i * 64 * WPR + part * 64 + lane;
    const uint2 o = quant8(make_uint4(v[i].x, v[i].y, v[i].z, v[i].w), s, inv, fast);
    __builtin_amdgcn_raw_buffer_store_b64((u32x2_t){o.x, o.y}, dst, c * 8, 0, 0);
  }
}

// ---- RMSNorm with gain, its int8 form, and the residual add before it --------
// Rows normalised by whole waves, the quantiser's layout: WPR waves per row
// (one row per workgroup), each lane holding CPL 16-byte chunks of its row
// in registers (dim <= 512 * WPR * CPL); chunk i of wave p, lane l is
// chunk i * 64 * WPR + p * 64 + l.  Loads past the row read zeros through
// the buffer resource's range and stores past it are dropped.
//   ADD:  x = bf16(x + d) first, stored back to x (the residual stream),
//         and the row normalised from those bf16 values;
//   y = bf16((x * inv) * w),  inv = rsqrt(sum(x^2) / dim + eps),
// the sum in f32 (lane partials, then the wave and the row by xor shuffles
// and LDS); rows below m_und take w_und, the rest w_gen.  QUANT: the row's
// bf16 results, as they would be read back, give its int8 scale and codes
// by the quantiser's own steps (absmax8, quant8), so (q, sc) equal
// quant_rows_i8 applied to y bit for bit; y itself is stored only when `y`
// is not null.  y may be x: every store of a row depends on the row's sum,
// so all of its loads come first.
template <int WPR, int CPL, bool QUANT, bool ADD>
__global__ __launch_bounds__(64 * WPR) void
rms_norm_rows_kernel(uint16_t* x, const uint16_t* __restrict__ d,
                     const uint16_t* __restrict__ w_und,
                     const uint16_t* __restrict__ w_gen, int m_und, int dim,
                     float eps, uint16_t* y, int8_t* __restrict__ q,
                     float* __restrict__ sc)
{
  const int part = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x;
  const __amdgpu_buffer_rsrc_t src = make_rsrc(x + (size_t)r * dim, dim * 2);
  const __amdgpu_buffer_rsrc_t wsrc = make_rsrc(r < m_und ? w_und : w_gen, dim * 2);
  u32x4_t v[CPL], g[CPL];
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = i * 64 * WPR + part * 64 + lane;
    v[i] = __builtin_amdgcn_raw_buffer_load_b128(src, c * 16, 0, 0);
    g[i] = __builtin_amdgcn_raw_buffer_load_b128(wsrc, c * 16, 0, 0);
  }
  if constexpr (ADD) {
    const __amdgpu_buffer_rsrc_t dsrc = make_rsrc(d + (size_t)r * dim, dim * 2);
    u32x4_t dv[CPL];
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int c = i * 64 * WPR + part * 64 + lane;
      dv[i] = __builtin_amdgcn_raw_buffer_load_b128(dsrc, c * 16, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const uint32_t xv[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
      const uint32_t ev[4] = {dv[i].x, dv[i].y, dv[i].z, dv[i].w};
      uint32_t o[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        o[e] = pack_bf16x2(__uint_as_float(xv[e] << 16) + __uint_as_float(ev[e] << 16),
                           __uint_as_float(xv[e] & 0xffff0000u) +
                               __uint_as_float(ev[e] & 0xffff0000u));
      }
      v[i] = (u32x4_t){o[0], o[1], o[2], o[3]};
    }
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int c = i * 64 * WPR + part * 64 + lane;
      __builtin_amdgcn_raw_buffer_store_b128(v[i], src, c * 16, 0, 0);
    }
  }
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const uint32_t wv[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float lo = __uint_as_float(wv[e] << 16);
      const float hi = __uint_as_float(wv[e] & 0xffff0000u);
      ss += lo * lo;
      ss += hi * hi;
    }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) { ss += __shfl_xor(ss, o); }
  __shared__ float red[2][WPR];
  if constexpr (WPR > 1) {
    if (lane == 0) { red[0][part] = ss; }
    __syncthreads();
    ss = red[0][0];
#pragma unroll
    for (int p = 1; p < WPR; ++p) { ss += red[0][p]; }
  }
  const float inv = rsqrtf(ss / (float)dim + eps);
  uint4 out[CPL];
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const uint32_t xv[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
    const uint32_t gv[4] = {g[i].x, g[i].y, g[i].z, g[i].w};
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float lo = (__uint_as_float(xv[e] << 16) * inv) * __uint_as_float(gv[e] << 16);
      const float hi = (__uint_as_float(xv[e] & 0xffff0000u) * inv) *
                       __uint_as_float(gv[e] & 0xffff0000u);
      o[e] = pack_bf16x2(lo, hi);
    }
    out[i] = make_uint4(o[0], o[1], o[2], o[3]);
  }
  if (!QUANT || y != nullptr) {
    const __amdgpu_buffer_rsrc_t dst = make_rsrc(y + (size_t)r * dim, dim * 2);
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int c = i * 64 * WPR + part * 64 + lane;
      __builtin_amdgcn_raw_buffer_store_b128(
          (u32x4_t){out[i].x, out[i].y, out[i].z, out[i].w}, dst, c * 16, 0, 0);
    }
  }
  if constexpr (QUANT) {
    // chunks past the row hold bf16(0 * inv * 0) = 0: they leave the
    // absmax alone and their codes are dropped by the range
    float amax = 0.0f;
#pragma unroll
    for (int i = 0; i < CPL; ++i) { amax = absmax8(out[i], amax); }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) { amax = fmaxf(amax, __shfl_xor(amax, o)); }
    if constexpr (WPR > 1) {
      if (lane == 0) { red[1][part] = amax; }
      __syncthreads();
      amax = red[1][0];
#pragma unroll
      for (int p = 1; p < WPR; ++p) { amax = fmaxf(amax, red[1][p]); }
    }
    const float s = amax / 127.0f;
    const float qinv = s != 0.0f ? 1.0f / s : 0.0f;
    // 1/s overflows for rows with absmax below ~3.7e-37: division only.
    const bool fast = qinv <= 3.4028234663852886e38f;
    if (part == 0 && lane == 0) { sc[r] = s; }
    const __amdgpu_buffer_rsrc_t qd = make_rsrc(q + (size_t)r * dim, dim);
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int c = i * 64 * WPR + part * 64 + lane;
      const uint2 o = quant8(out[i], s, qinv, fast);
      __builtin_amdgcn_raw_buffer_store_b64((u32x2_t){o.x, o.y}, qd, c * 8, 0, 0);
    }
  }
}

// ---- SwiGLU with the int8 tier's per-token quantisation ---------------------
// The down projection's int8 input in one pass: h = swiglu(gate, up) per
// element (swiglu_f, the elementwise kernel's arithmetic), then the row's
// absmax, scale and codes by the quantiser's own steps, so (q, sc) equal
// quant_rows_i8 on swiglu's output bit for bit; h is stored only when not
// null.  The rows' layout is rms_norm_rows_kernel's (dim <= 512 * WPR * CPL).
template <int WPR, int CPL>
__global__ __launch_bounds__(64 * WPR) void
swiglu_quant_rows_kernel(const uint16_t* __restrict__ gate,
                         const uint16_t* __restrict__ up, int dim,
                         uint16_t* __restrict__ h, int8_t* __restrict__ q,
                         float* __restrict__ sc)
{
  const int part = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x;
  const __amdgpu_buffer_rsrc_t gs = make_rsrc(gate + (size_t)r * dim, dim * 2);
  const __amdgpu_buffer_rsrc_t us = make_rsrc(up + (size_t)r * dim, dim * 2);
  u32x4_t gv[CPL], uv[CPL];
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = i * 64 * WPR + part * 64 + lane;
    gv[i] = __builtin_amdgcn_raw_buffer_load_b128(gs, c * 16, 0, 0);
    uv[i] = __builtin_amdgcn_raw_buffer_load_b128(us, c * 16, 0, 0);
  }
  uint4 out[CPL];
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const uint32_t ga[4] = {gv[i].x, gv[i].y, gv[i].z, gv[i].w};
    const uint32_t ua[4] = {uv[i].x, uv[i].y, uv[i].z, uv[i].w};
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      o[e] = pack_bf16x2(swiglu_f(bf16_to_f32(ga[e] & 0xffffu), bf16_to_f32(ua[e] & 0xffffu)),
                         swiglu_f(bf16_to_f32(ga[e] >> 16), bf16_to_f32(ua[e] >> 16)));
    }
    out[i] = make_uint4(o[0], o[1], o[2], o[3]);
  }
  if (h != nullptr) {
    const __amdgpu_buffer_rsrc_t hd = make_rsrc(h + (size_t)r * dim, dim * 2);
#pragma unroll
    for (int i = 0; i < CPL; ++i) {
      const int c = i * 64 * WPR + part * 64 + lane;
      __builtin_amdgcn_raw_buffer_store_b128(
          (u32x4_t){out[i].x, out[i].y, out[i].z, out[i].w}, hd, c * 16, 0, 0);
    }
  }
  // chunks past the row hold swiglu(0, 0) = 0 and leave the absmax alone
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < CPL; ++i) { amax = absmax8(out[i], amax); }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) { amax = fmaxf(amax, __shfl_xor(amax, o)); }
  if constexpr (WPR > 1) {
    __shared__ float red[WPR];
    if (lane == 0) { red[part] = amax; }
    __syncthreads();
    amax = red[0];
#pragma unroll
    for (int p = 1; p < WPR; ++p) { amax = fmaxf(amax, red[p]); }
  }
  const float s = amax / 127.0f;
  const float qinv = s != 0.0f ? 1.0f / s : 0.0f;
  // 1/s overflows for rows with absmax below ~3.7e-37: division only.
  const bool fast = qinv <= 3.4028234663852886e38f;
  if (part == 0 && lane == 0) { sc[r] = s; }
  const __amdgpu_buffer_rsrc_t qd = make_rsrc(q + (size_t)r * dim, dim);
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = i * 64 * WPR + part * 64 + lane;
    const uint2 o = quant8(out[i], s, qinv, fast);
    __builtin_amdgcn_raw_buffer_store_b64((u32x2_t){o.x, o.y}, qd, c * 8, 0, 0);
  }
}

// ---- dst += src, the residual add (bf16, f32 add, one rounding) ------------
// Eight elements per thread where both pointers are 16-byte aligned; the
// tail (and misaligned operands) one element per thread.
__global__ __launch_bounds__(256) void
add_bf16_kernel(uint16_t* __restrict__ dst, const uint16_t* __restrict__ src,
                int64_t n, int64_t nvec)
{
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < nvec; i += stride) {
    const uint4 a = reinterpret_cast<const uint4*>(dst)[i];
    const uint4 b = reinterpret_cast<const uint4*>(src)[i];
    const uint32_t aw[4] = {a.x, a.y, a.z, a.w};
    const uint32_t bw[4] = {b.x, b.y, b.z, b.w};
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      o[e] = pack_bf16x2(__uint_as_float(aw[e] << 16) + __uint_as_float(bw[e] << 16),
                         __uint_as_float(aw[e] & 0xffff0000u) +
                             __uint_as_float(bw[e] & 0xffff0000u));
    }
    reinterpret_cast<uint4*>(dst)[i] = make_uint4(o[0], o[1], o[2], o[3]);
  }
  for (int64_t i = nvec * 8 + (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += stride) {
    dst[i] = (uint16_t)bf16_bits(bf16_to_f32(dst[i]) + bf16_to_f32(src[i]));
  }
}

// ---- elementwise SwiGLU: out = silu(g) * u ------------------------------
__global__ __launch_bounds__(256) void
swiglu_kernel(const uint4* __restrict__ g, const uint4* __restrict__ u,
              uint4* __restrict__ o, int64_t nvec)
{
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < nvec;
       i += stride) {
    const uint4 gv = g[i], uv = u[i];
    const uint32_t gw[4] = {gv.x, gv.y, gv.z, gv.w};
    const uint32_t uw[4] = {uv.x, uv.y, uv.z, uv.w};
    uint32_t ow[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float g0 = bf16_to_f32(gw[e] & 0xffffu), g1 = bf16_to_f32(gw[e] >> 16);
      const float u0 = bf16_to_f32(uw[e] & 0xffffu), u1 = bf16_to_f32(uw[e] >> 16);
      ow[e] = pack_bf16x2(swiglu_f(g0, u0), swiglu_f(g1, u1));
    }
    o[i] = make_uint4(ow[0], ow[1], ow[2], ow[3]);
  }
}

// ---- affine-quantized weights: dequant once to bf16 ----------------------
// One thread per u32 code word (32/BITS codes of one row): w = scale * code
// + bias of the code's group, a multiply then an add in f32 (contraction
// into a fused multiply-add is switched off: it would round differently
// from the pack fixture's arithmetic where the product is subnormal),
// rounded to bf16 to nearest even by v_cvt_pk_bf16_f32.
template <int BITS>
__global__ __launch_bounds__(256) void
dequant_affine_kernel(const uint32_t* __restrict__ codes,
                      const uint16_t* __restrict__ sc,
                      const uint16_t* __restrict__ bi, int group, int N, int K,
                      uint16_t* __restrict__ w)
{
  constexpr int kPer = 32 / BITS;
  constexpr uint32_t kMask = (1u << BITS) - 1u;
  const int words = K / kPer;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)N * words) { return; }
  const int n = (int)(idx / words);
  const int wi = (int)(idx % words);
  const int k0 = wi * kPer;
  const int gidx = n * (K / group) + k0 / group;   // kPer divides group
  const float s = bf16_to_f32(sc[gidx]);
  const float b = bf16_to_f32(bi[gidx]);
  const uint32_t word = codes[idx];
  uint32_t out[kPer / 2];
#pragma unroll
  for (int e = 0; e < kPer; e += 2) {
    float p0 = s * (float)((word >> (e * BITS)) & kMask);
    float p1 = s * (float)((word >> ((e + 1) * BITS)) & kMask);
    asm("" : "+v"(p0), "+v"(p1));     // the products stay rounded: no fma
    out[e / 2] = pack_bf16x2(p0 + b, p1 + b);
  }
  uint16_t* dst = w + (size_t)n * K + k0;
  if constexpr (BITS == 8) {
    *reinterpret_cast<uint2*>(dst) = make_uint2(out[0], out[1]);
  } else {
    *reinterpret_cast<uint4*>(dst) = make_uint4(out[0], out[1], out[2], out[3]);
  }
}

// ---- y += bias, broadcast over rows (bf16, f32 add) ---------------------
__global__ __launch_bounds__(256) void
bias_add_kernel(uint16_t* __restrict__ y, const uint16_t* __restrict__ b,
                int N, int64_t nvec)
{
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < nvec;
       i += stride) {
    const int64_t e0 = i * 8;
    const int n0 = (int)(e0 % N);
    uint4 v = reinterpret_cast<uint4*>(y)[i];
    const uint4 bb = *reinterpret_cast<const uint4*>(b + n0);
    const uint32_t yw[4] = {v.x, v.y, v.z, v.w};
    const uint32_t bw[4] = {bb.x, bb.y, bb.z, bb.w};
    uint32_t o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float lo = bf16_to_f32(yw[e] & 0xffffu) + bf16_to_f32(bw[e] & 0xffffu);
      const float hi = bf16_to_f32(yw[e] >> 16) + bf16_to_f32(bw[e] >> 16);
      o[e] = bf16_bits(lo) | (bf16_bits(hi) << 16);
    }
    reinterpret_cast<uint4*>(y)[i] = make_uint4(o[0], o[1], o[2], o[3]);
  }
}

// ---- f32 -> bf16, round to nearest even ----------------------------------
__global__ __launch_bounds__(256) void
f32_to_bf16_kernel(const float4* __restrict__ src, uint2* __restrict__ dst,
                   int64_t nvec)
{
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < nvec;
       i += stride) {
    const float4 v = src[i];
    dst[i] = make_uint2(bf16_bits(v.x) | (bf16_bits(v.y) << 16),
                        bf16_bits(v.z) | (bf16_bits(v.w) << 16));
  }
}

// ---- split q/k norm and three-way split RoPE ------------------------------
// x [T][H*D] bf16 in place, one wave per (token, head) row of D elements,
// four rows per workgroup.  The row is staged in LDS (f32) so the rotation
// can read each element's partner, which sits in another lane.
//   NORM: the halves [0, D/2) and [D/2, D) are RMS-normalised separately,
//         y = x * rsqrt(mean(half^2) + eps) * w (w_t, w_hw), sums in f32.
//   ROPE: rotate_half on the ranges [0,d_t) (t), [d_t,d_t+d_h) (h) and
//         [d_t+d_h,D) (w) with the packed f32 tables cos/sin [T][D]:
//         out[j] = x[j] c[j] - x[j+r] s[j],  out[j+r] = x[j+r] c[j+r] +
//         x[j] s[j+r] (r = half the range; the tables are doubled).
// With both, the normalised row stays in f32 between the two steps.
constexpr int kNormRopeMaxD = 512;

template <bool NORM, bool ROPE>
__global__ __launch_bounds__(256) void
split_norm_rope_kernel(uint16_t* __restrict__ x,
                       const uint16_t* __restrict__ w_t,
                       const uint16_t* __restrict__ w_hw,
                       const float* __restrict__ cosf,
                       const float* __restrict__ sinf, int rows, int H, int D,
                       int d_t, int d_h, float eps)
{
  __shared__ float buf[4][kNormRopeMaxD];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + wave;
  const bool active = row < rows;
  const int half = D >> 1;
  float* b = buf[wave];
  uint16_t* xr = x + (size_t)(active ? row : 0) * D;
  float st = 0.0f, sh = 0.0f;
  if (active) {
    for (int i = lane; i < D; i += 64) {
      const float v = bf16_to_f32(xr[i]);
      b[i] = v;
      if (i < half) { st += v * v; } else { sh += v * v; }
    }
  }
  if constexpr (NORM) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      st += __shfl_xor(st, o);
      sh += __shfl_xor(sh, o);
    }
    const float it = rsqrtf(st / (float)half + eps);
    const float ih = rsqrtf(sh / (float)half + eps);
    if (active) {
      for (int i = lane; i < D; i += 64) {
        b[i] = i < half ? b[i] * it * bf16_to_f32(w_t[i])
                        : b[i] * ih * bf16_to_f32(w_hw[i - half]);
      }
    }
  }
  __syncthreads();
  if (!active) { return; }
  const int t = row / H;
  for (int i = lane; i < D; i += 64) {
    float v = b[i];
    if constexpr (ROPE) {
      const int off = i < d_t ? 0 : (i < d_t + d_h ? d_t : d_t + d_h);
      const int r = (i < d_t ? d_t : d_h) >> 1;
      const int j = i - off;
      const float c = cosf[(size_t)t * D + i];
      const float sn = sinf[(size_t)t * D + i];
      v = j < r ? v * c - b[i + r] * sn : v * c + b[i - r] * sn;
    }
    xr[i] = (uint16_t)bf16_bits(v);
  }
}

// The same pass with one thread per 16-byte chunk (8 elements), the row's
// D/8 chunks on D/8 adjacent lanes: the half sums reduce by xor shuffles
// over the D/16 lanes of each half, and an element's rotation partner, r
// elements away (r = half its range), sits on the lane r/8 away (xor, as
// every range starts at a multiple of its own width).  Shapes: D a power of
// two in [16, 512], d_t/16 and d_h/16 powers of two, d_h dividing d_t.
// Every lane of a row runs this (the shuffles read the row's other lanes).
// `w_t`/`w_hw` are the norm weights, `cs`/`sn` the chunk's 8 table entries.
template <bool NORM, bool ROPE>
__device__ __forceinline__ void
norm_rope_chunk(float (&v)[8], int c, int D, int d_t, int d_h, float eps,
                const uint16_t* w_t, const uint16_t* w_hw, const float (&cs)[8],
                const float (&sn)[8])
{
  const int cpr = D >> 3;                          // chunks (lanes) per row
  const int hc = cpr >> 1;                         // chunks per half
  if constexpr (NORM) {
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) { ss += v[i] * v[i]; }
    for (int o = 1; o < hc; o <<= 1) { ss += __shfl_xor(ss, o); }
    const float inv = rsqrtf(ss / (float)(D >> 1) + eps);
    const uint16_t* w = c < hc ? w_t + c * 8 : w_hw + (c - hc) * 8;
    const i32x4_t wr = *reinterpret_cast<const i32x4_t*>(w);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = v[2 * i] * inv * __uint_as_float((uint32_t)wr[i] << 16);
      v[2 * i + 1] = v[2 * i + 1] * inv * __uint_as_float((uint32_t)wr[i] & 0xffff0000u);
    }
  }
  if constexpr (ROPE) {
    const int e0 = c * 8;
    const int off = e0 < d_t ? 0 : (e0 < d_t + d_h ? d_t : d_t + d_h);
    const int r = (e0 < d_t ? d_t : d_h) >> 1;
    const bool lower = e0 - off < r;
    float vp[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) { vp[i] = __shfl_xor(v[i], r >> 3); }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      v[i] = lower ? v[i] * cs[i] - vp[i] * sn[i] : v[i] * cs[i] + vp[i] * sn[i];
    }
  }
}

// The 8 cos and sin entries of chunk c of one token's table rows.
__device__ __forceinline__ void
load_rope_chunk(const float* cp, const float* sp, int c, float (&cs)[8],
                float (&sn)[8])
{
  const int e0 = c * 8;
  *reinterpret_cast<i32x4_t*>(cs) = *reinterpret_cast<const i32x4_t*>(cp + e0);
  *reinterpret_cast<i32x4_t*>(cs + 4) = *reinterpret_cast<const i32x4_t*>(cp + e0 + 4);
  *reinterpret_cast<i32x4_t*>(sn) = *reinterpret_cast<const i32x4_t*>(sp + e0);
  *reinterpret_cast<i32x4_t*>(sn + 4) = *reinterpret_cast<const i32x4_t*>(sp + e0 + 4);
}

__device__ __forceinline__ void
unpack_bf16x8(const i32x4_t raw, float (&v)[8])
{
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = __uint_as_float((uint32_t)raw[i] << 16);
    v[2 * i + 1] = __uint_as_float((uint32_t)raw[i] & 0xffff0000u);
  }
}

__device__ __forceinline__ i32x4_t
pack_bf16x8(const float (&v)[8])
{
  i32x4_t o;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    o[i] = (int)(bf16_bits(v[2 * i]) | (bf16_bits(v[2 * i + 1]) << 16));
  }
  return o;
}

template <bool NORM, bool ROPE>
__global__ __launch_bounds__(256) void
split_norm_rope_vec_kernel(uint16_t* __restrict__ x,
                           const uint16_t* __restrict__ w_t,
                           const uint16_t* __restrict__ w_hw,
                           const float* __restrict__ cosf,
                           const float* __restrict__ sinf, int rows, int H,
                           int D, int d_t, int d_h, float eps)
{
  const int cpr = D >> 3;
  const long long gid = (long long)blockIdx.x * 256 + threadIdx.x;
  const long long row = gid / cpr;
  const int c = (int)(gid % cpr);
  const bool active = row < rows;
  uint16_t* p = x + (active ? row : 0) * D + c * 8;
  const i32x4_t raw = active ? *reinterpret_cast<const i32x4_t*>(p) : i32x4_t{0, 0, 0, 0};
  float v[8];
  unpack_bf16x8(raw, v);
  float cs[8], sn[8];
  if constexpr (ROPE) {
    const long long t = (active ? row : 0) / H;
    load_rope_chunk(cosf + t * D, sinf + t * D, c, cs, sn);
  }
  norm_rope_chunk<NORM, ROPE>(v, c, D, d_t, d_h, eps, w_t, w_hw, cs, sn);
  if (!active) { return; }
  *reinterpret_cast<i32x4_t*>(p) = pack_bf16x8(v);
}

// The attention prologue of a two-group pass (PrologueArgs), one thread
// per 16-byte chunk as above, each thread holding that chunk of RPT heads
// of one token (the token's table entries loaded once for all of them).
// The grid is three runs of whole workgroups: q rows (token-major [t][h],
// normed and rotated in place), k rows (normed and rotated, stored to
// k_cache[h][offset + t]) and v rows (copied to v_cache[h][offset + t]),
// so every branch below is uniform per workgroup.  Rows of tokens below
// m_und take the und norm weights.  RPT divides hq and hkv.
template <int RPT>
__global__ __launch_bounds__(256) void
attention_prologue_kernel(const PrologueArgs a)
{
  const int D = a.d;
  const int cpr = D >> 3;
  const int gpb = 256 / cpr;                       // head groups per workgroup
  const long long nq = (long long)a.tokens * (a.hq / RPT);
  const long long nk = (long long)a.tokens * (a.hkv / RPT);
  const long long bq = (nq + gpb - 1) / gpb;
  const long long bk = (nk + gpb - 1) / gpb;
  long long blk = blockIdx.x;
  int part;                                        // 0 q, 1 k, 2 v
  long long ngroups;
  if (blk < bq) {
    part = 0; ngroups = nq;
  } else if (blk < bq + bk) {
    part = 1; ngroups = nk; blk -= bq;
  } else {
    part = 2; ngroups = nk; blk -= bq + bk;
  }
  const long long grp = blk * gpb + threadIdx.x / cpr;
  const int c = threadIdx.x % cpr;
  const bool active = grp < ngroups;
  const long long gg = active ? grp : 0;
  const int H = part == 0 ? a.hq : a.hkv;
  const long long t = gg / (H / RPT);
  const int h0 = (int)(gg % (H / RPT)) * RPT;
  const uint16_t* src = (part == 0 ? a.q : (part == 1 ? a.k : a.v)) +
                        (t * H + h0) * D + c * 8;
  i32x4_t raw[RPT];
#pragma unroll
  for (int j = 0; j < RPT; ++j) {
    raw[j] = active ? *reinterpret_cast<const i32x4_t*>(src + j * D)
                    : i32x4_t{0, 0, 0, 0};
  }
  if (part == 2) {
    if (active) {
#pragma unroll
      for (int j = 0; j < RPT; ++j) {
        *reinterpret_cast<i32x4_t*>(
            a.v_cache + ((long long)(h0 + j) * a.cap + a.offset + t) * D + c * 8) = raw[j];
      }
    }
    return;
  }
  float cs[8], sn[8];
  load_rope_chunk(a.cosf + t * D, a.sinf + t * D, c, cs, sn);
  const int e = t < a.m_und ? 0 : 1;
  const uint16_t* w_t = a.w[e][2 * part];
  const uint16_t* w_hw = a.w[e][2 * part + 1];
  i32x4_t out[RPT];
#pragma unroll
  for (int j = 0; j < RPT; ++j) {
    float v[8];
    unpack_bf16x8(raw[j], v);
    norm_rope_chunk<true, true>(v, c, D, a.d_t, a.d_h, a.eps, w_t, w_hw, cs, sn);
    out[j] = pack_bf16x8(v);
  }
  if (!active) { return; }
#pragma unroll
  for (int j = 0; j < RPT; ++j) {
    uint16_t* dst = part == 0
        ? a.q + (t * H + h0 + j) * D
        : a.k_cache + ((long long)(h0 + j) * a.cap + a.offset + t) * D;
    *reinterpret_cast<i32x4_t*>(dst + c * 8) = out[j];
  }
}

// ---- f16 -> bf16, the loader's conversion -----------------------------------
// Widen f16 to f32 with integer operations (subnormals renormalised; Inf
// and NaN keep their payload bits, which the hardware conversion would
// quiet), then the same RNE as every other bf16 rounding here.
__device__ __forceinline__ uint32_t
f16_bits_to_bf16(uint32_t h)
{
  const uint32_t sign = (h & 0x8000u) << 16;
  uint32_t exp = (h >> 10) & 0x1fu;
  uint32_t man = h & 0x3ffu;
  uint32_t f;
  if (exp == 0) {
    if (man == 0) {
      f = sign;
    } else {
      // a subnormal: shift the leading one into the implicit position
      const int lz = __clz(man) - 21;            // leading zeros in 11 bits
      man = (man << lz) & 0x3ffu;
      f = sign | ((uint32_t)(127 - 15 + 1 - lz) << 23) | (man << 13);
    }
  } else if (exp == 31) {
    f = sign | 0x7f800000u | (man << 13);
  } else {
    f = sign | ((exp - 15 + 127) << 23) | (man << 13);
  }
  return (f + ((f >> 16) & 1u) + 0x7fffu) >> 16;
}

__global__ __launch_bounds__(256) void
f16_to_bf16_kernel(const uint2* __restrict__ src, uint2* __restrict__ dst,
                   int64_t nvec)
{
  const int64_t stride = (int64_t)gridDim.x * 256;
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < nvec;
       i += stride) {
    const uint2 v = src[i];
    dst[i] = make_uint2(f16_bits_to_bf16(v.x & 0xffffu) |
                            (f16_bits_to_bf16(v.x >> 16) << 16),
                        f16_bits_to_bf16(v.y & 0xffffu) |
                            (f16_bits_to_bf16(v.y >> 16) << 16));
  }
}

// ---- flash attention ------------------------------------------------------
// Grouped-query attention over a K/V cache, one workgroup per 32 * NWV
// queries of one head (NWV waves of 32: 8 bidirectional, 4 causal), keys
// streamed in tiles of 64.
//
// The score tile is computed TRANSPOSED, S^T = K Q^T, with the key
// fragment as the MFMA's first operand: a lane then holds 32 scores (two
// 32-key blocks) of ONE query, its column, so the online softmax is per
// lane plus one exchange with the lane 32 apart, and the output rescale is
// one scalar per lane.  The output is accumulated transposed too,
// O^T = V^T P^T: the second operand is P^T, whose lane layout (8 keys of
// one query) is exactly the lane's own probabilities when the keys of each
// 16 are taken in the order the score layout holds them (key 8*(e/4) +
// 4*half + e%4 at operand position 8*half + e).  The first operand, V^T,
// comes from V in its natural [key][dim] layout by LDS transpose reads:
// ds_read_b64_tr_b16 hands lane B+i of each 16-lane group element i%4 of
// the 4-element chunks addressed by lanes B + i/4 + 4j, j = 0..3, so lane
// s addresses dims 16*((s/16)%2) + 4*(s%4) of key 4*half + (s%16)/4 (and
// that key + 8 for the second read).
//
// Software pipeline, one barrier per tile: iteration t takes the scores of
// tile t+1 (MFMA) while it exponentiates tile t (VALU), then accumulates
// tile t's P V; K of tile t+2 and V of tile t+1 are copied global -> LDS
// directly (no registers) meanwhile.  Each buffer is its own __shared__
// object and the loop is unrolled by two so every buffer choice is static:
// the compiler then knows a copy into one buffer does not alias reads of
// the other and does not hold those reads until the copy lands.
//
// The softmax work per score is one FMA (scale and running max), one
// exp2, one add and half a bf16 pack; a tile needing no mask (every key
// below tk and, for the causal masks, below the workgroup's first query)
// skips the mask.  The running max m is raised only when a tile's max
// exceeds it by more than kLazy/scale: until then probabilities are
// exp2((s - m) * scale) <= 2^kLazy, and the output and the sum share the
// same m, so the quotient is unchanged while most tiles skip the rescale.
//
// LDS layouts (per buffer): K [64][D] with 16-byte chunk c of row r at
// c ^ (r % (D/8)), so a fragment read (32 rows at one chunk) spreads over
// the banks; V [64][D] with 64-byte block b of row r at b ^ vswz(r), so
// the transpose reads (4 rows x 64 bytes per half-wave) hit every bank
// once.  The copies place each lane's 16 bytes at its landing slot and
// fetch the chunk the swizzle puts there.  K and V are read through
// buffer resources bounded at tk keys: keys past tk read as zeros and are
// masked to -inf, which adds 0 to every sum.
// max of v over lanes l and l ^ 32
__device__ __forceinline__ float
max_halves(float v)
{
  const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(v),
                                                  __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
}

__device__ __forceinline__ float
sum_halves(float v)
{
  const auto s = __builtin_amdgcn_permlane32_swap(__float_as_uint(v),
                                                  __float_as_uint(v), false, false);
  return __uint_as_float(s[0]) + __uint_as_float(s[1]);
}

constexpr float kLazy = 8.0f;

// Waves (32 queries each) per attention workgroup.  Bidirectional: 8, so
// each K/V tile copied into LDS serves 256 queries (the generation pass
// 0.295-0.302 ms against 0.309-0.311 with 4).  The causal masks keep 4:
// a workgroup runs to the last key its last query sees, and 256-query
// workgroups waste more masked keys (causal 12% slower with 8).
template <int MODE>
constexpr int attn_waves()
{
  return MODE == 0 ? 8 : 4;
}

// 64-byte block swizzle of V row r: four consecutive rows at one block
// land on four different 64-byte bank ranges
template <int D>
__device__ __forceinline__ int
vswz(int r)
{
  return (r * (D / 32) / 4) % (D / 32);
}

typedef short i16x4_t __attribute__((ext_vector_type(4)));
typedef short i16x2_t __attribute__((ext_vector_type(2)));

template <int D, int MODE, int NWV>
__global__ __launch_bounds__(64 * NWV, 8 / NWV) void
attention_kernel(const AttnArgs A)
{
  constexpr int BK = 64;
  constexpr int KCH = D / 8;                 // 16-byte chunks per row
  constexpr int NDS = D / 16;                // MFMA K-steps of the scores
  constexpr int NCB = D / 32;                // 32-row blocks of O^T
  constexpr int QT = 32 * NWV;               // queries per workgroup
  constexpr int kTileKiB = BK * D * 2 / 1024;
  // 1 KiB copies per copying wave per tile, and the waves that copy
  constexpr int CPW = kTileKiB >= NWV ? kTileKiB / NWV : 1;
  constexpr int kCopyWaves = kTileKiB / CPW;
  // Tile j's K sits in ks<j & 1>, its V in vs<j & 1>, its t entries in
  // ts[j % 3]: iteration t reads K of tile t+1, V and t of tile t, and
  // writes K of tile t+2, V of tile t+1, t of tile t+2.
  __shared__ __attribute__((aligned(16))) uint16_t ks0[BK * D];
  __shared__ __attribute__((aligned(16))) uint16_t ks1[BK * D];
  __shared__ __attribute__((aligned(16))) uint16_t vs0[BK * D];
  __shared__ __attribute__((aligned(16))) uint16_t vs1[BK * D];
  __shared__ int32_t ts[3][BK];
  // block-causal: whether every key of the tile in ts[i] carries the one t
  // all the workgroup's queries share (then the tile needs no mask)
  __shared__ int32_t tsame[3];

  // Work item: (query head, 128-query tile), ordered kv head first, so
  // that cutting the list into 8 runs (one per XCD, workgroups b, b+8, ...
  // run on XCD b % 8) keeps each kv head's keys in one XCD's L2.
  const int ntq = (A.tq + QT - 1) / QT;
  const int items = A.hq * ntq;
  const int b = blockIdx.x;
  const int item = (items % 8 == 0) ? (b % 8) * (items / 8) + b / 8 : b;
  const int h = item / ntq;
  // With a mask, later query tiles see more keys: they are dealt first, so
  // the long workgroups start early instead of forming the tail.
  const int qt = MODE == 0 ? item % ntq : ntq - 1 - item % ntq;
  const int kvh = h / (A.hq / A.hkv);

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);   // wave-uniform
  const int lane = tid & 63;
  const int lq = lane & 31;
  const int half = lane >> 5;
  const int qrow = qt * QT + wave * 32 + lq;      // this lane's query
  const bool qvalid = qrow < A.tq;
  const int qpos = A.q_offset + qrow;
  const float scale = 1.4426950408889634f * rsqrtf((float)D);
  const float lazy = kLazy / scale;               // in raw score units

  i32x4_t qf[NDS];
  const uint16_t* qp = A.q + (long long)h * A.q_head + (long long)qrow * A.q_tok;
#pragma unroll
  for (int ds = 0; ds < NDS; ++ds) {
    qf[ds] = qvalid ? *reinterpret_cast<const i32x4_t*>(qp + ds * 16 + half * 8)
                    : i32x4_t{0, 0, 0, 0};
  }
  int tq_idx = 0;
  if constexpr (MODE == 2) { tq_idx = qvalid ? A.t_index[qpos] : 0; }

  // ---- tile copies: global -> LDS ------------------------------------------
  // Each copy reads through a buffer resource based at the tile's first key
  // whose range ends at key tk: keys past tk read as zeros, and the
  // per-lane offsets (landing slot -> swizzled source chunk) are the same
  // for every tile.  Instruction i of a wave fills 1 KiB of the tile (64
  // lanes x 16 bytes).
  const uint16_t* kbase = A.k + (long long)kvh * A.cap * D;
  const uint16_t* vbase = A.v + (long long)kvh * A.cap * D;
  // (vectors, not arrays: a lambda capturing a local array of template-
  // dependent size loses the kernel's host-side launch stub)
  static_assert(CPW <= 4, "copy offsets hold four instructions");
  i32x4_t koffs = {}, voffs = {};
#pragma unroll
  for (int i = 0; i < CPW; ++i) {
    const int idx = (wave * CPW + i) * 64 + lane;     // landing chunk
    const int r = idx / KCH;
    koffs[i] = (r * D + (((idx % KCH) ^ (r % KCH)) << 3)) * 2;
    voffs[i] = (r * D + (((idx % KCH) ^ (4 * vswz<D>(r))) << 3)) * 2;
  }
  int32_t tr = 0;
  auto copy_k = [&](int j0, uint16_t* dst_tile) {
    const int left = max(A.tk - j0, 0);
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(kbase + (long long)j0 * D, left * D * 2);
    char* dst = reinterpret_cast<char*>(dst_tile) + wave * CPW * 1024;
    if (kCopyWaves == NWV || wave < kCopyWaves) {
#pragma unroll
      for (int i = 0; i < CPW; ++i) {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rs, (__attribute__((address_space(3))) void*)(dst + i * 1024), 16, koffs[i],
            0, 0, 0);
      }
    }
    if constexpr (MODE == 2) {
      const __amdgpu_buffer_rsrc_t ts_rs = make_rsrc(A.t_index + j0, left * 4);
      tr = (int)__builtin_amdgcn_raw_buffer_load_b32(ts_rs, (tid & 63) * 4, 0, 0);
    }
  };
  auto copy_v = [&](int j0, uint16_t* dst_tile) {
    const int left = max(A.tk - j0, 0);
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(vbase + (long long)j0 * D, left * D * 2);
    char* dst = reinterpret_cast<char*>(dst_tile) + wave * CPW * 1024;
    if (kCopyWaves == NWV || wave < kCopyWaves) {
#pragma unroll
      for (int i = 0; i < CPW; ++i) {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            rs, (__attribute__((address_space(3))) void*)(dst + i * 1024), 16, voffs[i],
            0, 0, 0);
      }
    }
  };
  int t_wg = INT_MIN;        // block-causal: the queries' one t, or INT_MIN
  auto store_t = [&](int tbuf) {
    if constexpr (MODE == 2) {
      if (tid < BK) {
        ts[tbuf][tid] = tr;
        // wave 0 holds the tile's 64 t entries, one per lane
        const bool same = __all(tr == t_wg && t_wg != INT_MIN);
        if (tid == 0) { tsame[tbuf] = same; }
      }
    }
  };

  // per-lane fragment offsets (elements)
  const int koff = lq * D;                             // + swizzled chunk
  const int vrow = 4 * half + ((lane & 15) >> 2);      // transpose-read key
  const int vcol = 16 * ((lane >> 4) & 1) + 4 * (lane & 3);

  f32x16_t o[NCB];
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) { o[cb] = f32x16_t{}; }
  float m = -INFINITY;      // running max, raw score units
  float l = 0.0f;           // this half's share of the running sum
  f32x16_t sc[2];           // scores of the current tile
  float mb = -INFINITY;     // their max over the row (both halves)

  const int q_first = A.q_offset + qt * QT;       // workgroup's first query
  // One past the last key any of the workgroup's queries sees; the tiles
  // after it are fully masked and would add exactly 0.
  int kend = A.tk;
  if constexpr (MODE != 0) {
    const int q_last = A.q_offset + min(A.tq, qt * QT + QT) - 1;
    kend = min(A.tk, q_last + 1);
  }
  if constexpr (MODE == 2) {
    // Keys past q_last are visible only through an equal t.  Bound them by
    // the t range of the workgroup's queries: the last key whose t lies in
    // [tmin, tmax] (a superset of the visible keys; the mask is exact).
    __shared__ int kred[3][NWV];
    int tmin = INT_MAX, tmax = INT_MIN;
    if (tid < QT && qt * QT + tid < A.tq) {
      const int tv = A.t_index[q_first + tid];
      tmin = tv;
      tmax = tv;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
      tmin = min(tmin, __shfl_xor(tmin, o));
      tmax = max(tmax, __shfl_xor(tmax, o));
    }
    if (lane == 0) { kred[0][wave] = tmin; kred[1][wave] = tmax; }
    __syncthreads();
    tmin = kred[0][0];
    tmax = kred[1][0];
#pragma unroll
    for (int w = 1; w < NWV; ++w) {
      tmin = min(tmin, kred[0][w]);
      tmax = max(tmax, kred[1][w]);
    }
    if (tmin == tmax) { t_wg = tmin; }
    int jm = kend - 1;
#pragma unroll 8
    for (int j = kend + tid; j < A.tk; j += 64 * NWV) {
      const int tv = A.t_index[j];
      if (tv >= tmin && tv <= tmax) { jm = j; }
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) { jm = max(jm, __shfl_xor(jm, o)); }
    if (lane == 0) { kred[2][wave] = jm; }
    __syncthreads();
    jm = kred[2][0];
#pragma unroll
    for (int w = 1; w < NWV; ++w) { jm = max(jm, kred[2][w]); }
    kend = jm + 1;
  }
  const int ntiles = (kend + BK - 1) / BK;

  // -inf for the scores of tile j0 that the mode hides; a no-op for a tile
  // whose keys are all below tk and (causal masks) the first query
  auto mask = [&](f32x16_t (&s)[2], int j0, int tbuf) {
    bool full = j0 + BK <= A.tk && (MODE == 0 || j0 + BK - 1 <= q_first);
    // block-causal: every key of the tile shares the queries' one t
    if constexpr (MODE == 2) { full = full || (j0 + BK <= A.tk && tsame[tbuf] != 0); }
    if (full) { return; }
    // branch-free: every lane reads its t entry (kl < 64 is in bounds) and
    // the conditions combine bitwise, so the mask is a select
#pragma unroll
    for (int r = 0; r < 32; ++r) {
      const int kl = (r >> 4) * 32 + 8 * ((r & 15) >> 2) + 4 * half + (r & 3);
      const int key = j0 + kl;
      bool ok = key < A.tk;
      if constexpr (MODE == 1) { ok = ok & (key <= qpos); }
      if constexpr (MODE == 2) {
        const int t_key = ts[tbuf][kl];
        ok = ok & ((key <= qpos) | (t_key == tq_idx));
      }
      s[r >> 4][r & 15] = ok ? s[r >> 4][r & 15] : -INFINITY;
    }
  };
  // one probability pair: exp2((s - m) * scale), packed to bf16 and
  // summed as packed (one dot with (1, 1)): the sum then counts exactly
  // the rounded weights the P V product uses
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  uint32_t pk[16];
  float ps;
  float mc;
  auto expo = [&](const f32x16_t& s, int r, int slot) {
    const float p0 = __builtin_amdgcn_exp2f(fmaf(s[r], scale, -mc));
    const float p1 = __builtin_amdgcn_exp2f(fmaf(s[r + 1], scale, -mc));
    pk[slot] = pack_bf16x2(p0, p1);
    ps = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, pk[slot]),
                                         __builtin_bit_cast(bf16x2_t, 0x3f803f80u), ps,
                                         false);
  };
  // O^T block cb += V^T (16-key step k4) P^T
  auto pv = [&](const uint16_t* vread, int k4, int cb) {
    const i32x4_t pf = {(int)pk[k4 * 4 + 0], (int)pk[k4 * 4 + 1],
                        (int)pk[k4 * 4 + 2], (int)pk[k4 * 4 + 3]};
    const int r0 = k4 * 16 + vrow;
    const int c = (((cb ^ vswz<D>(r0)) << 5) | vcol);     // r0, r0+8 share it
    const i16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) i16x4_t*)(vread + r0 * D + c));
    const i16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (__attribute__((address_space(3))) i16x4_t*)(vread + (r0 + 8) * D + c));
    const i32x4_t vf = {__builtin_bit_cast(int, (i16x2_t){lo[0], lo[1]}),
                        __builtin_bit_cast(int, (i16x2_t){lo[2], lo[3]}),
                        __builtin_bit_cast(int, (i16x2_t){hi[0], hi[1]}),
                        __builtin_bit_cast(int, (i16x2_t){hi[2], hi[3]})};
    o[cb] = MmaBf16::run(vf, pf, o[cb]);
  };

  // One iteration over tile t, in three sections that each pair MFMA work
  // with VALU work of about the same length:
  //   A  scores of tile t+1 (16 MFMA)   | exponentials of keys 0..31
  //   B  P V of keys 0..31 (8 MFMA)     | exponentials of keys 32..63
  //   C  P V of keys 32..63 (8 MFMA)    | max of tile t+1's scores
  // kread / kfill are tile t+1's and tile t+2's K buffers, vread / vfill
  // tile t's and tile t+1's V buffers.
  constexpr int EPA = 16 / NDS;               // probabilities per K-step (A)
  constexpr int EPB = 16 / (2 * NCB);         // probabilities per MFMA (B)
  constexpr int MPC = 32 / (2 * NCB);         // maxed scores per MFMA (C)
  auto iteration = [&](int t, const uint16_t* kread, uint16_t* kfill,
                       const uint16_t* vread, uint16_t* vfill) {
    const int j0 = t * BK;
    if (mb > m + lazy) {
      const float alpha = exp2f((m - mb) * scale);     // 0 while m is -inf
      l *= alpha;
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) { o[cb][r] *= alpha; }
      }
      m = mb;
    }
    mc = m == -INFINITY ? 0.0f : m * scale;
    ps = 0.0f;
    copy_k((t + 2) * BK, kfill);        // past the last tile: zeros, unread
    copy_v((t + 1) * BK, vfill);

    // ---- A --------------------------------------------------------------
    // (past the last tile the scores come from stale K and are dropped)
    f32x16_t sn[2] = {f32x16_t{}, f32x16_t{}};
#pragma unroll
    for (int ds = 0; ds < NDS; ++ds) {
      const int off = koff + (((ds * 2 + half) ^ (lq % KCH)) << 3);
      const i32x4_t k0 = *reinterpret_cast<const i32x4_t*>(kread + off);
      const i32x4_t k1 = *reinterpret_cast<const i32x4_t*>(kread + 32 * D + off);
      sn[0] = MmaBf16::run(k0, qf[ds], sn[0]);
#pragma unroll
      for (int e = 0; e < EPA; e += 2) { expo(sc[0], ds * EPA + e, (ds * EPA + e) >> 1); }
      sn[1] = MmaBf16::run(k1, qf[ds], sn[1]);
    }
    // ---- B --------------------------------------------------------------
#pragma unroll
    for (int k4 = 0; k4 < 2; ++k4) {
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb) {
        pv(vread, k4, cb);
        const int r = (k4 * NCB + cb) * EPB;
#pragma unroll
        for (int e = 0; e < EPB; e += 2) { expo(sc[1], r + e, 8 + ((r + e) >> 1)); }
      }
    }
    // schedule A and B: each step's LDS reads one step ahead of its MFMA
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);                // reads 0, 1
#pragma unroll
    for (int ds = 0; ds < NDS; ++ds) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);              // MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, 6 * EPA / 4, 0);    // VALU
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);              // reads +2
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);              // MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, 6 * EPA / 4, 0);    // VALU
    }
#pragma unroll
    for (int i = 0; i < 2 * NCB; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);              // MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, 6 * EPB / 4, 0);    // VALU
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);              // reads +2
      __builtin_amdgcn_sched_group_barrier(0x002, 6 * EPB / 4, 0);    // VALU
    }
    // ---- C --------------------------------------------------------------
    mask(sn, j0 + BK, (t + 1) % 3);
    float mx = -INFINITY;
#pragma unroll
    for (int k4 = 2; k4 < 4; ++k4) {
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb) {
        pv(vread, k4, cb);
        const int r = ((k4 - 2) * NCB + cb) * MPC;
#pragma unroll
        for (int e = 0; e < MPC; ++e) { mx = fmaxf(mx, sn[(r + e) >> 4][(r + e) & 15]); }
      }
    }
    __builtin_amdgcn_sched_group_barrier(0x100, 4, 0);                // reads 0, 1
#pragma unroll
    for (int i = 0; i < 2 * NCB; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);              // MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, MPC / 2, 0);        // VALU
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);              // reads +2
    }
    mb = max_halves(mx);
    l += ps;
    store_t((t + 2) % 3);
    __syncthreads();
    sc[0] = sn[0];
    sc[1] = sn[1];
  };

  if (ntiles > 0) {
    // K and t of tiles 0 and 1, V of tile 0; the scores of tile 0, read
    // by every wave before the first iteration refills ks0
    copy_k(0, ks0);
    store_t(0);
    copy_k(BK, ks1);
    store_t(1);
    copy_v(0, vs0);
    __syncthreads();
    sc[0] = f32x16_t{};
    sc[1] = f32x16_t{};
#pragma unroll
    for (int ds = 0; ds < NDS; ++ds) {
      const int off = koff + (((ds * 2 + half) ^ (lq % KCH)) << 3);
      sc[0] = MmaBf16::run(*reinterpret_cast<const i32x4_t*>(ks0 + off), qf[ds], sc[0]);
      sc[1] = MmaBf16::run(*reinterpret_cast<const i32x4_t*>(ks0 + 32 * D + off),
                           qf[ds], sc[1]);
    }
    mask(sc, 0, 0);
    float mx = sc[0][0];
#pragma unroll
    for (int r = 1; r < 32; ++r) { mx = fmaxf(mx, sc[r >> 4][r & 15]); }
    mb = max_halves(mx);
    __syncthreads();
  }
  for (int t = 0; t < ntiles; t += 2) {
    iteration(t, ks1, ks0, vs0, vs1);
    if (t + 1 < ntiles) { iteration(t + 1, ks0, ks1, vs1, vs0); }
  }

  l = sum_halves(l);
  if (!qvalid) { return; }
  const float inv = l > 0.0f ? 1.0f / l : 0.0f;
  uint16_t* op = A.out + (long long)h * A.o_head + (long long)qrow * A.o_tok;
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int c = cb * 32 + 8 * g + 4 * half;
      u32x2_t w = {bf16_bits(o[cb][4 * g + 0] * inv) |
                       (bf16_bits(o[cb][4 * g + 1] * inv) << 16),
                   bf16_bits(o[cb][4 * g + 2] * inv) |
                       (bf16_bits(o[cb][4 * g + 3] * inv) << 16)};
      *reinterpret_cast<u32x2_t*>(op + c) = w;
    }
  }
}

// Row re-layout of [T][H][D] data between two strided views: element
// (t, h, c) moves from src[t * src_t + h * src_h + c] to dst[t * dst_t +
// h * dst_h + c]; 16 bytes per thread.
__global__ __launch_bounds__(256) void
transpose_rows_kernel(const uint16_t* __restrict__ src, uint16_t* __restrict__ dst,
                      int T, int H, int D, long long src_t, long long src_h,
                      long long dst_t, long long dst_h)
{
  const int per_row = D / 8;
  const long long n = (long long)T * H * per_row;
  for (long long i = (long long)blockIdx.x * 256 + threadIdx.x; i < n;
       i += (long long)gridDim.x * 256) {
    const int c = (int)(i % per_row) * 8;
    const long long th = i / per_row;
    const int hh = (int)(th % H);
    const long long t = th / H;
    *reinterpret_cast<uint4*>(dst + t * dst_t + hh * dst_h + c) =
        *reinterpret_cast<const uint4*>(src + t * src_t + hh * src_h + c);
  }
}

// ---- skinny GEMM: problems of at most 128 rows --------------------------
// Below a few hundred rows per weight set a projection streams its weights
// (N x K bf16) and little else; the tiled GEMM's 256-row tiles then run
// mostly empty, and its split-K tail sends 256 x 256 fp32 partial tiles
// through memory.  Two kernels cover this regime, both built on the same
// fragment layout:
//
// K order inside a 64-element K-block: lane group g (lanes 16g .. 16g+15)
// holds elements [16g, 16g + 16) of its row for both operands, the first
// eight as MFMA k-step 0 and the rest as k-step 1.  The products summed
// are exactly the block's, in another order, and each lane's bytes of a
// row are one 32-byte run (a row's 128 bytes in four lanes).
// v_mfma_f32_16x16x32_bf16 takes the weight fragment as A (16 output
// columns) and the activation fragment as B (16 rows): lane (g, r) ends
// with columns 4g .. 4g + 3 of its 16 for row r of each 16-row group.
//
// Loads of one wave return in issue order, so a wave can only run as far
// ahead of its data as its earliest outstanding load allows.  The register
// kernel keeps its operands kSkDepth K-blocks ahead, the LDS kernels D.
// Deeper is not faster: with N = 6144, K = 4096 and 12 rotated weight
// copies a call at 1 / 8 / 16 rows took 13.5 / 15.4 / 18.1 us at depth 2
// against 15.8 / 17.4 / 19.8 at 8 (the extra requests in flight only
// queue), and the LDS kernels 17.7 / 20.6 us at 32 / 64 rows with D = 4
// against 18.2 / 21.4 with D = 8.
//
// The accumulators are tied to their MFMAs (inline asm "+v"): the
// builtin's untied 16x16 result makes the compiler rotate them through
// copies.  The asm is volatile and writes no memory, so the loads and
// reads around it keep their place; the hazards the compiler's tracking
// would cover are covered with wait states (the zeroing before the first
// MFMA, the last results before the epilogue reads them).
constexpr int kSkDepth = 2;    // K-blocks in flight per wave

// One wave's weight fragments of a K-block: lane (g, r) holds row r,
// elements [16g, 16g + 16).  QB = 0: bf16 rows, two 16-byte loads.  QB = 4
// or 8: an affine-quantized pack (codes [n][K * QB / 32] u32, scale and
// bias bf16 [n][K / group]): the lane's 16 codes (one 16- or 8-byte load)
// and its group's scale and bias, dequantised when the MFMA takes them as
// w = bf16_rne(scale * code + bias) (a multiply, then an add) -- the
// bf16 weight the dequant-once expansion writes, bit for bit.
template <int QB>
struct SkW {
  i32x4_t c;
  uint32_t s, b;
};
template <>
struct SkW<0> {
  i32x4_t v[2];
};

// Per-lane load parameters of a wave's 16 weight rows.
struct SkWSrc {
  __amdgpu_buffer_rsrc_t w;     // bf16 rows or codes, rows [n0, n0 + 16)
  __amdgpu_buffer_rsrc_t qs;    // scales of those rows (QB > 0)
  __amdgpu_buffer_rsrc_t qb;    // biases of those rows (QB > 0)
  int wv;                       // the lane's byte offset in w (K-block 0)
  int sv;                       // the lane's byte offset in qs / qb
};

template <int QB>
__device__ __forceinline__ SkWSrc
sk_wsrc(const SkinnyBatch& B, const SkinnyProblem& P, int n0, int lane)
{
  const int g = lane >> 4, r = lane & 15;
  const int rows = max(0, min(16, P.n - n0));       // rows past n read zero
  const int nr = min(n0, P.n);
  SkWSrc d;
  if constexpr (QB == 0) {
    d.w = make_rsrc(static_cast<const char*>(P.w) + (size_t)nr * B.kbytes,
                    rows * B.kbytes);
    d.wv = r * B.kbytes + g * 32;
    d.qs = d.qb = d.w;
    d.sv = 0;
  } else {
    const int K = B.kbytes / 2;
    const int cpitch = K * QB / 8;                   // code bytes per row
    const int spitch = K / B.qgroup * 2;             // scale bytes per row
    d.w = make_rsrc(static_cast<const char*>(P.w) + (size_t)nr * cpitch, rows * cpitch);
    d.qs = make_rsrc(reinterpret_cast<const char*>(P.qs) + (size_t)nr * spitch, rows * spitch);
    d.qb = make_rsrc(reinterpret_cast<const char*>(P.qb) + (size_t)nr * spitch, rows * spitch);
    d.wv = r * cpitch + g * 16 * QB / 8;
    d.sv = r * spitch + (B.qgroup == 32 ? (g >> 1) * 2 : 0);
  }
  return d;
}

// Loads K-block kb (oob: an offset past every row, zeros).
template <int QB>
__device__ __forceinline__ void
sk_load_w(SkW<QB>& d, const SkWSrc& src, int kb, int oob, int qgroup)
{
  if constexpr (QB == 0) {
    const int ko = __builtin_amdgcn_readfirstlane(kb * 128);
    d.v[0] = __builtin_amdgcn_raw_buffer_load_b128(src.w, src.wv + oob, ko, 0);
    d.v[1] = __builtin_amdgcn_raw_buffer_load_b128(src.w, src.wv + 16 + oob, ko, 0);
  } else {
    const int ko = __builtin_amdgcn_readfirstlane(kb * 64 * QB / 8);
    if constexpr (QB == 8) {
      d.c = __builtin_amdgcn_raw_buffer_load_b128(src.w, src.wv + oob, ko, 0);
    } else {
      const auto c2 = __builtin_amdgcn_raw_buffer_load_b64(src.w, src.wv + oob, ko, 0);
      d.c = i32x4_t{(int)c2[0], (int)c2[1], 0, 0};
    }
    const int so = __builtin_amdgcn_readfirstlane(kb * (64 / qgroup) * 2);
    d.s = __builtin_amdgcn_raw_buffer_load_b16(src.qs, src.sv + oob, so, 0);
    d.b = __builtin_amdgcn_raw_buffer_load_b16(src.qb, src.sv + oob, so, 0);
  }
}

// The bf16 A fragment of k-step ks (elements [16g + 8ks, 16g + 8ks + 8)).
template <int QB>
__device__ __forceinline__ i32x4_t
sk_frag(const SkW<QB>& d, int ks)
{
  if constexpr (QB == 0) {
    return d.v[ks];
  } else {
    const float sc = bf16_to_f32(d.s & 0xffffu);
    const float bi = bf16_to_f32(d.b & 0xffffu);
    constexpr uint32_t kMask = (1u << QB) - 1u;
    uint32_t codes[2];
    if constexpr (QB == 8) {
      codes[0] = (uint32_t)d.c[2 * ks];
      codes[1] = (uint32_t)d.c[2 * ks + 1];
    }
    i32x4_t f;
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
      uint32_t c0, c1;
      if constexpr (QB == 8) {
        c0 = (codes[e >> 2] >> ((e & 3) * 8)) & kMask;
        c1 = (codes[e >> 2] >> (((e & 3) + 1) * 8)) & kMask;
      } else {
        c0 = ((uint32_t)d.c[ks] >> (e * 4)) & kMask;
        c1 = ((uint32_t)d.c[ks] >> ((e + 1) * 4)) & kMask;
      }
      // a multiply, then an add (not fused), as dequant_affine_kernel
      float p0 = sc * (float)c0;
      float p1 = sc * (float)c1;
      asm("" : "+v"(p0), "+v"(p1));
      f[e >> 1] = (int)pack_bf16x2(p0 + bi, p1 + bi);
    }
    return f;
  }
}

// A 16x16x32 bf16 MFMA with its accumulator tied ("+v").  With QB > 0 the
// A fragment comes from VALU arithmetic just before: two wait states
// separate that write from the MFMA's read.
template <int QB>
__device__ __forceinline__ void
sk_mfma(f32x4_t& acc, i32x4_t a, i32x4_t b)
{
  if constexpr (QB == 0) {
    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+v"(acc) : "v"(a), "v"(b));
  } else {
    asm volatile("s_nop 1\n\tv_mfma_f32_16x16x32_bf16 %0, %1, %2, %0"
                 : "+v"(acc) : "v"(a), "v"(b));
  }
}

// Bias, rounding and store of 4 output columns n..n+3 of row m.
__device__ __forceinline__ void
skinny_store(const SkinnyProblem& P, int m, int n, f32x4_t v, uint2 bb)
{
  const float v0 = v[0] + bf16_to_f32(bb.x & 0xffffu);
  const float v1 = v[1] + bf16_to_f32(bb.x >> 16);
  const float v2 = v[2] + bf16_to_f32(bb.y & 0xffffu);
  const float v3 = v[3] + bf16_to_f32(bb.y >> 16);
  *reinterpret_cast<uint2*>(static_cast<uint16_t*>(P.y) + (size_t)m * P.ldy + n) =
      make_uint2(pack_bf16x2(v0, v1), pack_bf16x2(v2, v3));
}

// Problem of a column block (uniform over the workgroup).
__device__ __forceinline__ int
skinny_problem(const SkinnyBatch& B, int cbg)
{
  int pi = 0;
#pragma unroll
  for (int q = 1; q < kMaxProb; ++q) {
    if (q < B.nprob && cbg >= B.p[q].cb_begin) { pi = q; }
  }
  return pi;
}

// Rows <= 16: a workgroup computes 16 output columns
// over a K share; its four waves take every fourth K-block each and load
// both operands straight into registers (the activation rows are few and
// L2-resident), with no barrier until the four partial sums meet in LDS,
// where wave 0 adds them in wave order.
template <int MT, int QB>
__global__ __launch_bounds__(256) void
skinny_reg_kernel(const SkinnyBatch B)
{
  __shared__ f32x4_t red[4][MT][64];
  const int S = B.split;
  const int cbg = blockIdx.x / S;
  const int share = blockIdx.x - cbg * S;
  const SkinnyProblem& P = B.p[skinny_problem(B, cbg)];
  const int kbytes = B.kbytes;
  const int nkb = kbytes / 128;
  const int kb0 = share * nkb / S;
  const int nk = (share + 1) * nkb / S - kb0;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane >> 4, r = lane & 15;
  const int n0 = (cbg - P.cb_begin) * 16;
  const int nw = (nk - wave + 3) / 4;              // this wave's K-blocks

  // weight rows [n0, n0 + 16) and activation rows [0, rows); rows past
  // either read as zero
  const SkWSrc wsrc = sk_wsrc<QB>(B, P, n0, lane);
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(P.a, P.rows * kbytes);
  const int lv = r * kbytes + g * 32;               // row r, bytes 32g..

  SkW<QB> wreg[kSkDepth];
  i32x4_t xreg[kSkDepth][MT][2];
  auto issue = [&](int slot, int j) {
    const int oob = j < nw ? 0 : kOobOffset;        // past the share: zeros
    const int kb = kb0 + wave + 4 * min(j, max(nw - 1, 0));
    const int ko = __builtin_amdgcn_readfirstlane(kb * 128);
    sk_load_w<QB>(wreg[slot], wsrc, kb, oob, B.qgroup);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int v = lv + mt * 16 * kbytes + oob;
      xreg[slot][mt][0] = __builtin_amdgcn_raw_buffer_load_b128(xr, v, ko, 0);
      xreg[slot][mt][1] = __builtin_amdgcn_raw_buffer_load_b128(xr, v + 16, ko, 0);
    }
  };

  f32x4_t acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    acc[mt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    asm volatile("" : "+v"(acc[mt]));
  }
  asm volatile("s_nop 4");
  // the loads in K order (compiler fences between the blocks)
#pragma unroll
  for (int d = 0; d < kSkDepth; ++d) {
    asm volatile("" ::: "memory");
    issue(d, d);
  }
  const int nw_pad = (nw + kSkDepth - 1) / kSkDepth * kSkDepth;
  for (int j0 = 0; j0 < nw_pad; j0 += kSkDepth) {
#pragma unroll
    for (int d = 0; d < kSkDepth; ++d) {
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const i32x4_t wf = sk_frag<QB>(wreg[d], ks);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) { sk_mfma<QB>(acc[mt], wf, xreg[d][mt][ks]); }
      }
      asm volatile("" ::: "memory");
      issue(d, j0 + d + kSkDepth);
    }
  }
  asm volatile("s_waitcnt vmcnt(0)\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7"
               ::: "memory");
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    asm volatile("" : "+v"(acc[mt]));
    red[wave][mt][lane] = acc[mt];
  }
  __syncthreads();
  if (wave != 0) { return; }
  const int n = n0 + 4 * g;
  if (n >= P.n) { return; }
  uint2 bb = make_uint2(0u, 0u);
  if (S == 1 && P.bias != nullptr) { bb = *reinterpret_cast<const uint2*>(P.bias + n); }
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = mt * 16 + r;
    if (m >= P.rows) { continue; }
    const f32x4_t v = ((red[0][mt][lane] + red[1][mt][lane]) + red[2][mt][lane]) +
                      red[3][mt][lane];
    if (S == 1) {
      skinny_store(P, m, n, v, bb);
    } else {
      float* ws = B.ws + P.ws_off + (size_t)share * P.rows * P.n;
      *reinterpret_cast<f32x4_t*>(ws + (size_t)m * P.n + n) = v;
    }
  }
}

// Rows <= 16 with bf16 weights: skinny_reg_kernel's work split, but each
// wave's 16 weight rows of a K-block arrive by two whole-line direct loads
// global -> LDS (instruction i: rows 8i .. 8i+7, 8 lanes x 16 bytes per
// 128-byte row) into the wave's own slot of a kSkDmaDepth-stage ring, and
// the fragments are read back in the MFMA's layout (lane (g, r): row r,
// 16-byte chunks 2g and 2g+1, the same K order as the register kernel, so
// the two agree bit for bit).  The register kernel's lane layout asks for
// every 128-byte line in two half-used requests.  Chunk c of row r sits at
// position c ^ ((r >> 1) & 7) of its row, so the 16 lanes of a fragment
// read (16 rows, one chunk) cover the 64 banks once.  The slots are
// private to their wave: no barrier until the partial sums meet.
// Measured (N = 6144, K = 4096, 12 rotated weight copies, same box): 12.6
// / 13.2 / 15.4 us per call at 1 / 8 / 16 rows against 13.6-13.9 / 15.6 /
// 18.2 for the register kernel.
constexpr int kSkDmaDepth = 2;    // K-blocks in flight per wave (4 measured slower)

template <int MT>
__global__ __launch_bounds__(256) void
skinny_dma_kernel(const SkinnyBatch B)
{
  static_assert(kSkDmaDepth == 2 || kSkDmaDepth == 4, "ring of 2 or 4 stages");
  __shared__ f32x4_t red[4][MT][64];
  // one __shared__ object per stage, so the compiler tells a stage's reads
  // from the copies filling another
  __shared__ __attribute__((aligned(1024))) char wr0[4 * 2048];
  __shared__ __attribute__((aligned(1024))) char wr1[4 * 2048];
  __shared__ __attribute__((aligned(1024))) char wr2[kSkDmaDepth == 4 ? 4 * 2048 : 16];
  __shared__ __attribute__((aligned(1024))) char wr3[kSkDmaDepth == 4 ? 4 * 2048 : 16];
  const int S = B.split;
  const int cbg = blockIdx.x / S;
  const int share = blockIdx.x - cbg * S;
  const SkinnyProblem& P = B.p[skinny_problem(B, cbg)];
  const int kbytes = B.kbytes;
  const int nkb = kbytes / 128;
  const int kb0 = share * nkb / S;
  const int nk = (share + 1) * nkb / S - kb0;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane >> 4, r = lane & 15;
  const int n0 = (cbg - P.cb_begin) * 16;
  const int nw = (nk - wave + 3) / 4;              // this wave's K-blocks

  // weight rows [n0, n0 + 16) and activation rows [0, rows); rows past
  // either read as zero
  const int wrows = max(0, min(16, P.n - n0));
  const __amdgpu_buffer_rsrc_t wrs =
      make_rsrc(static_cast<const char*>(P.w) + (size_t)min(n0, P.n) * kbytes,
                wrows * kbytes);
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(P.a, P.rows * kbytes);
  const int lv = r * kbytes + g * 32;               // row r, bytes 32g..
  int dv[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int row = 8 * i + (lane >> 3);
    dv[i] = row * kbytes + (((lane & 7) ^ ((row >> 1) & 7)) << 4);
  }
  const int slot = wave * 2048;
  int rdo[2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    rdo[ks] = slot + r * 128 + (((2 * g + ks) ^ ((r >> 1) & 7)) << 4);
  }

  i32x4_t xreg[kSkDmaDepth][MT][2];
  auto issue = [&](char* stage, int d, int j) {
    const int oob = j < nw ? 0 : kOobOffset;        // past the share: zeros
    const int kb = kb0 + wave + 4 * min(j, max(nw - 1, 0));
    const int ko = __builtin_amdgcn_readfirstlane(kb * 128);
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          wrs, (__attribute__((address_space(3))) void*)(stage + slot + i * 1024), 16,
          dv[i] + oob, ko, 0, 0);
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int v = lv + mt * 16 * kbytes + oob;
      xreg[d][mt][0] = __builtin_amdgcn_raw_buffer_load_b128(xr, v, ko, 0);
      xreg[d][mt][1] = __builtin_amdgcn_raw_buffer_load_b128(xr, v + 16, ko, 0);
    }
  };
  char* const ring[4] = {wr0, wr1, wr2, wr3};

  f32x4_t acc[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    acc[mt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    asm volatile("" : "+v"(acc[mt]));
  }
  asm volatile("s_nop 4");
  // the loads in K order (compiler fences between the blocks)
#pragma unroll
  for (int d = 0; d < kSkDmaDepth; ++d) {
    asm volatile("" ::: "memory");
    issue(ring[d], d, d);
  }
  // a block's copies have landed once at most the later blocks' loads are
  // in flight (loads complete in issue order; the compiler may order a
  // block's copies and activation loads either way, so the whole block is
  // waited for)
  constexpr int kAfter = (kSkDmaDepth - 1) * (2 + 2 * MT);
  static_assert(kAfter < 64, "vmcnt holds at most 63");
  const int nw_pad = (nw + kSkDmaDepth - 1) / kSkDmaDepth * kSkDmaDepth;
  for (int j0 = 0; j0 < nw_pad; j0 += kSkDmaDepth) {
#pragma unroll
    for (int d = 0; d < kSkDmaDepth; ++d) {
      asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kAfter) : "memory");
      i32x4_t wf[2];
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        wf[ks] = *reinterpret_cast<const i32x4_t*>(ring[d] + rdo[ks]);
      }
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) { sk_mfma<0>(acc[mt], wf[ks], xreg[d][mt][ks]); }
      }
      // the MFMAs consumed this stage's reads; its slot takes block j + depth
      asm volatile("" ::: "memory");
      issue(ring[d], d, j0 + d + kSkDmaDepth);
    }
  }
  asm volatile("s_waitcnt vmcnt(0)\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7"
               ::: "memory");
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    asm volatile("" : "+v"(acc[mt]));
    red[wave][mt][lane] = acc[mt];
  }
  __syncthreads();
  if (wave != 0) { return; }
  const int n = n0 + 4 * g;
  if (n >= P.n) { return; }
  uint2 bb = make_uint2(0u, 0u);
  if (S == 1 && P.bias != nullptr) { bb = *reinterpret_cast<const uint2*>(P.bias + n); }
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const int m = mt * 16 + r;
    if (m >= P.rows) { continue; }
    const f32x4_t v = ((red[0][mt][lane] + red[1][mt][lane]) + red[2][mt][lane]) +
                      red[3][mt][lane];
    if (S == 1) {
      skinny_store(P, m, n, v, bb);
    } else {
      float* ws = B.ws + P.ws_off + (size_t)share * P.rows * P.n;
      *reinterpret_cast<f32x4_t*>(ws + (size_t)m * P.n + n) = v;
    }
  }
}

// Rows 17..128: a workgroup computes 64 CW output columns over a K share.
// Wave w streams weight rows [16 CW w, 16 CW (w + 1)) of the block -- into
// its slot of a weight ring by whole-line direct loads for bf16 weights,
// into registers for packs -- while the activation rows' K-block, which
// all four waves use, goes to LDS by DMA through a ring of D stages (one
// __shared__ object each, so the compiler can tell a stage's DMA from
// another stage's reads).  MT row groups of 16; with CW = 2 every
// activation fragment read from LDS serves two weight fragments.
template <int MT, int D, int QB, int CW>
__device__ __forceinline__ void
skinny_lds_tile(const SkinnyBatch& B, char* const (&xs)[D], char* const (&wsr)[D])
{
  constexpr int kXInst = MT / 2;                    // DMA loads per wave
  // bf16 weights arrive like skinny_dma_kernel's: whole-line direct loads
  // into the wave's slot of a D-stage weight ring; packs load theirs into
  // registers
  constexpr bool kWDma = QB == 0;
  const int S = B.split;
  const int cbg = blockIdx.x / S;
  const int share = blockIdx.x - cbg * S;
  const SkinnyProblem& P = B.p[skinny_problem(B, cbg)];
  const int kbytes = B.kbytes;
  const int nkb = kbytes / 128;
  const int kb0 = share * nkb / S;
  const int nk = (share + 1) * nkb / S - kb0;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = lane >> 4, r = lane & 15;
  const int n0 = (cbg - P.cb_begin) * 64 * CW + wave * 16 * CW;

  // weight rows [n0 + 16c, n0 + 16c + 16) clipped to n: rows past it read
  // as zero
  SkWSrc wsrc[CW];
#pragma unroll
  for (int c = 0; c < CW; ++c) { wsrc[c] = sk_wsrc<QB>(B, P, n0 + 16 * c, lane); }
  // the direct loads' view: rows [n0, n0 + 16 CW) clipped to n
  const __amdgpu_buffer_rsrc_t wdr = make_rsrc(
      static_cast<const char*>(P.w) + (size_t)min(n0, P.n) * kbytes,
      max(0, min(16 * CW, P.n - n0)) * kbytes);
  // activation rows [0, rows): rows past them read as zero
  const __amdgpu_buffer_rsrc_t xr = make_rsrc(P.a, P.rows * kbytes);
  // DMA: instruction j of wave w fills 16-byte stage slots
  // p = 32 MT w + 64 j + lane, slot p of row p / 8 holding chunk
  // (p % 8) ^ (row % 8) of the row's K-block
  int xv[kXInst];
#pragma unroll
  for (int j = 0; j < kXInst; ++j) {
    const int p = 32 * MT * wave + 64 * j + lane;
    const int m = p >> 3;
    xv[j] = m * kbytes + ((((p & 7) ^ (m & 7))) << 4);
  }
  // fragment reads: row r of a 16-row group, chunk 2g + ks
  int xo[2];
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    xo[ks] = r * 128 + (((2 * g + ks) ^ (r & 7)) << 4);
  }

  auto issue_x = [&](char* st, int i) {
    const int oob = i < nk ? 0 : kOobOffset;       // past the share: zeros
    const int ko = __builtin_amdgcn_readfirstlane((kb0 + min(i, nk - 1)) * 128);
#pragma unroll
    for (int j = 0; j < kXInst; ++j) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          xr, (__attribute__((address_space(3))) void*)(st + 32 * MT * 16 * wave + 1024 * j),
          16, xv[j] + oob, ko, 0, 0);
    }
  };
  SkW<QB> wreg[kWDma ? 1 : D][CW];
  // direct load j of a K-block: the wave's rows 8j .. 8j + 7, lane l
  // landing at slot l % 8 of row 8j + l / 8 and carrying chunk
  // (l % 8) ^ ((row / 2) % 8) (conflict-free fragment reads)
  int dv[2 * CW], rdo[2];
#pragma unroll
  for (int j = 0; j < 2 * CW; ++j) {
    const int row = 8 * j + (lane >> 3);
    dv[j] = row * kbytes + (((lane & 7) ^ ((row >> 1) & 7)) << 4);
  }
#pragma unroll
  for (int ks = 0; ks < 2; ++ks) {
    rdo[ks] = wave * 2048 * CW + r * 128 + (((2 * g + ks) ^ ((r >> 1) & 7)) << 4);
  }
  auto issue_w = [&](int slot, int i) {
    const int oob = i < nk ? 0 : kOobOffset;
    if constexpr (kWDma) {
      const int ko = __builtin_amdgcn_readfirstlane((kb0 + min(i, nk - 1)) * 128);
#pragma unroll
      for (int j = 0; j < 2 * CW; ++j) {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(
            wdr, (__attribute__((address_space(3))) void*)(wsr[slot] + wave * 2048 * CW + j * 1024),
            16, dv[j] + oob, ko, 0, 0);
      }
    } else {
#pragma unroll
      for (int c = 0; c < CW; ++c) {
        sk_load_w<QB>(wreg[slot][c], wsrc[c], kb0 + min(i, nk - 1), oob, B.qgroup);
      }
    }
  };

  f32x4_t acc[CW][MT];
#pragma unroll
  for (int c = 0; c < CW; ++c) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      acc[c][mt] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
      asm volatile("" : "+v"(acc[c][mt]));
    }
  }
  asm volatile("s_nop 4");

  // The wait before each barrier counts loads in issue order, so the order
  // is pinned with compiler fences.  In each block: the x refill, then the
  // weight refill.  Prologue with weights in LDS: the blocks in K order,
  // weights before x (the last block's x stage comes with the loop), so
  // that block j's weight copies always go out before its x stage.  With
  // weights in registers, whose reads the compiler makes wait by itself:
  // the x stages, then the weight blocks (measured 1-2% faster for the
  // w8 pack at 32-64 rows than the interleaved order).
  if constexpr (kWDma) {
#pragma unroll
    for (int i = 0; i < D; ++i) {
      asm volatile("" ::: "memory");
      issue_w(i, i);
      asm volatile("" ::: "memory");
      if (i + 1 < D) { issue_x(xs[i], i); }
    }
  } else {
#pragma unroll
    for (int i = 0; i + 1 < D; ++i) { issue_x(xs[i], i); }
#pragma unroll
    for (int i = 0; i < D; ++i) {
      asm volatile("" ::: "memory");
      issue_w(i, i);
    }
  }
  // Before block i's barrier this wave's DMA of x stage i (and, in LDS,
  // block i's weights) has landed: at most the loads issued after it may
  // be in flight -- the weight loads of block i + 1 and D - 2 later
  // blocks' x and weight loads (in the register prologue more follow x
  // stage i, and the wait holds more back than it needs).
  constexpr int kWLoads = (QB == 0 ? 2 : 3) * CW;   // per K-block
  constexpr int kAfterX = kWLoads + (D - 2) * (kXInst + kWLoads);
  static_assert(kAfterX < 64, "vmcnt holds at most 63");
  const int nk_pad = (nk + D - 1) / D * D;
  for (int i0 = 0; i0 < nk_pad; i0 += D) {
#pragma unroll
    for (int d = 0; d < D; ++d) {
      const int i = i0 + d;
      // (a bare s_barrier: __syncthreads' fence would wait for every
      // weight load in flight)
      asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(kAfterX) : "memory");
      // every wave is past its reads of stage i - 1: refill it
      issue_x(xs[(d + D - 1) % D], i + D - 1);
      asm volatile("" ::: "memory");
      const char* st = xs[d];
      i32x4_t xf[MT][2];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
          xf[mt][ks] = *reinterpret_cast<const i32x4_t*>(st + mt * 2048 + xo[ks]);
        }
      }
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
        for (int c = 0; c < CW; ++c) {
          i32x4_t wf;
          if constexpr (kWDma) {
            // block i's weight copies were issued before its x stage, which
            // the barrier above has seen land
            wf = *reinterpret_cast<const i32x4_t*>(wsr[d] + c * 2048 + rdo[ks]);
          } else {
            wf = sk_frag<QB>(wreg[d][c], ks);
          }
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) { sk_mfma<QB>(acc[c][mt], wf, xf[mt][ks]); }
        }
      }
      // (the MFMAs consumed this block's weight reads before the refill)
      asm volatile("" ::: "memory");
      issue_w(d, i + D);
    }
  }
  // no DMA may still be writing LDS when the workgroup retires; wait
  // states between the last MFMA results and the epilogue's reads
  asm volatile("s_waitcnt vmcnt(0)\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7\n\ts_nop 7"
               ::: "memory");
#pragma unroll
  for (int c = 0; c < CW; ++c) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) { asm volatile("" : "+v"(acc[c][mt])); }
  }

#pragma unroll
  for (int c = 0; c < CW; ++c) {
    const int n = n0 + 16 * c + 4 * g;
    if (n >= P.n) { return; }
    uint2 bb = make_uint2(0u, 0u);
    if (S == 1 && P.bias != nullptr) { bb = *reinterpret_cast<const uint2*>(P.bias + n); }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int m = mt * 16 + r;
      if (m >= P.rows) { continue; }
      if (S == 1) {
        skinny_store(P, m, n, acc[c][mt], bb);
      } else {
        float* ws = B.ws + P.ws_off + (size_t)share * P.rows * P.n;
        *reinterpret_cast<f32x4_t*>(ws + (size_t)m * P.n + n) = acc[c][mt];
      }
    }
  }
}

template <int MT, int D, int QB, int CW = 1>
__global__ __launch_bounds__(256) void
skinny_lds_kernel(const SkinnyBatch B)
{
  static_assert(D == 3 || D == 4, "a ring of 3 or 4 stages (8 measured slower)");
  constexpr int kStage = MT * 16 * 128;
  constexpr int kWStage = QB == 0 ? 4 * 2048 * CW : 16;   // weight ring stage
  __shared__ __attribute__((aligned(1024))) char xs0[kStage];
  __shared__ __attribute__((aligned(1024))) char xs1[kStage];
  __shared__ __attribute__((aligned(1024))) char xs2[kStage];
  __shared__ __attribute__((aligned(1024))) char xs3[D == 4 ? kStage : 16];
  __shared__ __attribute__((aligned(1024))) char ws0[kWStage];
  __shared__ __attribute__((aligned(1024))) char ws1[kWStage];
  __shared__ __attribute__((aligned(1024))) char ws2[kWStage];
  __shared__ __attribute__((aligned(1024))) char ws3[D == 4 ? kWStage : 16];
  if constexpr (D == 4) {
    char* const xs[4] = {xs0, xs1, xs2, xs3};
    char* const wsr[4] = {ws0, ws1, ws2, ws3};
    skinny_lds_tile<MT, 4, QB, CW>(B, xs, wsr);
  } else {
    char* const xs[3] = {xs0, xs1, xs2};
    char* const wsr[3] = {ws0, ws1, ws2};
    skinny_lds_tile<MT, 3, QB, CW>(B, xs, wsr);
  }
}

// Sums the S partial sums of every output in share order, adds the bias
// and rounds to bf16: one thread per 4 columns of a row; blockIdx.y is the
// problem.
__global__ __launch_bounds__(256) void
skinny_reduce_kernel(const SkinnyBatch B)
{
  const SkinnyProblem& P = B.p[blockIdx.y];
  const int q = P.n / 4;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)P.rows * q) { return; }
  const int m = (int)(idx / q);
  const int n = (int)(idx - (int64_t)m * q) * 4;
  const size_t plane = (size_t)P.rows * P.n;
  const float* ws = B.ws + P.ws_off + (size_t)m * P.n + n;
  f32x4_t v = *reinterpret_cast<const f32x4_t*>(ws);
  for (int sh = 1; sh < B.split; ++sh) {
    v += *reinterpret_cast<const f32x4_t*>(ws + sh * plane);
  }
  uint2 bb = make_uint2(0u, 0u);
  if (P.bias != nullptr) { bb = *reinterpret_cast<const uint2*>(P.bias + n); }
  skinny_store(P, m, n, v, bb);
}

// ---- row gather / scatter for per-token routing ------------------------
template <bool kScatter>
__global__ __launch_bounds__(256) void
gather_rows_kernel(const uint16_t* __restrict__ src,
                   const int32_t* __restrict__ perm, int M, int cols,
                   uint16_t* __restrict__ dst)
{
  const int i = blockIdx.x;
  const int pr = perm[i];
  // perm is caller data in device memory: an index outside [0, M) copies
  // nothing rather than touching memory outside the two matrices.
  if (pr < 0 || pr >= M) { return; }
  const size_t from = (size_t)(kScatter ? i : pr) * cols;
  const size_t to = (size_t)(kScatter ? pr : i) * cols;
  const uint4* s = reinterpret_cast<const uint4*>(src + from);
  uint4* d = reinterpret_cast<uint4*>(dst + to);
  for (int c = threadIdx.x; c < cols / 8; c += 256) { d[c] = s[c]; }
}

// A launch whose start / end timestamps go to e0 / e1 when either is set
// (events bound to the dispatch itself, so profiling adds no packets to
// the stream).
template <class F, class... A>
void
launch_timed(F kernel, dim3 grid, dim3 block, hipStream_t s, hipEvent_t e0,
             hipEvent_t e1, A... args)
{
  if (e0 != nullptr || e1 != nullptr) {
    hipExtLaunchKernelGGL(kernel, grid, block, 0, s, e0, e1, 0, args...);
  } else {
    hipLaunchKernelGGL(kernel, grid, block, 0, s, args...);
  }
}

template <class Mma, Epi E, int WN>
hipError_t
launch_gemm(const GemmBatch& b, int cus, hipStream_t s, const GemmEvents& ev)
{
  if (b.total_tiles <= 0) { return hipSuccess; }
  const int items = grid_blocks(b);
  const int grid = (cus > 0 && cus < items) ? cus : items;
  launch_timed(mot_gemm_kernel<Mma, E, WN>, dim3(grid), dim3(128 * WN), s,
               ev.before, ev.after, b);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || b.split_begin >= b.total_tiles) { return e; }
  constexpr bool kInt = Mma::kInt;
  launch_timed(split_reduce_kernel<kInt, E, WN>,
               dim3((b.total_tiles - b.split_begin) * (kBM / (4 * kReduceRowsPerThread))),
               dim3(256), s, ev.red_before, ev.red_after, b);
  return hipGetLastError();
}

template <class F>
hipError_t
launch_skinny(F kernel, const SkinnyBatch& b, hipStream_t s, const GemmEvents& ev)
{
  launch_timed(kernel, dim3(b.total_cb * b.split), dim3(256), s, ev.before,
               ev.after, b);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess || b.split <= 1) { return e; }
  int64_t most = 0;
  for (int i = 0; i < b.nprob; ++i) {
    most = std::max<int64_t>(most, (int64_t)b.p[i].rows * (b.p[i].n / 4));
  }
  launch_timed(skinny_reduce_kernel, dim3((unsigned)((most + 255) / 256), b.nprob),
               dim3(256), s, ev.red_before, ev.red_after, b);
  return hipGetLastError();
}

template <int QB>
hipError_t
launch_skinny_q(const SkinnyBatch& b, hipStream_t s, const GemmEvents& ev)
{
  if (b.max_rows <= 16) {
    if constexpr (QB == 0) {
      return launch_skinny(skinny_dma_kernel<1>, b, s, ev);
    } else {
      return launch_skinny(skinny_reg_kernel<1, QB>, b, s, ev);
    }
  }
  if (b.max_rows <= 32) { return launch_skinny(skinny_lds_kernel<2, 4, QB>, b, s, ev); }
  if (b.max_rows <= 64) { return launch_skinny(skinny_lds_kernel<4, 4, QB>, b, s, ev); }
  if (b.max_rows <= 96) {
    if (QB == 0 && b.cols == 128) { return launch_skinny(skinny_lds_kernel<6, 4, 0, 2>, b, s, ev); }
    return launch_skinny(skinny_lds_kernel<6, 4, QB>, b, s, ev);
  }
  if constexpr (QB == 0) {
    if (b.cols == 128) { return launch_skinny(skinny_lds_kernel<8, 4, QB, 2>, b, s, ev); }
    return launch_skinny(skinny_lds_kernel<8, 3, QB>, b, s, ev);
  } else {
    return launch_skinny(skinny_lds_kernel<8, 4, QB>, b, s, ev);
  }
}

}  // namespace

hipError_t
launch_skinny_bf16(const SkinnyBatch& b, hipStream_t s, const GemmEvents& ev)
{
  if (b.total_cb <= 0 || b.max_rows <= 0) { return hipSuccess; }
  if (b.max_rows > kSkinnyMaxRows || b.kbytes % 128 != 0 ||
      (b.cols != skinny_cols(b.max_rows, b.qbits) &&
       !(skinny_wide_ok(b.max_rows, b.qbits) && b.cols == 2 * skinny_cols(b.max_rows, b.qbits))) ||
      (b.qbits != 0 && b.qgroup != 32 && b.qgroup != 64)) {
    return hipErrorInvalidValue;
  }
  switch (b.qbits) {
    case 0: return launch_skinny_q<0>(b, s, ev);
    case 4: return launch_skinny_q<4>(b, s, ev);
    case 8: return launch_skinny_q<8>(b, s, ev);
    default: return hipErrorInvalidValue;
  }
}

namespace {

template <class Mma, Epi E>
hipError_t
launch_gemm_waves(const GemmBatch& b, const GemmShape& g, hipStream_t s,
                  const GemmEvents& ev)
{
  // the 4-wave workgroup (one wave per SIMD, 512 registers) runs the 16x16
  // MFMAs; the 8-wave one the 32x32 MFMAs, whose fragments fit 256
  if (g.waves == 4) { return launch_gemm<typename Mma::x16, E, 2>(b, g.cus, s, ev); }
  const bool x16 = g.mfma16 > 0 || (g.mfma16 < 0 && Mma::kInt);
  return x16 ? launch_gemm<typename Mma::x16, E, 4>(b, g.cus, s, ev)
             : launch_gemm<Mma, E, 4>(b, g.cus, s, ev);
}

}  // namespace

hipError_t
launch_gemm_bf16(const GemmBatch& b, Epi epi, const GemmShape& g,
                 hipStream_t s, const GemmEvents& ev)
{
  switch (epi) {
    case Epi::kBf16:
      return launch_gemm_waves<MmaBf16, Epi::kBf16>(b, g, s, ev);
    case Epi::kSwiglu:
      return launch_gemm_waves<MmaBf16, Epi::kSwiglu>(b, g, s, ev);
    default: return hipErrorInvalidValue;
  }
}

hipError_t
launch_gemm_i8(const GemmBatch& b, Epi epi, const GemmShape& g, hipStream_t s,
               const GemmEvents& ev)
{
  switch (epi) {
    case Epi::kI32:
      return launch_gemm_waves<MmaI8, Epi::kI32>(b, g, s, ev);
    case Epi::kDequantBf16:
      return launch_gemm_waves<MmaI8, Epi::kDequantBf16>(b, g, s, ev);
    default: return hipErrorInvalidValue;
  }
}

hipError_t
launch_quant_rows_i8(const uint16_t* x, int rows, int K, int8_t* q,
                     float* sc, hipStream_t s, hipEvent_t start, hipEvent_t end)
{
  if (rows <= 0) { return hipSuccess; }
  // Up to 8192 columns: four waves per row, each lane holding 1, 2 or 4
  // chunks (K = 4096, 4224 rows: 12.6 us against 14.7 for the earlier
  // row kernel, one box, interleaved).  8192 < K <= 16384 (K % 16 == 0;
  // the down projection's 12288): the wide kernel.  Longer rows stream
  // their rest twice.
  if (K <= 2048) {
    launch_timed(quant_rows_i8_waves_kernel<4, 1, 1>, dim3(rows), dim3(256), s,
                 start, end, x, rows, K, q, sc);
  } else if (K <= 4096) {
    launch_timed(quant_rows_i8_waves_kernel<4, 2, 1>, dim3(rows), dim3(256), s,
                 start, end, x, rows, K, q, sc);
  } else if (K <= 8192) {
    launch_timed(quant_rows_i8_waves_kernel<4, 4, 1>, dim3(rows), dim3(256), s,
                 start, end, x, rows, K, q, sc);
  } else if (K <= 16384 && K % 16 == 0) {
    launch_timed(quant_rows_i8_wide_kernel, dim3(rows), dim3(512), s, start, end,
                 x, K, q, sc);
  } else {
    launch_timed(quant_rows_i8_kernel<6>, dim3(rows), dim3(256), s, start, end,
                 x, K, q, sc);
  }
  return hipGetLastError();
}

hipError_t
launch_rms_norm(uint16_t* x, const uint16_t* d, const uint16_t* w_und,
                const uint16_t* w_gen, int m_und, int rows, int dim, float eps,
                uint16_t* y, int8_t* q, float* sc, hipStream_t s)
{
  if (rows <= 0) { return hipSuccess; }
  const int sel = (q != nullptr ? 1 : 0) | (d != nullptr ? 2 : 0);
  // one row per workgroup: four waves up to 8192 columns, eight above
#define U15H_NORM1(WPR, CPL, QU, AD)                                          \
  hipLaunchKernelGGL((rms_norm_rows_kernel<WPR, CPL, QU, AD>), dim3(rows),    \
                     dim3(64 * WPR), 0, s, x, d, w_und, w_gen, m_und, dim,    \
                     eps, y, q, sc)
#define U15H_NORM(WPR, CPL)                                                   \
  do {                                                                        \
    switch (sel) {                                                            \
      case 0: U15H_NORM1(WPR, CPL, false, false); break;                      \
      case 1: U15H_NORM1(WPR, CPL, true, false); break;                       \
      case 2: U15H_NORM1(WPR, CPL, false, true); break;                       \
      default: U15H_NORM1(WPR, CPL, true, true); break;                       \
    }                                                                         \
  } while (0)
  if (dim <= 2048) {
    U15H_NORM(4, 1);
  } else if (dim <= 4096) {
    U15H_NORM(4, 2);
  } else if (dim <= 8192) {
    U15H_NORM(4, 4);
  } else {
    U15H_NORM(8, 4);
  }
#undef U15H_NORM
#undef U15H_NORM1
  return hipGetLastError();
}

hipError_t
launch_swiglu_quant(const uint16_t* gate, const uint16_t* up, int rows, int dim,
                    uint16_t* h, int8_t* q, float* sc, hipStream_t s)
{
  if (rows <= 0) { return hipSuccess; }
#define U15H_SWQ(WPR, CPL)                                                    \
  hipLaunchKernelGGL((swiglu_quant_rows_kernel<WPR, CPL>), dim3(rows),        \
                     dim3(64 * WPR), 0, s, gate, up, dim, h, q, sc)
  if (dim <= 2048) {
    U15H_SWQ(4, 1);
  } else if (dim <= 4096) {
    U15H_SWQ(4, 2);
  } else if (dim <= 8192) {
    U15H_SWQ(4, 4);
  } else if (dim <= 12288) {
    U15H_SWQ(8, 3);
  } else {
    U15H_SWQ(8, 4);
  }
#undef U15H_SWQ
  return hipGetLastError();
}

hipError_t
launch_add_bf16(uint16_t* dst, const uint16_t* src, int64_t n, hipStream_t s)
{
  if (n <= 0) { return hipSuccess; }
  const bool vec = (reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src)) % 16 == 0;
  const int64_t nvec = vec ? n / 8 : 0;
  const int64_t work = nvec > 0 ? nvec : n;
  const int64_t want = (work + 255) / 256;
  hipLaunchKernelGGL(add_bf16_kernel, dim3((unsigned)(want < 8192 ? want : 8192)),
                     dim3(256), 0, s, dst, src, n, nvec);
  return hipGetLastError();
}

hipError_t
launch_swiglu(const uint16_t* g, const uint16_t* u, uint16_t* o, int64_t n,
              hipStream_t s)
{
  const int64_t nvec = n / 8;
  if (nvec <= 0) { return hipSuccess; }
  const int64_t want = (nvec + 255) / 256;
  const int blocks = (int)(want < 8192 ? want : 8192);
  hipLaunchKernelGGL(swiglu_kernel, dim3(blocks), dim3(256), 0, s,
                     reinterpret_cast<const uint4*>(g),
                     reinterpret_cast<const uint4*>(u),
                     reinterpret_cast<uint4*>(o), nvec);
  return hipGetLastError();
}

hipError_t
launch_dequant_affine(const uint32_t* codes, const uint16_t* sc,
                      const uint16_t* bi, int bits, int group, int N, int K,
                      uint16_t* w, hipStream_t s)
{
  const int64_t words = (int64_t)N * (K * bits / 32);
  if (words <= 0) { return hipSuccess; }
  const dim3 grid((unsigned)((words + 255) / 256));
  if (bits == 8) {
    hipLaunchKernelGGL(dequant_affine_kernel<8>, grid, dim3(256), 0, s, codes,
                       sc, bi, group, N, K, w);
  } else {
    hipLaunchKernelGGL(dequant_affine_kernel<4>, grid, dim3(256), 0, s, codes,
                       sc, bi, group, N, K, w);
  }
  return hipGetLastError();
}

hipError_t
launch_bias_add(uint16_t* y, const uint16_t* b, int M, int N, hipStream_t s)
{
  const int64_t nvec = (int64_t)M * N / 8;
  if (nvec <= 0) { return hipSuccess; }
  const int64_t want = (nvec + 255) / 256;
  hipLaunchKernelGGL(bias_add_kernel, dim3((unsigned)(want < 8192 ? want : 8192)),
                     dim3(256), 0, s, y, b, N, nvec);
  return hipGetLastError();
}

hipError_t
launch_f32_to_bf16(const float* src, int64_t n, uint16_t* dst, hipStream_t s)
{
  const int64_t nvec = n / 4;
  if (nvec <= 0) { return hipSuccess; }
  const int64_t want = (nvec + 255) / 256;
  hipLaunchKernelGGL(f32_to_bf16_kernel,
                     dim3((unsigned)(want < 8192 ? want : 8192)), dim3(256), 0,
                     s, reinterpret_cast<const float4*>(src),
                     reinterpret_cast<uint2*>(dst), nvec);
  return hipGetLastError();
}

hipError_t
launch_split_norm_rope(uint16_t* x, const uint16_t* w_t, const uint16_t* w_hw,
                       const float* cosf, const float* sinf, int rows, int H,
                       int D, int d_t, int d_h, float eps, bool norm, bool rope,
                       hipStream_t s)
{
  if (rows <= 0) { return hipSuccess; }
  auto pow2 = [](int v) { return v > 0 && (v & (v - 1)) == 0; };
  const uintptr_t addr_bits =
      reinterpret_cast<uintptr_t>(x) |
      (norm ? reinterpret_cast<uintptr_t>(w_t) | reinterpret_cast<uintptr_t>(w_hw) : 0) |
      (rope ? reinterpret_cast<uintptr_t>(cosf) | reinterpret_cast<uintptr_t>(sinf) : 0);
  const bool ranges_ok = d_t % 16 == 0 && d_h % 16 == 0 && pow2(d_t / 16) &&
                         pow2(d_h / 16) && d_t % d_h == 0;
  if (addr_bits % 16 == 0 && pow2(D) && D >= 16 && D <= 512 && (!rope || ranges_ok)) {
    const long long threads = (long long)rows * (D / 8);
    const dim3 vgrid((unsigned)((threads + 255) / 256));
    if (norm && rope) {
      hipLaunchKernelGGL((split_norm_rope_vec_kernel<true, true>), vgrid, dim3(256), 0, s,
                         x, w_t, w_hw, cosf, sinf, rows, H, D, d_t, d_h, eps);
    } else if (norm) {
      hipLaunchKernelGGL((split_norm_rope_vec_kernel<true, false>), vgrid, dim3(256), 0, s,
                         x, w_t, w_hw, cosf, sinf, rows, H, D, d_t, d_h, eps);
    } else {
      hipLaunchKernelGGL((split_norm_rope_vec_kernel<false, true>), vgrid, dim3(256), 0, s,
                         x, w_t, w_hw, cosf, sinf, rows, H, D, d_t, d_h, eps);
    }
    return hipGetLastError();
  }
  const dim3 grid((unsigned)((rows + 3) / 4));
  if (norm && rope) {
    hipLaunchKernelGGL((split_norm_rope_kernel<true, true>), grid, dim3(256),
                       0, s, x, w_t, w_hw, cosf, sinf, rows, H, D, d_t, d_h,
                       eps);
  } else if (norm) {
    hipLaunchKernelGGL((split_norm_rope_kernel<true, false>), grid, dim3(256),
                       0, s, x, w_t, w_hw, cosf, sinf, rows, H, D, d_t, d_h,
                       eps);
  } else {
    hipLaunchKernelGGL((split_norm_rope_kernel<false, true>), grid, dim3(256),
                       0, s, x, w_t, w_hw, cosf, sinf, rows, H, D, d_t, d_h,
                       eps);
  }
  return hipGetLastError();
}

template <int RPT>
static hipError_t
launch_attention_prologue_rpt(const PrologueArgs& a, hipStream_t s)
{
  const int gpb = 256 / (a.d / 8);
  const long long nq = (long long)a.tokens * (a.hq / RPT);
  const long long nk = (long long)a.tokens * (a.hkv / RPT);
  const long long blocks = (nq + gpb - 1) / gpb + 2 * ((nk + gpb - 1) / gpb);
  hipLaunchKernelGGL(attention_prologue_kernel<RPT>, dim3((unsigned)blocks),
                     dim3(256), 0, s, a);
  return hipGetLastError();
}

hipError_t
launch_attention_prologue(const PrologueArgs& a, hipStream_t s, int max_rpt)
{
  if (a.tokens <= 0) { return hipSuccess; }
  if (max_rpt >= 4 && a.hq % 4 == 0 && a.hkv % 4 == 0) {
    return launch_attention_prologue_rpt<4>(a, s);
  }
  if (max_rpt >= 2 && a.hq % 2 == 0 && a.hkv % 2 == 0) {
    return launch_attention_prologue_rpt<2>(a, s);
  }
  return launch_attention_prologue_rpt<1>(a, s);
}

hipError_t
launch_f16_to_bf16(const uint16_t* src, int64_t n, uint16_t* dst, hipStream_t s)
{
  const int64_t nvec = n / 4;
  if (nvec <= 0) { return hipSuccess; }
  const int64_t want = (nvec + 255) / 256;
  hipLaunchKernelGGL(f16_to_bf16_kernel,
                     dim3((unsigned)(want < 8192 ? want : 8192)), dim3(256), 0,
                     s, reinterpret_cast<const uint2*>(src),
                     reinterpret_cast<uint2*>(dst), nvec);
  return hipGetLastError();
}

template <int D, int MODE>
hipError_t
launch_attention_d(const AttnArgs& a, hipStream_t s)
{
  constexpr int NWV = attn_waves<MODE>();
  const int ntq = (a.tq + 32 * NWV - 1) / (32 * NWV);
  hipLaunchKernelGGL((attention_kernel<D, MODE, NWV>), dim3(a.hq * ntq), dim3(64 * NWV),
                     0, s, a);
  return hipGetLastError();
}

template <int D>
hipError_t
launch_attention_mode(const AttnArgs& a, hipStream_t s)
{
  if (a.mode == 1) { return launch_attention_d<D, 1>(a, s); }
  if (a.mode == 2) { return launch_attention_d<D, 2>(a, s); }
  return launch_attention_d<D, 0>(a, s);
}

hipError_t
launch_attention(const AttnArgs& a, hipStream_t s)
{
  if (a.tq <= 0) { return hipSuccess; }
  if (a.d == 128) { return launch_attention_mode<128>(a, s); }
  if (a.d == 64) { return launch_attention_mode<64>(a, s); }
  return launch_attention_mode<32>(a, s);
}

hipError_t
launch_transpose_rows(const uint16_t* src, uint16_t* dst, int T, int H, int D,
                      long long src_t, long long src_h, long long dst_t,
                      long long dst_h, hipStream_t s)
{
  const long long n = (long long)T * H * (D / 8);
  if (n <= 0) { return hipSuccess; }
  const long long want = (n + 255) / 256;
  hipLaunchKernelGGL(transpose_rows_kernel,
                     dim3((unsigned)(want < 8192 ? want : 8192)), dim3(256), 0,
                     s, src, dst, T, H, D, src_t, src_h, dst_t, dst_h);
  return hipGetLastError();
}

hipError_t
launch_gather_rows(const uint16_t* src, const int32_t* perm, int M, int cols,
                   uint16_t* dst, bool scatter, hipStream_t s)
{
  if (M <= 0) { return hipSuccess; }
  if (scatter) {
    hipLaunchKernelGGL(gather_rows_kernel<true>, dim3(M), dim3(256), 0, s, src,
                       perm, M, cols, dst);
  } else {
    hipLaunchKernelGGL(gather_rows_kernel<false>, dim3(M), dim3(256), 0, s,
                       src, perm, M, cols, dst);
  }
  return hipGetLastError();
}

}  // namespace u15h

// ---- the allocation-free entry point's scratch ----------------------------
// Split-K partial sums for u15h_mot_linear_noalloc: one 256 x 256 tile of
// 4-byte partial sums per compute unit of a GPU with up to 256 CUs (the
// planner never asks for more than one per CU), 64 MiB per device, held
// by every device the library runs on until the process ends.  Host code
// must not pass `scratch` itself to a kernel: in host code the name is a
// host-side stand-in, not a device address.  Its per-device address comes
// from hipGetSymbolAddress below and is the only handle host code uses.
static __device__ __align__(256) char scratch[u15h::kNoAllocScratchBytes];

namespace u15h {

hipError_t
noalloc_scratch(int device, void** out)
{
  // Looked up once per device (with that device current: u15h_create
  // calls this right after binding it) and kept; each GPU holds its own
  // copy of the array at its own address.
  static std::mutex mu;
  static bool done[kMaxScratchDevices];
  static hipError_t res[kMaxScratchDevices];
  static void* ptr[kMaxScratchDevices];
  *out = nullptr;
  if (device < 0 || device >= kMaxScratchDevices) { return hipErrorInvalidDevice; }
  std::lock_guard<std::mutex> lock(mu);
  if (!done[device]) {
    void* p = nullptr;
    res[device] = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    ptr[device] = res[device] == hipSuccess ? p : nullptr;
    done[device] = true;
  }
  *out = ptr[device];
  return res[device];
}

namespace {

template <class MB, class MI, int WN>
bool
gemm_kernels_loadable()
{
  const void* fns[] = {
      reinterpret_cast<const void*>(&mot_gemm_kernel<MB, Epi::kBf16, WN>),
      reinterpret_cast<const void*>(&mot_gemm_kernel<MB, Epi::kSwiglu, WN>),
      reinterpret_cast<const void*>(&mot_gemm_kernel<MI, Epi::kI32, WN>),
      reinterpret_cast<const void*>(&mot_gemm_kernel<MI, Epi::kDequantBf16, WN>),
      reinterpret_cast<const void*>(&split_reduce_kernel<false, Epi::kBf16, WN>),
      reinterpret_cast<const void*>(&split_reduce_kernel<false, Epi::kSwiglu, WN>),
      reinterpret_cast<const void*>(&split_reduce_kernel<true, Epi::kI32, WN>),
      reinterpret_cast<const void*>(&split_reduce_kernel<true, Epi::kDequantBf16, WN>),
  };
  for (const void* f : fns) {
    hipFuncAttributes a;
    if (hipFuncGetAttributes(&a, f) != hipSuccess) { return false; }
  }
  return true;
}

}  // namespace

bool
kernels_loadable()
{
  const void* fns[] = {
      reinterpret_cast<const void*>(&f16_to_bf16_kernel),
      reinterpret_cast<const void*>(&attention_kernel<128, 0, attn_waves<0>()>),
      reinterpret_cast<const void*>(&attention_kernel<128, 1, attn_waves<1>()>),
      reinterpret_cast<const void*>(&attention_kernel<128, 2, attn_waves<2>()>),
      reinterpret_cast<const void*>(&attention_kernel<64, 0, attn_waves<0>()>),
      reinterpret_cast<const void*>(&attention_kernel<64, 1, attn_waves<1>()>),
      reinterpret_cast<const void*>(&attention_kernel<64, 2, attn_waves<2>()>),
      reinterpret_cast<const void*>(&attention_kernel<32, 0, attn_waves<0>()>),
      reinterpret_cast<const void*>(&attention_kernel<32, 1, attn_waves<1>()>),
      reinterpret_cast<const void*>(&attention_kernel<32, 2, attn_waves<2>()>),
      reinterpret_cast<const void*>(&transpose_rows_kernel),
      reinterpret_cast<const void*>(&split_norm_rope_kernel<true, true>),
      reinterpret_cast<const void*>(&split_norm_rope_kernel<true, false>),
      reinterpret_cast<const void*>(&split_norm_rope_kernel<false, true>),
      reinterpret_cast<const void*>(&split_norm_rope_vec_kernel<true, true>),
      reinterpret_cast<const void*>(&split_norm_rope_vec_kernel<true, false>),
      reinterpret_cast<const void*>(&split_norm_rope_vec_kernel<false, true>),
      reinterpret_cast<const void*>(&attention_prologue_kernel<1>),
      reinterpret_cast<const void*>(&rms_norm_rows_kernel<4, 1, false, false>),
      reinterpret_cast<const void*>(&rms_norm_rows_kernel<4, 1, true, false>),
      reinterpret_cast<const void*>(&rms_norm_rows_kernel<4, 1, false, true>),
      reinterpret_cast<const void*>(&rms_norm_rows_kernel<4, 1, true, true>),
      reinterpret_cast<const void*>(&rms_norm_rows_kernel<4, 2, false, false>),
      reinterpret_cast<const void*>(&rms_norm_rows_kernel<4, 2, true, false>),
      reinterpret_cast<const void*>(&rms_norm_rows_kernel<4, 2, false, true>),
      reinterpret_cast<const void*>(&rms_norm_rows_kernel<4, 2, true, true>),
      reinterpret_cast<const void*>(&rms_norm_rows_kernel<4, 4, false, false>),
      reinterpret_cast<const void*>(&rms_norm_rows_kernel<4, 4, true, false>),
      reinterpret_cast<const void*>(&rms_norm_rows_kernel<4, 4, false, true>),
      reinterpret_cast<const void*>(&rms_norm_rows_kernel<4, 4, true, true>),
      reinterpret_cast<const void*>(&rms_norm_rows_kernel<8, 4, false, false>),
      reinterpret_cast<const void*>(&rms_norm_rows_kernel<8, 4, true, false>),
      reinterpret_cast<const void*>(&rms_norm_rows_kernel<8, 4, false, true>),
      reinterpret_cast<const void*>(&rms_norm_rows_kernel<8, 4, true, true>),
      reinterpret_cast<const void*>(&add_bf16_kernel),
      reinterpret_cast<const void*>(&swiglu_quant_rows_kernel<4, 1>),
      reinterpret_cast<const void*>(&swiglu_quant_rows_kernel<4, 2>),
      reinterpret_cast<const void*>(&swiglu_quant_rows_kernel<4, 4>),
      reinterpret_cast<const void*>(&swiglu_quant_rows_kernel<8, 3>),
      reinterpret_cast<const void*>(&swiglu_quant_rows_kernel<8, 4>),
      reinterpret_cast<const void*>(&attention_prologue_kernel<2>),
      reinterpret_cast<const void*>(&attention_prologue_kernel<4>),
      reinterpret_cast<const void*>(&quant_rows_i8_waves_kernel<4, 1, 1>),
      reinterpret_cast<const void*>(&quant_rows_i8_waves_kernel<4, 2, 1>),
      reinterpret_cast<const void*>(&quant_rows_i8_waves_kernel<4, 4, 1>),
      reinterpret_cast<const void*>(&quant_rows_i8_kernel<6>),
      reinterpret_cast<const void*>(&quant_rows_i8_wide_kernel),
      reinterpret_cast<const void*>(&swiglu_kernel),
      reinterpret_cast<const void*>(&dequant_affine_kernel<8>),
      reinterpret_cast<const void*>(&dequant_affine_kernel<4>),
      reinterpret_cast<const void*>(&bias_add_kernel),
      reinterpret_cast<const void*>(&f32_to_bf16_kernel),
      reinterpret_cast<const void*>(&gather_rows_kernel<true>),
      reinterpret_cast<const void*>(&gather_rows_kernel<false>),
      reinterpret_cast<const void*>(&skinny_reg_kernel<1, 0>),
      reinterpret_cast<const void*>(&skinny_dma_kernel<1>),
      reinterpret_cast<const void*>(&skinny_lds_kernel<2, 4, 0>),
      reinterpret_cast<const void*>(&skinny_lds_kernel<4, 4, 0>),
      reinterpret_cast<const void*>(&skinny_lds_kernel<6, 4, 0>),
      reinterpret_cast<const void*>(&skinny_lds_kernel<8, 3, 0>),
      reinterpret_cast<const void*>(&skinny_lds_kernel<8, 4, 0, 2>),
      reinterpret_cast<const void*>(&skinny_lds_kernel<6, 4, 0, 2>),
      reinterpret_cast<const void*>(&skinny_reg_kernel<1, 4>),
      reinterpret_cast<const void*>(&skinny_lds_kernel<2, 4, 4>),
      reinterpret_cast<const void*>(&skinny_lds_kernel<4, 4, 4>),
      reinterpret_cast<const void*>(&skinny_lds_kernel<6, 4, 4>),
      reinterpret_cast<const void*>(&skinny_lds_kernel<8, 4, 4>),
      reinterpret_cast<const void*>(&skinny_reg_kernel<1, 8>),
      reinterpret_cast<const void*>(&skinny_lds_kernel<2, 4, 8>),
      reinterpret_cast<const void*>(&skinny_lds_kernel<4, 4, 8>),
      reinterpret_cast<const void*>(&skinny_lds_kernel<6, 4, 8>),
      reinterpret_cast<const void*>(&skinny_lds_kernel<8, 4, 8>),
      reinterpret_cast<const void*>(&skinny_reduce_kernel),
  };
  for (const void* f : fns) {
    hipFuncAttributes a;
    if (hipFuncGetAttributes(&a, f) != hipSuccess) { return false; }
  }
  return gemm_kernels_loadable<MmaBf16x16, MmaI8x16, 2>() &&
         gemm_kernels_loadable<MmaBf16x16, MmaI8x16, 4>() &&
         gemm_kernels_loadable<MmaBf16, MmaI8, 4>();
}

}  // namespace u15h
