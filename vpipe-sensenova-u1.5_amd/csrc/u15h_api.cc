// u15h_api.cc -- the C ABI (include/u15h.h) over the gfx950 kernels.
//
// Host side of the boundary: argument checks (nothing is launched on a
// refusal), the batch tables the kernels read, the int8 tier's on/decline
// state and its grow-only scratch.
#include "u15h.h"

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "u15h_internal.h"

struct u15h_ctx {
  int device = 0;
  int num_cu = 256;
  int gemm_cus = 256;        // CUs the tiled GEMM's rounds are planned for
  bool split_on = true;      // env U15H_SPLIT=0 turns the split-K tail off
  // env U15H_SKINNY=0 keeps batches of <= 128-row problems on the tiled GEMM
  bool skinny_on = true;
  // heads of one token per thread in u15h_mot_attention_prologue (1, 2 or
  // 4; env U15H_PROLOGUE_RPT).  At config 2 (4224 tokens, 32 + 8 + 8
  // heads of 128) 2 measured 21.6-21.9 us against 22.9-24.5 (1) and
  // 23.0-24.9 (4), three interleaved rounds on one box.
  int prologue_rpt = 2;
  // u15h_linear_q below this many rows reads the pack directly (the
  // reference's _mma_q_min_m, u15-metal-ops.h:502; env U15H_Q_MIN_M)
  int q_min_m = 96;
  // GEMM kernel build: 8 or 4 waves per workgroup (env U15H_WAVES) and the
  // 8-wave build's MFMA shape (env U15H_MFMA16).
  u15h::GemmShape gemm = {8, 0, 1};
  // One-shot profiling events, bound to the next launches of a quantiser,
  // a GEMM kernel and its reduction (start and end of each); all dropped
  // when the next GEMM call has launched.
  hipEvent_t prof_quant[2] = {nullptr, nullptr};
  u15h::GemmEvents prof_gemm;
  // Partial-sum workspace of split tiles: at most num_cu K shares of one
  // 256x256 tile each (allocated on first use, kept until destroy).
  void* split_ws = nullptr;
  // The device address of the static split-K scratch that
  // u15h_mot_linear_noalloc uses instead (looked up at create; null if the
  // lookup failed, with the HIP error kept for the message).
  void* noalloc_ws = nullptr;
  hipError_t noalloc_err = hipSuccess;
  bool i8_on = false;
  int i8_min_m = 1024;
  // Grow-only scratch of the int8 route of u15h_linear: activation and
  // weight codes + scales.
  void* i8_scratch = nullptr;
  size_t i8_scratch_bytes = 0;
  // Grow-only bf16 expansion of an affine-quantized weight (the
  // reference's `_w_deq`, u15-metal-ops.h:461-469).
  void* w_deq = nullptr;
  size_t w_deq_bytes = 0;
  std::string err;
};

namespace {

using u15h::Epi;
using u15h::GemmBatch;
using u15h::GemmProblem;

u15h_status
fail(u15h_ctx* ctx, u15h_status st, const char* fmt, ...)
{
  if (ctx != nullptr) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    std::vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    ctx->err = buf;
  }
  return st;
}

bool
aligned16(const void* p)
{
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

// Makes the context's device current for the calling thread.
u15h_status
bind_device(u15h_ctx* ctx)
{
  int cur = -1;
  if (hipGetDevice(&cur) != hipSuccess) {
    return fail(ctx, U15H_ENODEV, "hipGetDevice failed");
  }
  if (cur != ctx->device && hipSetDevice(ctx->device) != hipSuccess) {
    return fail(ctx, U15H_ENODEV, "hipSetDevice(%d) failed", ctx->device);
  }
  return U15H_OK;
}

// The profiling events of the next GEMM launch (one-shot: taking them
// drops every pending profiling event, the quantiser's included).
u15h::GemmEvents
take_profile_event(u15h_ctx* ctx)
{
  const u15h::GemmEvents e = ctx->prof_gemm;
  ctx->prof_gemm = u15h::GemmEvents{};
  ctx->prof_quant[0] = ctx->prof_quant[1] = nullptr;
  return e;
}

// The profiling events of the next quantiser launch (one-shot).
void
take_quant_events(u15h_ctx* ctx, hipEvent_t* start, hipEvent_t* end)
{
  *start = ctx->prof_quant[0];
  *end = ctx->prof_quant[1];
  ctx->prof_quant[0] = ctx->prof_quant[1] = nullptr;
}

u15h_status
launched(u15h_ctx* ctx, hipError_t e, const char* what)
{
  if (e != hipSuccess) {
    return fail(ctx, U15H_ELAUNCH, "%s: %s", what, hipGetErrorString(e));
  }
  ctx->err.clear();
  return U15H_OK;
}

// Appends one problem (one weight set applied to one row range) to a
// batch.  Empty row ranges add no tiles.
void
add_problem(GemmBatch& b, const void* a, const void* w, const void* w2,
            void* y, const uint16_t* bias, const float* sa, const float* sw,
            int rows, int n, int ldy, int tile_cols, int wld = 0)
{
  if (rows <= 0) { return; }
  GemmProblem& p = b.p[b.nprob++];
  p.a = a;
  p.w = w;
  p.w2 = w2;
  p.y = y;
  p.bias = bias;
  p.sa = sa;
  p.sw = sw;
  p.rows = rows;
  p.n = n;
  p.wld = wld > 0 ? wld : b.kbytes;
  p.ldy = ldy;
  p.tiles_m = (rows + u15h::kBM - 1) / u15h::kBM;
  p.tiles_n = (n + tile_cols - 1) / tile_cols;
  p.tile_begin = b.total_tiles;
  b.total_tiles += p.tiles_m * p.tiles_n;
}

GemmBatch
empty_batch(int kbytes)
{
  GemmBatch b;
  std::memset(&b, 0, sizeof b);
  b.kbytes = kbytes;
  b.split = 1;
  return b;
}

// Fewest K stages a split share may have.
constexpr int kMinStagesPerShare = 4;

size_t
split_ws_capacity(const u15h_ctx* ctx)
{
  return (size_t)ctx->num_cu * u15h::kBM * u15h::kBN * 4;
}

// Chooses the split-K tail of a batch once its tiles are known.  With T
// tiles on C compute units, the last T % C tiles would run as a last,
// partial round that leaves most units idle; instead each is cut into
// S = C / (T % C) shares of its K stages (so the shares fill about one
// round), at least kMinStagesPerShare stages each.  The partial sums go to
// the context's workspace (allocated on first use), or with `noalloc` to
// the static scratch, which allocates nothing.
u15h_status
plan_split(u15h_ctx* ctx, GemmBatch& b, bool noalloc = false)
{
  b.split = 1;
  b.split_begin = b.total_tiles;
  b.ws = nullptr;
  const int T = b.total_tiles;
  const int C = ctx->gemm_cus;
  const int rem = T % C;
  if (!ctx->split_on || T <= 0 || rem == 0) { return U15H_OK; }
  const int nk = (b.kbytes + u15h::kKB - 1) / u15h::kKB;
  const int S = std::min(C / rem, nk / kMinStagesPerShare);
  if (S < 2) { return U15H_OK; }
  b.split = S;
  b.split_begin = T - rem;
  if (noalloc) {
    if (ctx->noalloc_ws == nullptr) {
      return fail(ctx, U15H_ENODEV, "static split-K scratch unavailable: %s",
                  hipGetErrorString(ctx->noalloc_err));
    }
    if (split_ws_bytes(b) > u15h::kNoAllocScratchBytes) {
      return fail(ctx, U15H_EINVAL, "split-K partial sums of %zu bytes exceed "
                  "the static scratch of %zu bytes", split_ws_bytes(b),
                  u15h::kNoAllocScratchBytes);
    }
    b.ws = ctx->noalloc_ws;
    return U15H_OK;
  }
  if (ctx->split_ws == nullptr) {
    if (hipMalloc(&ctx->split_ws, split_ws_capacity(ctx)) != hipSuccess) {
      ctx->split_ws = nullptr;
      return fail(ctx, U15H_ENOMEM, "split-K workspace of %zu bytes",
                  split_ws_capacity(ctx));
    }
  }
  b.ws = ctx->split_ws;
  return split_ws_bytes(b) <= split_ws_capacity(ctx)
             ? U15H_OK
             : fail(ctx, U15H_EINVAL, "split workspace overflow");
}

// The skinny route: a bf16 batch whose problems all have at most 128 rows
// (und prefill, small decode-like steps) and plain [N][K] weights.  There
// the weights are the traffic; the tiled GEMM would run its 256-row tiles
// mostly empty.
bool
skinny_fits(const u15h_ctx* ctx, const GemmBatch& b)
{
  if (!ctx->skinny_on || b.nprob <= 0 || b.kbytes % 128 != 0) { return false; }
  for (int i = 0; i < b.nprob; ++i) {
    const GemmProblem& p = b.p[i];
    if (p.rows > u15h::kSkinnyMaxRows || p.wld != b.kbytes || p.n % 4 != 0) {
      return false;
    }
  }
  return true;
}

// Launches a batch that skinny_fits on the skinny kernels.  K shares S
// (a power of two) are added while the workgroups stay within what the
// CUs hold at once, each share keeps enough K-blocks to fill its waves'
// prefetch, and the fp32 partial sums (written and read once) stay at most
// half the weight bytes: S * rows * 8 <= K.
// The partials go to the split-K workspace (or, with `noalloc`, the static
// scratch); a batch whose partials would not fit takes fewer shares.
u15h_status
skinny_launch(u15h_ctx* ctx, const GemmBatch& b, hipStream_t s, bool noalloc,
              const u15h::GemmEvents& ev, const u15h_qweight* q = nullptr)
{
  u15h::SkinnyBatch k;
  std::memset(&k, 0, sizeof k);
  k.kbytes = b.kbytes;
  k.nprob = b.nprob;
  if (q != nullptr) {         // one problem whose w is the pack's codes
    k.qbits = q->bits;
    k.qgroup = q->group;
    k.p[0].qs = static_cast<const uint16_t*>(q->scales);
    k.p[0].qb = static_cast<const uint16_t*>(q->biases);
  }
  for (int i = 0; i < b.nprob; ++i) { k.max_rows = std::max(k.max_rows, b.p[i].rows); }
  const int K = b.kbytes / 2;
  const int nkb = b.kbytes / 128;
  // Resident workgroups per CU: two for the 16-column-wave builds (at most
  // 80 KiB of LDS each), one for the 32-column-wave builds (112-128 KiB).
  // A share keeps 32 K-blocks (8 per wave) in the register kernel, 16 in
  // the LDS kernels.
  auto blocks = [&](int cols) {
    int cb = 0;
    for (int i = 0; i < b.nprob; ++i) { cb += (b.p[i].n + cols - 1) / cols; }
    return cb;
  };
  auto shares = [&](int cols, int cb, int per_cu) {
    const int min_kb = cols == 16 ? 32 : 16;
    int S = 1;
    while (S < 16 && 2 * S * cb <= per_cu * ctx->num_cu &&
           nkb / (2 * S) >= min_kb && 2 * S * k.max_rows * 8 <= K) {
      S *= 2;
    }
    return S;
  };
  k.cols = u15h::skinny_cols(k.max_rows, k.qbits);
  int S = shares(k.cols, blocks(k.cols), 2);
  // Above 64 rows, bf16 weights: waves of 32 columns (each activation
  // fragment read from LDS serves two weight fragments), with no more K
  // shares than 16-column waves take, where that keeps at least 3/4 of the
  // CUs busy (one such workgroup per CU)
  if (u15h::skinny_wide_ok(k.max_rows, k.qbits)) {
    const int cb2 = blocks(2 * k.cols);
    const int S2 = std::min(shares(2 * k.cols, cb2, 1), S);
    if (4 * S2 * cb2 >= 3 * ctx->num_cu) {
      k.cols *= 2;
      S = S2;
    }
  }
  for (int i = 0; i < b.nprob; ++i) {
    const GemmProblem& p = b.p[i];
    u15h::SkinnyProblem& q = k.p[i];
    q.a = p.a;
    q.w = p.w;
    q.y = p.y;
    q.bias = p.bias;
    q.rows = p.rows;
    q.n = p.n;
    q.ldy = p.ldy;
    q.cb_begin = k.total_cb;
    k.total_cb += (p.n + k.cols - 1) / k.cols;
  }
  // One cap for both destinations, so u15h_mot_linear and
  // u15h_mot_linear_noalloc pick the same share count (and the same bits)
  // on every GPU.
  const size_t cap = std::min(u15h::kNoAllocScratchBytes, split_ws_capacity(ctx));
  for (;;) {
    k.split = S;
    if (S == 1 || u15h::skinny_ws_floats(k) * 4 <= cap) { break; }
    S /= 2;
  }
  if (S > 1) {
    if (noalloc) {
      if (ctx->noalloc_ws == nullptr) {
        return fail(ctx, U15H_ENODEV, "static split-K scratch unavailable: %s",
                    hipGetErrorString(ctx->noalloc_err));
      }
      k.ws = static_cast<float*>(ctx->noalloc_ws);
    } else {
      if (ctx->split_ws == nullptr &&
          hipMalloc(&ctx->split_ws, split_ws_capacity(ctx)) != hipSuccess) {
        ctx->split_ws = nullptr;
        return fail(ctx, U15H_ENOMEM, "split-K workspace of %zu bytes",
                    split_ws_capacity(ctx));
      }
      k.ws = static_cast<float*>(ctx->split_ws);
    }
    size_t off = 0;
    for (int i = 0; i < k.nprob; ++i) {
      k.p[i].ws_off = off;
      off += (size_t)S * k.p[i].rows * k.p[i].n;
    }
  }
  return launched(ctx, u15h::launch_skinny_bf16(k, s, ev), "skinny_gemm_bf16");
}

// Shape limits shared by every GEMM entry point.  Byte offsets inside a
// tile are 32-bit, so one row of K may be at most 2^31 / 256 / 2 bytes.
u15h_status
check_k(u15h_ctx* ctx, int K, int elem, int kmult)
{
  if (K <= 0 || K % kmult != 0) {
    return fail(ctx, U15H_EINVAL, "K=%d must be a positive multiple of %d", K,
                kmult);
  }
  if ((long long)K * elem > (1 << 22)) {
    return fail(ctx, U15H_EINVAL, "K=%d too large", K);
  }
  return U15H_OK;
}

u15h_status
check_rows(u15h_ctx* ctx, int M_und, int M_gen)
{
  if (M_und < 0 || M_gen < 0) {
    return fail(ctx, U15H_EINVAL, "negative row count (M_und=%d M_gen=%d)",
                M_und, M_gen);
  }
  if ((long long)M_und + M_gen > (1 << 24)) {
    return fail(ctx, U15H_EINVAL, "too many rows");
  }
  return U15H_OK;
}

u15h_status
check_n(u15h_ctx* ctx, int N)
{
  if (N <= 0 || N % 8 != 0) {
    return fail(ctx, U15H_EINVAL, "N=%d must be a positive multiple of 8", N);
  }
  // a 256-row output tile of ldy = N bf16 columns addresses below 2^30 bytes
  if (N > (1 << 20)) {
    return fail(ctx, U15H_EINVAL, "N=%d too large (at most 2^20)", N);
  }
  return U15H_OK;
}

// Grid-size guard: the tile count must fit a 1-D grid.
u15h_status
check_tiles(u15h_ctx* ctx, const GemmBatch& b)
{
  if (b.total_tiles < 0 || b.total_tiles > (1 << 30)) {
    return fail(ctx, U15H_EINVAL, "tile count out of range");
  }
  return U15H_OK;
}

int
env_int(const char* name, int dflt)
{
  const char* s = std::getenv(name);
  if (s == nullptr || *s == '\0') { return dflt; }
  return std::atoi(s);
}

hipStream_t
as_stream(u15h_stream s)
{
  return reinterpret_cast<hipStream_t>(s);
}

// The int8 route of u15h_linear: quantise x per row and w per output
// channel into the context's scratch, then the int8 GEMM with the fused
// dequant epilogue.
u15h_status
linear_i8_route(u15h_ctx* ctx, hipStream_t s, const u15h_bf16* x,
                const u15h_bf16* w, const u15h_bf16* bias, u15h_bf16* y,
                int M, int K, int N)
{
  const size_t xq = (size_t)M * K, wq = (size_t)N * K;
  const size_t off_wq = (xq + 255) & ~size_t(255);
  const size_t off_sx = (off_wq + wq + 255) & ~size_t(255);
  const size_t off_sw = (off_sx + (size_t)M * 4 + 255) & ~size_t(255);
  const size_t need = off_sw + (size_t)N * 4;
  if (ctx->i8_scratch_bytes < need) {
    if (ctx->i8_scratch != nullptr) {
      // The old scratch may still be read by queued work on `s`.
      (void)hipStreamSynchronize(s);
      (void)hipFree(ctx->i8_scratch);
      ctx->i8_scratch = nullptr;
      ctx->i8_scratch_bytes = 0;
    }
    if (hipMalloc(&ctx->i8_scratch, need) != hipSuccess) {
      ctx->i8_scratch = nullptr;
      return fail(ctx, U15H_ENOMEM, "int8 scratch of %zu bytes", need);
    }
    ctx->i8_scratch_bytes = need;
  }
  char* base = static_cast<char*>(ctx->i8_scratch);
  int8_t* xqp = reinterpret_cast<int8_t*>(base);
  int8_t* wqp = reinterpret_cast<int8_t*>(base + off_wq);
  float* sx = reinterpret_cast<float*>(base + off_sx);
  float* sw = reinterpret_cast<float*>(base + off_sw);
  hipError_t e = u15h::launch_quant_rows_i8(x, M, K, xqp, sx, s);
  if (e == hipSuccess) { e = u15h::launch_quant_rows_i8(w, N, K, wqp, sw, s); }
  if (e != hipSuccess) { return launched(ctx, e, "quant_rows_i8"); }
  GemmBatch b = empty_batch(K);
  add_problem(b, xqp, wqp, nullptr, y, bias, sx, sw, M, N, N,
              u15h::tile_cols(Epi::kDequantBf16));
  u15h_status st = plan_split(ctx, b);
  if (st != U15H_OK) { return st; }
  return launched(ctx, u15h::launch_gemm_i8(b, Epi::kDequantBf16, ctx->gemm, s, take_profile_event(ctx)),
                  "gemm_i8");
}

}  // namespace

u15h_status
u15h::set_error(u15h_ctx* ctx, u15h_status st, const char* msg)
{
  return fail(ctx, st, "%s", msg);
}

extern "C" {

int
u15h_abi_version(void)
{
  return U15H_ABI_VERSION;
}

const char*
u15h_status_str(u15h_status s)
{
  switch (s) {
    case U15H_OK: return "ok";
    case U15H_EINVAL: return "invalid argument";
    case U15H_ENODEV: return "no usable gfx950 device";
    case U15H_ELAUNCH: return "launch failed";
    case U15H_ENOMEM: return "out of device memory";
  }
  return "unknown status";
}

u15h_status
u15h_create(int device, u15h_ctx** out)
{
  if (out == nullptr) { return U15H_EINVAL; }
  *out = nullptr;
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) {
    return U15H_ENODEV;
  }
  if (device < 0 || device >= count) { return U15H_EINVAL; }
  hipDeviceProp_t prop;
  if (hipGetDeviceProperties(&prop, device) != hipSuccess) {
    return U15H_ENODEV;
  }
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
    return U15H_ENODEV;
  }
  int prev = -1;
  (void)hipGetDevice(&prev);
  if (hipSetDevice(device) != hipSuccess) { return U15H_ENODEV; }
  // Every kernel must load: a missing one is a refusal, not a silent no-op
  // (the reference validates every function at init,
  // src/u15-metal-ops.cc:205-243).
  const bool ok = u15h::kernels_loadable();
  // The static scratch's address on this device, looked up once per
  // device while it is current.
  void* noalloc_ws = nullptr;
  const hipError_t noalloc_err = ok ? u15h::noalloc_scratch(device, &noalloc_ws)
                                    : hipErrorNotReady;
  if (prev >= 0 && prev != device) { (void)hipSetDevice(prev); }
  if (!ok) { return U15H_ENODEV; }
  u15h_ctx* ctx = new u15h_ctx;
  ctx->device = device;
  ctx->noalloc_ws = noalloc_ws;
  ctx->noalloc_err = noalloc_err;
  ctx->num_cu = prop.multiProcessorCount > 0 ? prop.multiProcessorCount : 256;
  ctx->split_on = env_int("U15H_SPLIT", 1) != 0;
  ctx->skinny_on = env_int("U15H_SKINNY", 1) != 0;
  ctx->prologue_rpt = env_int("U15H_PROLOGUE_RPT", 2);
  ctx->q_min_m = std::max(0, std::min(u15h::kSkinnyMaxRows + 1, env_int("U15H_Q_MIN_M", 96)));
  ctx->gemm.waves = env_int("U15H_WAVES", 8) == 4 ? 4 : 8;
  // env U15H_GEMM_CUS caps the tiled GEMM's persistent grid (a multiple of
  // 8, so each XCD keeps the same share), leaving CUs to work on another
  // stream; the split-K planner then fills rounds of that many tiles
  ctx->gemm_cus = std::max(8, std::min(ctx->num_cu,
                                       env_int("U15H_GEMM_CUS", ctx->num_cu) / 8 * 8));
  ctx->gemm.cus = env_int("U15H_PERSIST", 1) != 0 ? ctx->gemm_cus : 0;
  ctx->gemm.mfma16 = std::max(-1, std::min(1, env_int("U15H_MFMA16", 1)));
  ctx->i8_min_m = std::max(1, env_int("U15H_I8_MIN_M", 1024));
  *out = ctx;
  return U15H_OK;
}

void
u15h_destroy(u15h_ctx* ctx)
{
  if (ctx == nullptr) { return; }
  u15h_release_i8_scratch(ctx);
  if (ctx->w_deq != nullptr) {
    (void)hipDeviceSynchronize();
    (void)hipFree(ctx->w_deq);
  }
  if (ctx->split_ws != nullptr) {
    (void)hipDeviceSynchronize();
    (void)hipFree(ctx->split_ws);
  }
  delete ctx;
}

const char*
u15h_last_error(const u15h_ctx* ctx)
{
  return ctx != nullptr ? ctx->err.c_str() : "null context";
}

// The dense bf16 GEMM on checked, bound arguments.
static u15h_status
dense_bf16(u15h_ctx* ctx, hipStream_t s, const u15h_bf16* x,
           const u15h_bf16* w, const u15h_bf16* bias, u15h_bf16* y, int M,
           int K, int N)
{
  GemmBatch b = empty_batch(K * 2);
  add_problem(b, x, w, nullptr, y, bias, nullptr, nullptr, M, N, N,
              u15h::tile_cols(Epi::kBf16));
  if (skinny_fits(ctx, b)) {
    return skinny_launch(ctx, b, s, false, take_profile_event(ctx));
  }
  u15h_status st = plan_split(ctx, b);
  if (st != U15H_OK) { return st; }
  return launched(ctx, u15h::launch_gemm_bf16(b, Epi::kBf16, ctx->gemm, s, take_profile_event(ctx)), "gemm_bf16");
}

u15h_status
u15h_linear(u15h_ctx* ctx, u15h_stream stream, const u15h_bf16* x,
            const u15h_bf16* w, const u15h_bf16* bias, u15h_bf16* y, int M,
            int K, int N)
{
  if (ctx == nullptr) { return U15H_EINVAL; }
  if (M < 0) { return fail(ctx, U15H_EINVAL, "M=%d", M); }
  u15h_status st = check_k(ctx, K, 2, 8);
  if (st == U15H_OK) { st = check_n(ctx, N); }
  if (st == U15H_OK) { st = check_rows(ctx, M, 0); }
  if (st != U15H_OK) { return st; }
  if (M == 0) { ctx->err.clear(); return U15H_OK; }
  if (x == nullptr || w == nullptr || y == nullptr) {
    return fail(ctx, U15H_EINVAL, "null x/w/y");
  }
  if (!aligned16(x) || !aligned16(w) || !aligned16(y) ||
      (bias != nullptr && !aligned16(bias))) {
    return fail(ctx, U15H_EINVAL, "pointers must be 16-byte aligned");
  }
  if ((st = bind_device(ctx)) != U15H_OK) { return st; }
  hipStream_t s = as_stream(stream);
  // The int8 interception, as MetalOps::linear_mma_ does it
  // (src/u15-metal-ops.cc:291-306): taken only when the tier is on and the
  // shape qualifies; otherwise the bf16 path runs exactly as before.
  if (ctx->i8_on && M >= ctx->i8_min_m && K % 128 == 0) {
    return linear_i8_route(ctx, s, x, w, bias, y, M, K, N);
  }
  return dense_bf16(ctx, s, x, w, bias, y, M, K, N);
}

static u15h_status
mot_linear_impl(u15h_ctx* ctx, u15h_stream stream, const u15h_bf16* x,
                int M_und, int M_gen, int K, const u15h_mot_proj* proj,
                int nproj, bool noalloc)
{
  if (ctx == nullptr) { return U15H_EINVAL; }
  u15h_status st = check_k(ctx, K, 2, 8);
  if (st == U15H_OK) { st = check_rows(ctx, M_und, M_gen); }
  if (st != U15H_OK) { return st; }
  if (proj == nullptr || nproj < 1 || nproj > U15H_MAX_PROJ) {
    return fail(ctx, U15H_EINVAL, "nproj=%d must be in [1, %d]", nproj,
                U15H_MAX_PROJ);
  }
  if (M_und + M_gen > 0 && (x == nullptr || !aligned16(x))) {
    return fail(ctx, U15H_EINVAL, "x null or misaligned");
  }
  for (int i = 0; i < nproj; ++i) {
    const u15h_mot_proj& p = proj[i];
    if ((st = check_n(ctx, p.N)) != U15H_OK) { return st; }
    if (p.y == nullptr || !aligned16(p.y)) {
      return fail(ctx, U15H_EINVAL, "proj[%d].y null or misaligned", i);
    }
    if (M_und > 0 && (p.w_und == nullptr || !aligned16(p.w_und) ||
                      (p.bias_und != nullptr && !aligned16(p.bias_und)))) {
      return fail(ctx, U15H_EINVAL, "proj[%d] und weights", i);
    }
    if (M_gen > 0 && (p.w_gen == nullptr || !aligned16(p.w_gen) ||
                      (p.bias_gen != nullptr && !aligned16(p.bias_gen)))) {
      return fail(ctx, U15H_EINVAL, "proj[%d] gen weights", i);
    }
  }
  if (M_und + M_gen == 0) { ctx->err.clear(); return U15H_OK; }
  if ((st = bind_device(ctx)) != U15H_OK) { return st; }
  const int tc = u15h::tile_cols(Epi::kBf16);
  const size_t kb = (size_t)K * 2;
  GemmBatch b = empty_batch(K * 2);
  // Gen problems first: they are the bulk of the tiles; the small und
  // group fills in behind them.
  for (int i = 0; i < nproj; ++i) {
    const u15h_mot_proj& p = proj[i];
    add_problem(b, reinterpret_cast<const char*>(x) + (size_t)M_und * kb,
                p.w_gen, nullptr, p.y + (size_t)M_und * p.N, p.bias_gen,
                nullptr, nullptr, M_gen, p.N, p.N, tc);
  }
  for (int i = 0; i < nproj; ++i) {
    const u15h_mot_proj& p = proj[i];
    add_problem(b, x, p.w_und, nullptr, p.y, p.bias_und, nullptr, nullptr,
                M_und, p.N, p.N, tc);
  }
  if ((st = check_tiles(ctx, b)) != U15H_OK) { return st; }
  if (skinny_fits(ctx, b)) {
    return skinny_launch(ctx, b, as_stream(stream), noalloc, take_profile_event(ctx));
  }
  if ((st = plan_split(ctx, b, noalloc)) != U15H_OK) { return st; }
  return launched(ctx, u15h::launch_gemm_bf16(b, Epi::kBf16, ctx->gemm, as_stream(stream), take_profile_event(ctx)),
                  "mot_gemm_bf16");
}

u15h_status
u15h_mot_linear(u15h_ctx* ctx, u15h_stream stream, const u15h_bf16* x,
                int M_und, int M_gen, int K, const u15h_mot_proj* proj,
                int nproj)
{
  return mot_linear_impl(ctx, stream, x, M_und, M_gen, K, proj, nproj, false);
}

u15h_status
u15h_mot_linear_noalloc(u15h_ctx* ctx, u15h_stream stream, const u15h_bf16* x,
                        int M_und, int M_gen, int K, const u15h_mot_proj* proj,
                        int nproj)
{
  return mot_linear_impl(ctx, stream, x, M_und, M_gen, K, proj, nproj, true);
}

u15h_status
u15h_swiglu(u15h_ctx* ctx, u15h_stream stream, const u15h_bf16* gate,
            const u15h_bf16* up, u15h_bf16* out, int64_t n)
{
  if (ctx == nullptr) { return U15H_EINVAL; }
  if (n < 0 || n % 8 != 0) {
    return fail(ctx, U15H_EINVAL, "n=%lld must be a multiple of 8",
                (long long)n);
  }
  if (n == 0) { ctx->err.clear(); return U15H_OK; }
  if (gate == nullptr || up == nullptr || out == nullptr ||
      !aligned16(gate) || !aligned16(up) || !aligned16(out)) {
    return fail(ctx, U15H_EINVAL, "null or misaligned swiglu operand");
  }
  u15h_status st = bind_device(ctx);
  if (st != U15H_OK) { return st; }
  return launched(ctx, u15h::launch_swiglu(gate, up, out, n, as_stream(stream)),
                  "swiglu");
}

static u15h_status
rms_norm_call(u15h_ctx* ctx, u15h_stream stream, u15h_bf16* x,
              const u15h_bf16* d, int M_und, int M_gen, int dim,
              const u15h_bf16* w_und, const u15h_bf16* w_gen, float eps,
              u15h_bf16* y, int8_t* q, float* s, const char* what)
{
  if (ctx == nullptr) { return U15H_EINVAL; }
  if (M_und < 0 || M_gen < 0 || (long long)M_und + M_gen > (1 << 30) ||
      dim <= 0 || dim % 8 != 0 || dim > 16384) {
    return fail(ctx, U15H_EINVAL, "%s: rows=%d+%d dim=%d (dim %% 8 == 0, <= 16384)",
                what, M_und, M_gen, dim);
  }
  if (!(eps >= 0.0f)) {
    return fail(ctx, U15H_EINVAL, "%s: eps must be >= 0", what);
  }
  const int rows = M_und + M_gen;
  if (rows == 0) { ctx->err.clear(); return U15H_OK; }
  const bool quant = q != nullptr || s != nullptr;
  if (x == nullptr || !aligned16(x) ||
      (M_und > 0 && (w_und == nullptr || !aligned16(w_und))) ||
      (M_gen > 0 && (w_gen == nullptr || !aligned16(w_gen))) ||
      (d != nullptr && !aligned16(d)) || (y != nullptr && !aligned16(y)) ||
      (quant && (q == nullptr || s == nullptr || !aligned16(q) || !aligned16(s)))) {
    return fail(ctx, U15H_EINVAL, "%s: null or misaligned operand", what);
  }
  if (y == nullptr && !quant) {
    return fail(ctx, U15H_EINVAL, "%s: no output (y or the int8 codes)", what);
  }
  if (d != nullptr && y == x) {
    return fail(ctx, U15H_EINVAL, "%s: y must not be x when a residual is added "
                "(x keeps the sum)", what);
  }
  u15h_status st = bind_device(ctx);
  if (st != U15H_OK) { return st; }
  return launched(ctx,
                  u15h::launch_rms_norm(x, d, M_und > 0 ? w_und : w_gen,
                                        M_gen > 0 ? w_gen : w_und, M_und, rows,
                                        dim, eps, y, q, s, as_stream(stream)),
                  what);
}

u15h_status
u15h_rms_norm(u15h_ctx* ctx, u15h_stream stream, const u15h_bf16* x,
              const u15h_bf16* w, u15h_bf16* y, int rows, int dim, float eps)
{
  if (ctx != nullptr && y == nullptr && rows > 0) {
    return fail(ctx, U15H_EINVAL, "rms_norm: null output");
  }
  // x is only read without a residual
  return rms_norm_call(ctx, stream, const_cast<u15h_bf16*>(x), nullptr, rows, 0,
                       dim, w, w, eps, y, nullptr, nullptr, "rms_norm");
}

u15h_status
u15h_rms_norm_quant_i8(u15h_ctx* ctx, u15h_stream stream, const u15h_bf16* x,
                       const u15h_bf16* w, int rows, int dim, float eps,
                       u15h_bf16* y, int8_t* q, float* s)
{
  if (ctx != nullptr && rows > 0 && (q == nullptr || s == nullptr)) {
    return fail(ctx, U15H_EINVAL, "rms_norm_quant_i8: null codes or scales");
  }
  return rms_norm_call(ctx, stream, const_cast<u15h_bf16*>(x), nullptr, rows, 0,
                       dim, w, w, eps, y, q, s, "rms_norm_quant_i8");
}

u15h_status
u15h_mot_rms_norm(u15h_ctx* ctx, u15h_stream stream, u15h_bf16* x,
                  const u15h_bf16* delta, int M_und, int M_gen, int dim,
                  const u15h_bf16* w_und, const u15h_bf16* w_gen, float eps,
                  u15h_bf16* y, int8_t* q, float* s)
{
  if (ctx != nullptr && (q == nullptr) != (s == nullptr)) {
    return fail(ctx, U15H_EINVAL, "mot_rms_norm: codes and scales go together");
  }
  return rms_norm_call(ctx, stream, x, delta, M_und, M_gen, dim, w_und, w_gen,
                       eps, y, q, s, "mot_rms_norm");
}

u15h_status
u15h_add(u15h_ctx* ctx, u15h_stream stream, u15h_bf16* dst,
         const u15h_bf16* src, int64_t n)
{
  if (ctx == nullptr) { return U15H_EINVAL; }
  if (n < 0) { return fail(ctx, U15H_EINVAL, "add: n=%lld", (long long)n); }
  if (n == 0) { ctx->err.clear(); return U15H_OK; }
  if (dst == nullptr || src == nullptr) {
    return fail(ctx, U15H_EINVAL, "add: null operand");
  }
  u15h_status st = bind_device(ctx);
  if (st != U15H_OK) { return st; }
  return launched(ctx, u15h::launch_add_bf16(dst, src, n, as_stream(stream)), "add");
}

u15h_status
u15h_swiglu_quant_i8(u15h_ctx* ctx, u15h_stream stream, const u15h_bf16* gate,
                     const u15h_bf16* up, int rows, int inter, u15h_bf16* h,
                     int8_t* q, float* s)
{
  if (ctx == nullptr) { return U15H_EINVAL; }
  if (rows < 0 || inter <= 0 || inter % 8 != 0 || inter > 16384) {
    return fail(ctx, U15H_EINVAL, "swiglu_quant_i8: rows=%d inter=%d (inter %% 8 "
                "== 0, <= 16384)", rows, inter);
  }
  if (rows == 0) { ctx->err.clear(); return U15H_OK; }
  if (gate == nullptr || up == nullptr || q == nullptr || s == nullptr ||
      !aligned16(gate) || !aligned16(up) || !aligned16(q) || !aligned16(s) ||
      (h != nullptr && !aligned16(h))) {
    return fail(ctx, U15H_EINVAL, "swiglu_quant_i8: null or misaligned operand");
  }
  u15h_status st = bind_device(ctx);
  if (st != U15H_OK) { return st; }
  return launched(ctx,
                  u15h::launch_swiglu_quant(gate, up, rows, inter, h, q, s,
                                            as_stream(stream)),
                  "swiglu_quant_i8");
}

u15h_status
u15h_mot_gate_up_swiglu(u15h_ctx* ctx, u15h_stream stream,
                        const u15h_bf16* x, int M_und, int M_gen, int K,
                        const u15h_bf16* wg_und, const u15h_bf16* wu_und,
                        const u15h_bf16* wg_gen, const u15h_bf16* wu_gen,
                        u15h_bf16* h, int I)
{
  if (ctx == nullptr) { return U15H_EINVAL; }
  u15h_status st = check_k(ctx, K, 2, 8);
  if (st == U15H_OK) { st = check_rows(ctx, M_und, M_gen); }
  if (st == U15H_OK) { st = check_n(ctx, I); }
  if (st != U15H_OK) { return st; }
  if (M_und + M_gen == 0) { ctx->err.clear(); return U15H_OK; }
  if (x == nullptr || h == nullptr || !aligned16(x) || !aligned16(h)) {
    return fail(ctx, U15H_EINVAL, "x/h null or misaligned");
  }
  if (M_und > 0 && (wg_und == nullptr || wu_und == nullptr ||
                    !aligned16(wg_und) || !aligned16(wu_und))) {
    return fail(ctx, U15H_EINVAL, "und gate/up weights");
  }
  if (M_gen > 0 && (wg_gen == nullptr || wu_gen == nullptr ||
                    !aligned16(wg_gen) || !aligned16(wu_gen))) {
    return fail(ctx, U15H_EINVAL, "gen gate/up weights");
  }
  if ((st = bind_device(ctx)) != U15H_OK) { return st; }
  const int tc = u15h::tile_cols(Epi::kSwiglu);
  const size_t kb = (size_t)K * 2;
  GemmBatch b = empty_batch(K * 2);
  add_problem(b, reinterpret_cast<const char*>(x) + (size_t)M_und * kb,
              wg_gen, wu_gen, h + (size_t)M_und * I, nullptr, nullptr,
              nullptr, M_gen, I, I, tc);
  add_problem(b, x, wg_und, wu_und, h, nullptr, nullptr, nullptr, M_und, I, I,
              tc);
  if ((st = check_tiles(ctx, b)) != U15H_OK) { return st; }
  if ((st = plan_split(ctx, b)) != U15H_OK) { return st; }
  return launched(ctx, u15h::launch_gemm_bf16(b, Epi::kSwiglu, ctx->gemm, as_stream(stream), take_profile_event(ctx)),
                  "mot_gate_up_swiglu");
}

int
u15h_enable_i8_gemm(u15h_ctx* ctx, int want)
{
  if (ctx == nullptr) { return 0; }
  // U15H_I8_GEMM overrides `want` either way, which is how an A/B is run
  // without touching the caller (src/u15-metal-ops.h:85-92).
  const char* e = std::getenv("U15H_I8_GEMM");
  bool on = want != 0;
  if (e != nullptr && *e != '\0') { on = std::atoi(e) != 0; }
  ctx->i8_on = on;
  if (!on) { u15h_release_i8_scratch(ctx); }
  return ctx->i8_on ? 1 : 0;
}

void
u15h_release_i8_scratch(u15h_ctx* ctx)
{
  if (ctx == nullptr || ctx->i8_scratch == nullptr) { return; }
  // Queued work may still read it.
  (void)hipDeviceSynchronize();
  (void)hipFree(ctx->i8_scratch);
  ctx->i8_scratch = nullptr;
  ctx->i8_scratch_bytes = 0;
}

u15h_status
u15h_profile_next_gemm(u15h_ctx* ctx, void* event)
{
  return u15h_profile_bracket_next_gemm(ctx, nullptr, event);
}

u15h_status
u15h_profile_bracket_next_gemm(u15h_ctx* ctx, void* before, void* after)
{
  return u15h_profile_next_kernels(ctx, nullptr, nullptr, before, after,
                                   nullptr, nullptr);
}

u15h_status
u15h_profile_next_kernels(u15h_ctx* ctx, void* quant_start, void* quant_end,
                          void* gemm_start, void* gemm_end, void* reduce_start,
                          void* reduce_end)
{
  if (ctx == nullptr) { return U15H_EINVAL; }
  ctx->prof_quant[0] = static_cast<hipEvent_t>(quant_start);
  ctx->prof_quant[1] = static_cast<hipEvent_t>(quant_end);
  ctx->prof_gemm.before = static_cast<hipEvent_t>(gemm_start);
  ctx->prof_gemm.after = static_cast<hipEvent_t>(gemm_end);
  ctx->prof_gemm.red_before = static_cast<hipEvent_t>(reduce_start);
  ctx->prof_gemm.red_after = static_cast<hipEvent_t>(reduce_end);
  return U15H_OK;
}

int
u15h_i8_min_m(const u15h_ctx* ctx)
{
  return ctx != nullptr ? ctx->i8_min_m : 0;
}

u15h_status
u15h_quant_rows_i8(u15h_ctx* ctx, u15h_stream stream, const u15h_bf16* x,
                   int rows, int K, int8_t* q, float* s)
{
  if (ctx == nullptr) { return U15H_EINVAL; }
  if (rows < 0 || K <= 0 || K % 8 != 0) {
    return fail(ctx, U15H_EINVAL, "rows=%d K=%d (K must be a multiple of 8)",
                rows, K);
  }
  if (rows == 0) { ctx->err.clear(); return U15H_OK; }
  if (x == nullptr || q == nullptr || s == nullptr || !aligned16(x) ||
      !aligned16(q) || !aligned16(s)) {
    return fail(ctx, U15H_EINVAL, "null or misaligned quant operand");
  }
  u15h_status st = bind_device(ctx);
  if (st != U15H_OK) { return st; }
  hipEvent_t e0 = nullptr, e1 = nullptr;
  take_quant_events(ctx, &e0, &e1);
  return launched(
      ctx, u15h::launch_quant_rows_i8(x, rows, K, q, s, as_stream(stream), e0, e1),
      "quant_rows_i8");
}

static u15h_status
mot_gemm_i8_common(u15h_ctx* ctx, u15h_stream stream, const int8_t* xq,
                   const float* sx, int M_und, int M_gen, int K,
                   const u15h_mot_proj_i8* proj, int nproj, Epi epi)
{
  if (ctx == nullptr) { return U15H_EINVAL; }
  u15h_status st = check_k(ctx, K, 1, 128);
  if (st == U15H_OK && K > 131072) {
    st = fail(ctx, U15H_EINVAL, "K=%d: int32 accumulation is exact only "
                                "up to K=131072", K);
  }
  if (st == U15H_OK) { st = check_rows(ctx, M_und, M_gen); }
  if (st != U15H_OK) { return st; }
  if (proj == nullptr || nproj < 1 || nproj > U15H_MAX_PROJ) {
    return fail(ctx, U15H_EINVAL, "nproj=%d must be in [1, %d]", nproj,
                U15H_MAX_PROJ);
  }
  const bool deq = epi == Epi::kDequantBf16;
  if (M_und + M_gen > 0 &&
      (xq == nullptr || !aligned16(xq) || (deq && (sx == nullptr)))) {
    return fail(ctx, U15H_EINVAL, "xq/sx null or misaligned");
  }
  for (int i = 0; i < nproj; ++i) {
    const u15h_mot_proj_i8& p = proj[i];
    if ((st = check_n(ctx, p.N)) != U15H_OK) { return st; }
    if (p.y == nullptr || !aligned16(p.y)) {
      return fail(ctx, U15H_EINVAL, "proj[%d].y null or misaligned", i);
    }
    if (M_und > 0 && (p.wq_und == nullptr || !aligned16(p.wq_und) ||
                      (deq && (p.sw_und == nullptr || !aligned16(p.sw_und))))) {
      return fail(ctx, U15H_EINVAL, "proj[%d] und weights/scales", i);
    }
    if (M_gen > 0 && (p.wq_gen == nullptr || !aligned16(p.wq_gen) ||
                      (deq && (p.sw_gen == nullptr || !aligned16(p.sw_gen))))) {
      return fail(ctx, U15H_EINVAL, "proj[%d] gen weights/scales", i);
    }
  }
  if (M_und + M_gen == 0) { ctx->err.clear(); return U15H_OK; }
  if ((st = bind_device(ctx)) != U15H_OK) { return st; }
  const int tc = u15h::tile_cols(epi);
  const size_t esz = deq ? 2 : 4;
  GemmBatch b = empty_batch(K);
  for (int i = 0; i < nproj; ++i) {
    const u15h_mot_proj_i8& p = proj[i];
    add_problem(b, xq + (size_t)M_und * K, p.wq_gen, nullptr,
                static_cast<char*>(p.y) + (size_t)M_und * p.N * esz, nullptr,
                deq ? sx + M_und : nullptr, deq ? p.sw_gen : nullptr, M_gen,
                p.N, p.N, tc);
  }
  for (int i = 0; i < nproj; ++i) {
    const u15h_mot_proj_i8& p = proj[i];
    add_problem(b, xq, p.wq_und, nullptr, p.y, nullptr, deq ? sx : nullptr,
                deq ? p.sw_und : nullptr, M_und, p.N, p.N, tc);
  }
  if ((st = check_tiles(ctx, b)) != U15H_OK) { return st; }
  if ((st = plan_split(ctx, b)) != U15H_OK) { return st; }
  return launched(ctx, u15h::launch_gemm_i8(b, epi, ctx->gemm, as_stream(stream), take_profile_event(ctx)),
                  deq ? "mot_gemm_i8" : "mot_gemm_i8_i32");
}

u15h_status
u15h_mot_gemm_i8_i32(u15h_ctx* ctx, u15h_stream stream, const int8_t* xq,
                     int M_und, int M_gen, int K,
                     const u15h_mot_proj_i8* proj, int nproj)
{
  return mot_gemm_i8_common(ctx, stream, xq, nullptr, M_und, M_gen, K, proj,
                            nproj, Epi::kI32);
}

u15h_status
u15h_mot_gemm_i8(u15h_ctx* ctx, u15h_stream stream, const int8_t* xq,
                 const float* sx, int M_und, int M_gen, int K,
                 const u15h_mot_proj_i8* proj, int nproj)
{
  return mot_gemm_i8_common(ctx, stream, xq, sx, M_und, M_gen, K, proj, nproj,
                            Epi::kDequantBf16);
}

// The grow-only bf16 expansion of an affine pack (the reference's _w_deq,
// u15-metal-ops.h:461-469).  Growing waits for the stream, since the old
// buffer may still be read by work queued on it.
static u15h_status
ensure_deq_scratch(u15h_ctx* ctx, u15h_stream stream, size_t need)
{
  if (ctx->w_deq_bytes >= need) { return U15H_OK; }
  if (ctx->w_deq != nullptr) {
    (void)hipStreamSynchronize(as_stream(stream));
    (void)hipFree(ctx->w_deq);
    ctx->w_deq = nullptr;
    ctx->w_deq_bytes = 0;
  }
  u15h_status st = bind_device(ctx);
  if (st != U15H_OK) { return st; }
  if (hipMalloc(&ctx->w_deq, need) != hipSuccess) {
    ctx->w_deq = nullptr;
    return fail(ctx, U15H_ENOMEM, "dequant scratch of %zu bytes", need);
  }
  ctx->w_deq_bytes = need;
  return U15H_OK;
}

static u15h_status
check_qweight(u15h_ctx* ctx, const u15h_qweight* w, int N, int K)
{
  if (w == nullptr || w->codes == nullptr || w->scales == nullptr ||
      w->biases == nullptr) {
    return fail(ctx, U15H_EINVAL, "null quantized weight pack");
  }
  if ((w->bits != 4 && w->bits != 8) || (w->group != 32 && w->group != 64)) {
    return fail(ctx, U15H_EINVAL, "pack w%dg%d: bits must be 4 or 8, group "
                "32 or 64", w->bits, w->group);
  }
  if (N <= 0 || K <= 0 || K % w->group != 0 || K % 8 != 0) {
    return fail(ctx, U15H_EINVAL, "N=%d K=%d do not close with group %d", N,
                K, w->group);
  }
  if ((long long)N * K > (1LL << 31)) {
    return fail(ctx, U15H_EINVAL, "pack too large");
  }
  if (!aligned16(w->codes)) {
    return fail(ctx, U15H_EINVAL, "codes must be 16-byte aligned");
  }
  return U15H_OK;
}

u15h_status
u15h_dequant_affine(u15h_ctx* ctx, u15h_stream stream, const u15h_qweight* w,
                    int N, int K, u15h_bf16* w_out)
{
  if (ctx == nullptr) { return U15H_EINVAL; }
  u15h_status st = check_qweight(ctx, w, N, K);
  if (st != U15H_OK) { return st; }
  if (w_out == nullptr || !aligned16(w_out)) {
    return fail(ctx, U15H_EINVAL, "w_out null or misaligned");
  }
  if ((st = bind_device(ctx)) != U15H_OK) { return st; }
  return launched(ctx,
                  u15h::launch_dequant_affine(w->codes, w->scales, w->biases,
                                              w->bits, w->group, N, K, w_out,
                                              as_stream(stream)),
                  "dequant_affine");
}

u15h_status
u15h_linear_q(u15h_ctx* ctx, u15h_stream stream, const u15h_bf16* x,
              const u15h_qweight* w, const u15h_bf16* bias, u15h_bf16* y,
              int M, int K, int N)
{
  if (ctx == nullptr) { return U15H_EINVAL; }
  u15h_status st = check_qweight(ctx, w, N, K);
  if (st == U15H_OK) { st = check_n(ctx, N); }
  if (st == U15H_OK) { st = check_k(ctx, K, 2, 8); }
  if (st == U15H_OK) { st = check_rows(ctx, M, 0); }
  if (st != U15H_OK) { return st; }
  if (M == 0) { ctx->err.clear(); return U15H_OK; }
  if (x == nullptr || y == nullptr || !aligned16(x) || !aligned16(y) ||
      (bias != nullptr && !aligned16(bias))) {
    return fail(ctx, U15H_EINVAL, "x/y null, or x/y/bias misaligned");
  }
  if ((st = bind_device(ctx)) != U15H_OK) { return st; }
  // Below the row floor the pack is read directly, as the reference's
  // steel qmm does (u15-metal-ops.cc:402-431): the skinny kernel
  // dequantises each weight in registers to exactly the expansion's bf16
  // value, so the product equals u15h_linear on the expansion bit for bit.
  if (M < ctx->q_min_m) {
    GemmBatch b = empty_batch(K * 2);
    add_problem(b, x, w->codes, nullptr, y, bias, nullptr, nullptr, M, N, N,
                u15h::tile_cols(Epi::kBf16));
    if (skinny_fits(ctx, b)) {
      return skinny_launch(ctx, b, as_stream(stream), false, take_profile_event(ctx), w);
    }
  }
  if ((st = ensure_deq_scratch(ctx, stream, (size_t)N * K * 2)) != U15H_OK) {
    return st;
  }
  u15h_bf16* wd = static_cast<u15h_bf16*>(ctx->w_deq);
  if ((st = u15h_dequant_affine(ctx, stream, w, N, K, wd)) != U15H_OK) {
    return st;
  }
  // From here the expansion is a dense weight and takes u15h_linear's
  // route: the reference's linear_mma_q_ re-enters linear_mma_, whose
  // first step is the int8 interception (u15-metal-ops.cc:291-300,
  // 393-399: a quantized weight arrives there as the _w_deq expansion).
  hipStream_t s = as_stream(stream);
  if (ctx->i8_on && M >= ctx->i8_min_m && K % 128 == 0) {
    return linear_i8_route(ctx, s, x, wd, bias, y, M, K, N);
  }
  return dense_bf16(ctx, s, x, wd, bias, y, M, K, N);
}

u15h_status
u15h_swiglu_fused(u15h_ctx* ctx, u15h_stream stream, const u15h_bf16* x,
                  const u15h_bf16* w_fused, u15h_bf16* y, int M, int K,
                  int inter)
{
  if (ctx == nullptr) { return U15H_EINVAL; }
  // Weight rows are 2K apart here, so K is held to half the plain limit.
  u15h_status st = check_k(ctx, K, 4, 8);
  if (st == U15H_OK) { st = check_n(ctx, inter); }
  if (st == U15H_OK) { st = check_rows(ctx, M, 0); }
  if (st != U15H_OK) { return st; }
  if (M == 0) { ctx->err.clear(); return U15H_OK; }
  if (x == nullptr || w_fused == nullptr || y == nullptr || !aligned16(x) ||
      !aligned16(w_fused) || !aligned16(y)) {
    return fail(ctx, U15H_EINVAL, "null or misaligned swiglu_fused operand");
  }
  if ((st = bind_device(ctx)) != U15H_OK) { return st; }
  // Row 2i of w_fused is gate row i and row 2i+1 up row i: two [inter][K]
  // weights 2K bytes apart per row, the second starting one row in.
  const size_t kb = (size_t)K * 2;
  GemmBatch b = empty_batch(K * 2);
  add_problem(b, x, w_fused, reinterpret_cast<const char*>(w_fused) + kb, y,
              nullptr, nullptr, nullptr, M, inter, inter,
              u15h::tile_cols(Epi::kSwiglu), (int)(2 * kb));
  if ((st = check_tiles(ctx, b)) != U15H_OK) { return st; }
  if ((st = plan_split(ctx, b)) != U15H_OK) { return st; }
  return launched(ctx,
                  u15h::launch_gemm_bf16(b, Epi::kSwiglu, ctx->gemm,
                                         as_stream(stream),
                                         take_profile_event(ctx)),
                  "swiglu_fused");
}

u15h_status
u15h_bias_add(u15h_ctx* ctx, u15h_stream stream, u15h_bf16* y,
              const u15h_bf16* bias, int M, int N)
{
  if (ctx == nullptr) { return U15H_EINVAL; }
  if (M < 0 || N <= 0 || N % 8 != 0) {
    return fail(ctx, U15H_EINVAL, "M=%d N=%d (N must be a multiple of 8)", M,
                N);
  }
  if (M == 0) { ctx->err.clear(); return U15H_OK; }
  if (y == nullptr || bias == nullptr || !aligned16(y) || !aligned16(bias)) {
    return fail(ctx, U15H_EINVAL, "y/bias null or misaligned");
  }
  u15h_status st = bind_device(ctx);
  if (st != U15H_OK) { return st; }
  return launched(ctx, u15h::launch_bias_add(y, bias, M, N, as_stream(stream)),
                  "bias_add");
}

u15h_status
u15h_f32_to_bf16(u15h_ctx* ctx, u15h_stream stream, const float* src,
                 int64_t n, u15h_bf16* dst)
{
  if (ctx == nullptr) { return U15H_EINVAL; }
  if (n < 0 || n % 4 != 0) {
    return fail(ctx, U15H_EINVAL, "n=%lld must be a multiple of 4",
                (long long)n);
  }
  if (n == 0) { ctx->err.clear(); return U15H_OK; }
  if (src == nullptr || dst == nullptr || !aligned16(src) || !aligned16(dst)) {
    return fail(ctx, U15H_EINVAL, "src/dst null or misaligned");
  }
  u15h_status st = bind_device(ctx);
  if (st != U15H_OK) { return st; }
  return launched(ctx,
                  u15h::launch_f32_to_bf16(src, n, dst, as_stream(stream)),
                  "f32_to_bf16");
}

u15h_status
u15h_f16_to_bf16(u15h_ctx* ctx, u15h_stream stream, const uint16_t* src,
                 int64_t n, u15h_bf16* dst)
{
  if (ctx == nullptr) { return U15H_EINVAL; }
  if (n < 0 || n % 4 != 0) {
    return fail(ctx, U15H_EINVAL, "n=%lld must be a multiple of 4",
                (long long)n);
  }
  if (n == 0) { ctx->err.clear(); return U15H_OK; }
  if (src == nullptr || dst == nullptr || reinterpret_cast<uintptr_t>(src) % 8 ||
      reinterpret_cast<uintptr_t>(dst) % 8) {
    return fail(ctx, U15H_EINVAL, "src/dst null or not 8-byte aligned");
  }
  u15h_status st = bind_device(ctx);
  if (st != U15H_OK) { return st; }
  return launched(ctx, u15h::launch_f16_to_bf16(src, n, dst, as_stream(stream)),
                  "f16_to_bf16");
}

u15h_status
u15h_qweight_geometry(int K, int64_t scales_cols, int64_t codes_cols,
                      int* bits, int* group)
{
  // group = K / scales_cols and bits = codes_cols * 32 / K, accepted only
  // when both close exactly on w4/w8, g32/g64.
  if (bits == nullptr || group == nullptr || K <= 0 || scales_cols <= 0 ||
      codes_cols <= 0) {
    return U15H_EINVAL;
  }
  const int64_t g = (int64_t)K / scales_cols;
  const int64_t b = codes_cols * 32 / (int64_t)K;
  if ((g != 32 && g != 64) || (b != 4 && b != 8) || scales_cols * g != K ||
      codes_cols * 32 != (int64_t)K * b) {
    return U15H_EINVAL;
  }
  *bits = (int)b;
  *group = (int)g;
  return U15H_OK;
}

u15h_status
u15h_repack_affine_i8(u15h_ctx* ctx, u15h_stream stream,
                      const u15h_qweight* w, int N, int K, int8_t* wq,
                      float* sw)
{
  if (ctx == nullptr) { return U15H_EINVAL; }
  u15h_status st = check_qweight(ctx, w, N, K);
  if (st != U15H_OK) { return st; }
  if (wq == nullptr || sw == nullptr || !aligned16(wq) ||
      reinterpret_cast<uintptr_t>(sw) % 4) {
    return fail(ctx, U15H_EINVAL, "wq/sw null or misaligned");
  }
  if ((st = ensure_deq_scratch(ctx, stream, (size_t)N * K * 2)) != U15H_OK) {
    return st;
  }
  u15h_bf16* wd = static_cast<u15h_bf16*>(ctx->w_deq);
  if ((st = u15h_dequant_affine(ctx, stream, w, N, K, wd)) != U15H_OK) {
    return st;
  }
  return launched(ctx,
                  u15h::launch_quant_rows_i8(wd, N, K, wq, sw,
                                             as_stream(stream)),
                  "repack_affine_i8");
}

static u15h_status
attention_call(u15h_ctx* ctx, u15h_stream stream, const u15h_bf16* q,
               const u15h_bf16* k, const u15h_bf16* v, u15h_bf16* out,
               const int32_t* t_index, int hq, int hkv, int tq, int tk, int d,
               int cap, int q_offset, int mode, bool token_major,
               const char* what)
{
  if (ctx == nullptr) { return U15H_EINVAL; }
  if (hq <= 0 || hkv <= 0 || hq % hkv != 0 || tq < 0 || tk < 0 || cap < tk ||
      q_offset < 0 || (d != 32 && d != 64 && d != 128)) {
    return fail(ctx, U15H_EINVAL, "%s: hq=%d hkv=%d tq=%d tk=%d d=%d cap=%d "
                "q_offset=%d (hq %% hkv == 0, tk <= cap, d in {32, 64, 128})",
                what, hq, hkv, tq, tk, d, cap, q_offset);
  }
  // one kv head's keys are read through a buffer resource: 2^31 bytes at most
  if ((long long)hkv * cap * d > (1LL << 40) || (long long)hq * tq * d > (1LL << 40) ||
      (long long)tk * d * 2 >= (1LL << 31)) {
    return fail(ctx, U15H_EINVAL, "%s: operands too large", what);
  }
  if (tq == 0) { ctx->err.clear(); return U15H_OK; }
  if (q == nullptr || out == nullptr || (tk > 0 && (k == nullptr || v == nullptr)) ||
      (mode == 2 && t_index == nullptr)) {
    return fail(ctx, U15H_EINVAL, "%s: null operand", what);
  }
  if (!aligned16(q) || !aligned16(out) || !aligned16(k) || !aligned16(v)) {
    return fail(ctx, U15H_EINVAL, "%s: pointers must be 16-byte aligned", what);
  }
  u15h_status st = bind_device(ctx);
  if (st != U15H_OK) { return st; }
  u15h::AttnArgs a;
  a.q = q;
  a.k = k;
  a.v = v;
  a.out = out;
  a.t_index = t_index;
  a.q_head = token_major ? d : (long long)tq * d;
  a.q_tok = token_major ? (long long)hq * d : d;
  a.o_head = a.q_head;
  a.o_tok = a.q_tok;
  a.hq = hq;
  a.hkv = hkv;
  a.tq = tq;
  a.tk = tk;
  a.cap = cap;
  a.q_offset = q_offset;
  a.d = d;
  a.mode = mode;
  return launched(ctx, u15h::launch_attention(a, as_stream(stream)), what);
}

u15h_status
u15h_sdpa(u15h_ctx* ctx, u15h_stream stream, const u15h_bf16* q,
          const u15h_bf16* k, const u15h_bf16* v, u15h_bf16* out, int hq,
          int hkv, int tq, int tk, int d, int cap, int causal, int q_offset)
{
  return attention_call(ctx, stream, q, k, v, out, nullptr, hq, hkv, tq, tk, d,
                        cap, q_offset, causal ? 1 : 0, false, "sdpa");
}

u15h_status
u15h_sdpa_block_causal(u15h_ctx* ctx, u15h_stream stream, const u15h_bf16* q,
                       const u15h_bf16* k, const u15h_bf16* v, u15h_bf16* out,
                       const int32_t* t_index, int hq, int hkv, int tq,
                       int tk, int d, int cap, int q_offset)
{
  return attention_call(ctx, stream, q, k, v, out, t_index, hq, hkv, tq, tk, d,
                        cap, q_offset, 2, false, "sdpa_block_causal");
}

u15h_status
u15h_attention_token_major(u15h_ctx* ctx, u15h_stream stream,
                           const u15h_bf16* q, const u15h_bf16* k,
                           const u15h_bf16* v, u15h_bf16* out,
                           const int32_t* t_index, int hq, int hkv, int tq,
                           int tk, int d, int cap, int q_offset, int mode)
{
  if (mode < 0 || mode > 2) {
    if (ctx != nullptr) { return fail(ctx, U15H_EINVAL, "mode=%d", mode); }
    return U15H_EINVAL;
  }
  return attention_call(ctx, stream, q, k, v, out, t_index, hq, hkv, tq, tk, d,
                        cap, q_offset, mode, true, "attention_token_major");
}

static u15h_status
transpose_call(u15h_ctx* ctx, u15h_stream stream, const u15h_bf16* in,
               u15h_bf16* out, int T, int H, int D, long long src_t,
               long long src_h, long long dst_t, long long dst_h,
               const char* what)
{
  if (ctx == nullptr) { return U15H_EINVAL; }
  if (T < 0 || H <= 0 || D <= 0 || D % 8 != 0) {
    return fail(ctx, U15H_EINVAL, "%s: T=%d H=%d D=%d (D %% 8 == 0)", what, T,
                H, D);
  }
  if (T == 0) { ctx->err.clear(); return U15H_OK; }
  if (in == nullptr || out == nullptr || !aligned16(in) || !aligned16(out)) {
    return fail(ctx, U15H_EINVAL, "%s: null or misaligned", what);
  }
  u15h_status st = bind_device(ctx);
  if (st != U15H_OK) { return st; }
  return launched(ctx,
                  u15h::launch_transpose_rows(in, out, T, H, D, src_t, src_h,
                                              dst_t, dst_h, as_stream(stream)),
                  what);
}

u15h_status
u15h_transpose_thd(u15h_ctx* ctx, u15h_stream stream, const u15h_bf16* in,
                   u15h_bf16* out, int T, int H, int D)
{
  return transpose_call(ctx, stream, in, out, T, H, D, (long long)H * D, D, D,
                        (long long)T * D, "transpose_thd");
}

u15h_status
u15h_transpose_htd(u15h_ctx* ctx, u15h_stream stream, const u15h_bf16* in,
                   u15h_bf16* out, int T, int H, int D)
{
  return transpose_call(ctx, stream, in, out, T, H, D, D, (long long)T * D,
                        (long long)H * D, D, "transpose_htd");
}

u15h_status
u15h_transpose_into_cache(u15h_ctx* ctx, u15h_stream stream,
                          const u15h_bf16* in, u15h_bf16* cache, int T, int H,
                          int D, int cap, int offset)
{
  if (ctx == nullptr) { return U15H_EINVAL; }
  if (offset < 0 || cap <= 0 || (long long)offset + T > cap) {
    return fail(ctx, U15H_EINVAL, "transpose_into_cache: offset %d + T %d "
                "exceeds capacity %d", offset, T, cap);
  }
  return transpose_call(ctx, stream, in,
                        cache == nullptr ? nullptr : cache + (size_t)offset * D,
                        T, H, D, (long long)H * D, D, D,
                        (long long)cap * D, "transpose_into_cache");
}

static u15h_status
check_head(u15h_ctx* ctx, int heads, int tokens, int head_dim, int d_t,
           int d_h)
{
  if (heads <= 0 || tokens < 0 || head_dim <= 0 || head_dim % 2 != 0 ||
      head_dim > 512) {
    return fail(ctx, U15H_EINVAL, "heads=%d tokens=%d head_dim=%d", heads,
                tokens, head_dim);
  }
  if (d_t <= 0 || d_h <= 0 || d_t % 2 != 0 || d_h % 2 != 0 ||
      d_t + 2 * d_h != head_dim) {
    return fail(ctx, U15H_EINVAL, "ranges d_t=%d d_h=%d do not split %d as "
                "[t | h | w] with even widths", d_t, d_h, head_dim);
  }
  if ((long long)heads * tokens > (1LL << 30)) {
    return fail(ctx, U15H_EINVAL, "heads x tokens too large");
  }
  return U15H_OK;
}

static u15h_status
norm_rope(u15h_ctx* ctx, u15h_stream stream, u15h_bf16* x,
          const u15h_bf16* w_t, const u15h_bf16* w_hw, const float* cosf,
          const float* sinf, int heads, int tokens, int head_dim, int d_t,
          int d_h, float eps, bool norm, bool rope, const char* what)
{
  if (ctx == nullptr) { return U15H_EINVAL; }
  u15h_status st = check_head(ctx, heads, tokens, head_dim, d_t, d_h);
  if (st != U15H_OK) { return st; }
  if (tokens == 0) { ctx->err.clear(); return U15H_OK; }
  if (x == nullptr || (norm && (w_t == nullptr || w_hw == nullptr)) ||
      (rope && (cosf == nullptr || sinf == nullptr))) {
    return fail(ctx, U15H_EINVAL, "%s: null operand", what);
  }
  if (norm && !(eps >= 0.0f)) {
    return fail(ctx, U15H_EINVAL, "%s: eps must be >= 0", what);
  }
  if ((st = bind_device(ctx)) != U15H_OK) { return st; }
  return launched(ctx,
                  u15h::launch_split_norm_rope(x, w_t, w_hw, cosf, sinf,
                                               heads * tokens, heads, head_dim,
                                               d_t, d_h, eps, norm, rope,
                                               as_stream(stream)),
                  what);
}

u15h_status
u15h_split_qk_norm(u15h_ctx* ctx, u15h_stream stream, u15h_bf16* x,
                   const u15h_bf16* w_t, const u15h_bf16* w_hw, int heads,
                   int tokens, int head_dim, float eps)
{
  return norm_rope(ctx, stream, x, w_t, w_hw, nullptr, nullptr, heads, tokens,
                   head_dim, head_dim / 2, head_dim / 4, eps, true, false,
                   "split_qk_norm");
}

u15h_status
u15h_split_rope(u15h_ctx* ctx, u15h_stream stream, u15h_bf16* x,
                const float* cos_tab, const float* sin_tab, int heads,
                int tokens, int head_dim, int d_t, int d_h)
{
  return norm_rope(ctx, stream, x, nullptr, nullptr, cos_tab, sin_tab, heads,
                   tokens, head_dim, d_t, d_h, 0.0f, false, true,
                   "split_rope");
}

u15h_status
u15h_split_qk_norm_rope(u15h_ctx* ctx, u15h_stream stream, u15h_bf16* x,
                        const u15h_bf16* w_t, const u15h_bf16* w_hw,
                        const float* cos_tab, const float* sin_tab, int heads,
                        int tokens, int head_dim, int d_t, int d_h, float eps)
{
  return norm_rope(ctx, stream, x, w_t, w_hw, cos_tab, sin_tab, heads, tokens,
                   head_dim, d_t, d_h, eps, true, true, "split_qk_norm_rope");
}

u15h_status
u15h_mot_attention_prologue(u15h_ctx* ctx, u15h_stream stream, u15h_bf16* q,
                            const u15h_bf16* k, const u15h_bf16* v,
                            const u15h_qk_norm* und, const u15h_qk_norm* gen,
                            const float* cos_tab, const float* sin_tab,
                            int M_und, int M_gen, int hq, int hkv,
                            int head_dim, int d_t, int d_h, float eps,
                            u15h_bf16* k_cache, u15h_bf16* v_cache, int cap,
                            int offset)
{
  if (ctx == nullptr) { return U15H_EINVAL; }
  const char* what = "mot_attention_prologue";
  if (M_und < 0 || M_gen < 0 || (long long)M_und + M_gen > (1 << 30)) {
    return fail(ctx, U15H_EINVAL, "%s: M_und=%d M_gen=%d", what, M_und, M_gen);
  }
  const int T = M_und + M_gen;
  u15h_status st = check_head(ctx, hq, T, head_dim, d_t, d_h);
  if (st != U15H_OK) { return st; }
  if ((st = check_head(ctx, hkv, T, head_dim, d_t, d_h)) != U15H_OK) { return st; }
  auto pow2 = [](int x) { return x > 0 && (x & (x - 1)) == 0; };
  if (!pow2(head_dim) || head_dim < 16 || d_t % 16 != 0 || d_h % 16 != 0 ||
      !pow2(d_t / 16) || !pow2(d_h / 16) || d_t % d_h != 0) {
    return fail(ctx, U15H_EINVAL, "%s: head_dim=%d d_t=%d d_h=%d (head_dim a "
                "power of two >= 16, d_t/16 and d_h/16 powers of two, d_h | "
                "d_t; other shapes take the separate calls)", what, head_dim,
                d_t, d_h);
  }
  if (offset < 0 || cap <= 0 || (long long)offset + T > cap) {
    return fail(ctx, U15H_EINVAL, "%s: offset %d + T %d exceeds capacity %d",
                what, offset, T, cap);
  }
  if (!(eps >= 0.0f)) {
    return fail(ctx, U15H_EINVAL, "%s: eps must be >= 0", what);
  }
  if (T == 0) { ctx->err.clear(); return U15H_OK; }
  const u15h_qk_norm* sets[2] = {und, gen};
  const bool used[2] = {M_und > 0, M_gen > 0};
  u15h::PrologueArgs a{};
  for (int e = 0; e < 2; ++e) {
    if (!used[e]) { continue; }
    const u15h_qk_norm* n = sets[e];
    if (n == nullptr || n->q_t == nullptr || n->q_hw == nullptr ||
        n->k_t == nullptr || n->k_hw == nullptr || !aligned16(n->q_t) ||
        !aligned16(n->q_hw) || !aligned16(n->k_t) || !aligned16(n->k_hw)) {
      return fail(ctx, U15H_EINVAL, "%s: %s norm weights null or misaligned",
                  what, e == 0 ? "und" : "gen");
    }
    a.w[e][0] = n->q_t;
    a.w[e][1] = n->q_hw;
    a.w[e][2] = n->k_t;
    a.w[e][3] = n->k_hw;
  }
  // an unused group's slots point at the used one's (never read)
  for (int j = 0; j < 4; ++j) {
    if (!used[0]) { a.w[0][j] = a.w[1][j]; }
    if (!used[1]) { a.w[1][j] = a.w[0][j]; }
  }
  const void* ptrs[7] = {q, k, v, k_cache, v_cache, cos_tab, sin_tab};
  for (const void* ptr : ptrs) {
    if (ptr == nullptr || !aligned16(ptr)) {
      return fail(ctx, U15H_EINVAL, "%s: null or misaligned operand", what);
    }
  }
  if ((st = bind_device(ctx)) != U15H_OK) { return st; }
  a.q = q;
  a.k = k;
  a.v = v;
  a.k_cache = k_cache;
  a.v_cache = v_cache;
  a.cosf = cos_tab;
  a.sinf = sin_tab;
  a.tokens = T;
  a.m_und = M_und;
  a.hq = hq;
  a.hkv = hkv;
  a.d = head_dim;
  a.d_t = d_t;
  a.d_h = d_h;
  a.cap = cap;
  a.offset = offset;
  a.eps = eps;
  return launched(ctx,
                  u15h::launch_attention_prologue(a, as_stream(stream),
                                                  ctx->prologue_rpt),
                  what);
}

u15h_status
u15h_build_rope_tables(const int32_t* pos_t, const int32_t* pos_h,
                       const int32_t* pos_w, int tokens, int head_dim, int d_t,
                       int d_h, double theta_t, double theta_hw,
                       float* cos_tab, float* sin_tab)
{
  if (tokens < 0 || head_dim <= 0 || d_t <= 0 || d_h <= 0 || d_t % 2 != 0 ||
      d_h % 2 != 0 || d_t + 2 * d_h != head_dim || !(theta_t > 0.0) ||
      !(theta_hw > 0.0)) {
    return U15H_EINVAL;
  }
  if (tokens == 0) { return U15H_OK; }
  if (pos_t == nullptr || pos_h == nullptr || pos_w == nullptr ||
      cos_tab == nullptr || sin_tab == nullptr) {
    return U15H_EINVAL;
  }
  // Per range its own ladder 1/theta^(2i/width), the angle pos * inv in
  // double, narrowed once; the range's second half repeats the first
  // (rotate_half reads c[j] and c[j + width/2] for one pair).
  struct Range { int off, width; double theta; const int32_t* pos; };
  const Range ranges[3] = {{0, d_t, theta_t, pos_t},
                           {d_t, d_h, theta_hw, pos_h},
                           {d_t + d_h, d_h, theta_hw, pos_w}};
  for (const Range& r : ranges) {
    const int half = r.width / 2;
    std::vector<double> inv((size_t)half);
    for (int i = 0; i < half; ++i) {
      inv[(size_t)i] = 1.0 / std::pow(r.theta, (double)(2 * i) / r.width);
    }
    for (int t = 0; t < tokens; ++t) {
      const size_t base = (size_t)t * head_dim + r.off;
      for (int i = 0; i < half; ++i) {
        const double a = (double)r.pos[t] * inv[(size_t)i];
        const float c = (float)std::cos(a), sn = (float)std::sin(a);
        cos_tab[base + i] = c;
        cos_tab[base + i + half] = c;
        sin_tab[base + i] = sn;
        sin_tab[base + i + half] = sn;
      }
    }
  }
  return U15H_OK;
}

u15h_status
u15h_route_rows(const uint8_t* expert, int M, int32_t* perm, int* M_und,
                int* M_gen)
{
  if (M < 0 || (M > 0 && (expert == nullptr || perm == nullptr)) ||
      M_und == nullptr || M_gen == nullptr) {
    return U15H_EINVAL;
  }
  int nu = 0;
  for (int i = 0; i < M; ++i) {
    if (expert[i] > 1) { return U15H_EINVAL; }
    if (expert[i] == 0) { ++nu; }
  }
  // Stable partition: und tokens first, then gen, original order kept.
  int iu = 0, ig = nu;
  for (int i = 0; i < M; ++i) {
    if (expert[i] == 0) { perm[iu++] = i; } else { perm[ig++] = i; }
  }
  *M_und = nu;
  *M_gen = M - nu;
  return U15H_OK;
}

static u15h_status
gather_common(u15h_ctx* ctx, u15h_stream stream, const u15h_bf16* src,
              const int32_t* perm, int M, int cols, u15h_bf16* dst,
              bool scatter)
{
  if (ctx == nullptr) { return U15H_EINVAL; }
  if (M < 0 || cols <= 0 || cols % 8 != 0) {
    return fail(ctx, U15H_EINVAL, "M=%d cols=%d (cols must be a multiple of 8)",
                M, cols);
  }
  if (M == 0) { ctx->err.clear(); return U15H_OK; }
  if (src == nullptr || perm == nullptr || dst == nullptr ||
      !aligned16(src) || !aligned16(dst)) {
    return fail(ctx, U15H_EINVAL, "null or misaligned gather operand");
  }
  u15h_status st = bind_device(ctx);
  if (st != U15H_OK) { return st; }
  return launched(ctx,
                  u15h::launch_gather_rows(src, perm, M, cols, dst, scatter,
                                           as_stream(stream)),
                  scatter ? "scatter_rows" : "gather_rows");
}

u15h_status
u15h_gather_rows(u15h_ctx* ctx, u15h_stream stream, const u15h_bf16* src,
                 const int32_t* perm, int M, int cols, u15h_bf16* dst)
{
  return gather_common(ctx, stream, src, perm, M, cols, dst, false);
}

u15h_status
u15h_scatter_rows(u15h_ctx* ctx, u15h_stream stream, const u15h_bf16* src,
                  const int32_t* perm, int M, int cols, u15h_bf16* dst)
{
  return gather_common(ctx, stream, src, perm, M, cols, dst, true);
}

}  // extern "C"
