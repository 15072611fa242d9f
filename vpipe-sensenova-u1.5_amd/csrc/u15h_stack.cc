// u15h_stack.cc -- the resident MoT layer stack (include/u15h.h).
//
// A host table of device pointers: per layer, the seven projection
// matrices of both experts (the reference's MotLayer{und, gen} of
// ExpertLayer, src/u15-weights.h:97-117), bound by the reference's tensor
// names (src/u15-weights.cc:539-578).  A layer's projections run as four
// grouped launches through the public entry points, each over both weight
// sets: q|k|v, o, gate|up, down -- the projection half of
// U15Backbone::layer_step_ (src/u15-backbone.cc:174-257).  Every argument
// of every step is checked before the first launch, so a refusal launches
// nothing.
#include "u15h.h"

#include <cstdio>
#include <cstring>
#include <initializer_list>
#include <string>
#include <vector>

#include "u15h_internal.h"

struct u15h_stack {
  int n_layers = 0;
  int hidden = 0, qdim = 0, kvdim = 0, inter = 0;
  int heads = 0, kv_heads = 0, head_dim = 0;
  // [layer][expert][which] the six norm vectors of ExpertLayer
  std::vector<const u15h_bf16*> norms;
  const u15h_bf16*& norm(int l, int e, int w)
  {
    return norms[((size_t)l * 2 + e) * U15H_NNORM + w];
  }
  const u15h_bf16* norm(int l, int e, int w) const
  {
    return norms[((size_t)l * 2 + e) * U15H_NNORM + w];
  }
  struct Slot {
    const u15h_bf16* w = nullptr;
    const int8_t* wq = nullptr;
    const float* sw = nullptr;
  };
  // [layer][expert][proj]
  std::vector<Slot> slots;

  Slot& at(int l, int e, int p) { return slots[((size_t)l * 2 + e) * U15H_NPROJ + p]; }
  const Slot& at(int l, int e, int p) const
  {
    return slots[((size_t)l * 2 + e) * U15H_NPROJ + p];
  }
  // Output columns (N) and input width (K) of a projection.
  int n_of(int p) const
  {
    switch (p) {
      case U15H_PROJ_Q: return qdim;
      case U15H_PROJ_K: case U15H_PROJ_V: return kvdim;
      case U15H_PROJ_O: case U15H_PROJ_DOWN: return hidden;
      default: return inter;   // gate, up
    }
  }
  int k_of(int p) const
  {
    switch (p) {
      case U15H_PROJ_O: return qdim;
      case U15H_PROJ_DOWN: return inter;
      default: return hidden;
    }
  }
};

namespace {

const char* const kProjName[U15H_NPROJ] = {"q", "k", "v", "o", "gate", "up", "down"};

bool
aligned16(const void* p)
{
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

// Consumes `lit` at *s.
bool
eat(const char** s, const char* lit)
{
  const size_t n = std::strlen(lit);
  if (std::strncmp(*s, lit, n) != 0) { return false; }
  *s += n;
  return true;
}

// The reference's name of a slot (for u15h_stack_check's message).
std::string
slot_name(int l, int e, int p)
{
  const std::string pre = "language_model.model.layers." + std::to_string(l) + ".";
  const std::string sfx = e == U15H_GEN ? "_mot_gen" : "";
  if (p <= U15H_PROJ_O) {
    return pre + "self_attn." + kProjName[p] + "_proj" + sfx + ".weight";
  }
  return pre + "mlp" + sfx + "." + kProjName[p] + "_proj.weight";
}

// The reference's name of a norm slot (for u15h_stack_check_full).
std::string
norm_name(int l, int w, int e)
{
  const std::string pre = "language_model.model.layers." + std::to_string(l) + ".";
  const std::string sfx = e == U15H_GEN ? "_mot_gen" : "";
  switch (w) {
    case U15H_NORM_INPUT: return pre + "input_layernorm" + sfx + ".weight";
    case U15H_NORM_POST: return pre + "post_attention_layernorm" + sfx + ".weight";
    case U15H_NORM_Q: return pre + "self_attn.q_norm" + sfx + ".weight";
    case U15H_NORM_K: return pre + "self_attn.k_norm" + sfx + ".weight";
    case U15H_NORM_Q_HW: return pre + "self_attn.q_norm_hw" + sfx + ".weight";
    default: return pre + "self_attn.k_norm_hw" + sfx + ".weight";
  }
}

// Weights of every step in `steps` are bound for the experts with rows.
bool
step_weights_ok(const u15h_stack* st, int layer, int steps, int tier,
                bool und, bool gen)
{
  static const int kStepProj[4][3] = {{U15H_PROJ_Q, U15H_PROJ_K, U15H_PROJ_V},
                                      {U15H_PROJ_O, -1, -1},
                                      {U15H_PROJ_GATE, U15H_PROJ_UP, -1},
                                      {U15H_PROJ_DOWN, -1, -1}};
  for (int b = 0; b < 4; ++b) {
    if ((steps & (1 << b)) == 0) { continue; }
    for (int j = 0; j < 3 && kStepProj[b][j] >= 0; ++j) {
      const int p = kStepProj[b][j];
      for (int e = 0; e < 2; ++e) {
        if ((e == U15H_UND && !und) || (e == U15H_GEN && !gen)) { continue; }
        const auto& s = st->at(layer, e, p);
        if (tier == U15H_TIER_I8 ? (s.wq == nullptr || s.sw == nullptr)
                                 : s.w == nullptr) {
          return false;
        }
      }
    }
  }
  return true;
}

// io pointers of every step in `steps` are present and 16-byte aligned.
bool
io_ok(const u15h_layer_io* io, int steps, int tier, int flags)
{
  auto ok = [](const void* p) { return p != nullptr && aligned16(p); };
  const bool fused = (flags & U15H_FUSED_SWIGLU) != 0;
  if ((steps & U15H_STEP_QKV) && !(ok(io->x) && ok(io->q) && ok(io->k) && ok(io->v))) {
    return false;
  }
  if ((steps & U15H_STEP_O) && !(ok(io->attn) && ok(io->o))) { return false; }
  if (steps & U15H_STEP_GATE_UP) {
    if (!ok(io->x2)) { return false; }
    if (fused ? !ok(io->h) : !(ok(io->gate) && ok(io->up))) { return false; }
  }
  if ((steps & U15H_STEP_DOWN) && !(ok(io->h) && ok(io->down))) { return false; }
  if (tier == U15H_TIER_I8 && !(ok(io->xq) && ok(io->sx))) { return false; }
  return true;
}

u15h_mot_proj
bf16_proj(const u15h_stack* st, int layer, int p, u15h_bf16* y)
{
  u15h_mot_proj r;
  r.w_und = st->at(layer, U15H_UND, p).w;
  r.w_gen = st->at(layer, U15H_GEN, p).w;
  r.bias_und = nullptr;
  r.bias_gen = nullptr;
  r.y = y;
  r.N = st->n_of(p);
  return r;
}

u15h_mot_proj_i8
i8_proj(const u15h_stack* st, int layer, int p, u15h_bf16* y)
{
  u15h_mot_proj_i8 r;
  const auto& u = st->at(layer, U15H_UND, p);
  const auto& g = st->at(layer, U15H_GEN, p);
  r.wq_und = u.wq;
  r.sw_und = u.sw;
  r.wq_gen = g.wq;
  r.sw_gen = g.sw;
  r.y = y;
  r.N = st->n_of(p);
  return r;
}

// One step, arguments already checked.
u15h_status
run_step(u15h_ctx* ctx, u15h_stream s, const u15h_stack* st, int layer,
         const u15h_layer_io* io, int M_und, int M_gen, int step, int tier,
         int flags)
{
  const int M = M_und + M_gen;
  const u15h_bf16* in = nullptr;
  int K = 0, np = 0;
  int ids[3] = {0, 0, 0};
  u15h_bf16* outs[3] = {nullptr, nullptr, nullptr};
  switch (step) {
    case U15H_STEP_QKV:
      in = io->x; K = st->hidden; np = 3;
      ids[0] = U15H_PROJ_Q; ids[1] = U15H_PROJ_K; ids[2] = U15H_PROJ_V;
      outs[0] = io->q; outs[1] = io->k; outs[2] = io->v;
      break;
    case U15H_STEP_O:
      in = io->attn; K = st->qdim; np = 1;
      ids[0] = U15H_PROJ_O; outs[0] = io->o;
      break;
    case U15H_STEP_GATE_UP:
      in = io->x2; K = st->hidden; np = 2;
      ids[0] = U15H_PROJ_GATE; ids[1] = U15H_PROJ_UP;
      outs[0] = io->gate; outs[1] = io->up;
      break;
    default:
      in = io->h; K = st->inter; np = 1;
      ids[0] = U15H_PROJ_DOWN; outs[0] = io->down;
      break;
  }
  if (tier == U15H_TIER_I8) {
    u15h_status r = u15h_quant_rows_i8(ctx, s, in, M, K, io->xq, io->sx);
    if (r != U15H_OK) { return r; }
    u15h_mot_proj_i8 p[3];
    for (int i = 0; i < np; ++i) { p[i] = i8_proj(st, layer, ids[i], outs[i]); }
    return u15h_mot_gemm_i8(ctx, s, io->xq, io->sx, M_und, M_gen, K, p, np);
  }
  if (step == U15H_STEP_GATE_UP && (flags & U15H_FUSED_SWIGLU)) {
    const auto& u = st->at(layer, U15H_UND, U15H_PROJ_GATE);
    const auto& uu = st->at(layer, U15H_UND, U15H_PROJ_UP);
    const auto& g = st->at(layer, U15H_GEN, U15H_PROJ_GATE);
    const auto& gu = st->at(layer, U15H_GEN, U15H_PROJ_UP);
    return u15h_mot_gate_up_swiglu(ctx, s, in, M_und, M_gen, K, u.w, uu.w, g.w,
                                   gu.w, io->h, st->inter);
  }
  u15h_mot_proj p[3];
  for (int i = 0; i < np; ++i) { p[i] = bf16_proj(st, layer, ids[i], outs[i]); }
  return u15h_mot_linear(ctx, s, in, M_und, M_gen, K, p, np);
}

// The int8 tier's limits on the stack's widths, each some projection's K:
// u15h_mot_gemm_i8's K % 128 == 0 and K <= 131072 (int32 accumulators stay
// exact).  Checked before a pass's first launch, so no step's quantiser or
// GEMM runs before a later step would refuse.
const char*
i8_widths_error(const u15h_stack* st)
{
  if (st->hidden % 128 || st->qdim % 128 || st->inter % 128) {
    return "int8 tier: every projection's K must be a multiple of 128";
  }
  if (st->hidden > 131072 || st->qdim > 131072 || st->inter > 131072) {
    return "int8 tier: every projection's K must be at most 131072";
  }
  return nullptr;
}

// Arguments of a stack call; nullptr if they are acceptable, else why not.
const char*
check_call(const u15h_stack* st, const u15h_layer_io* io, int M_und,
           int M_gen, int steps, int tier, int flags)
{
  if (st == nullptr || io == nullptr) { return "null stack or io"; }
  if (M_und < 0 || M_gen < 0 || (long long)M_und + M_gen > (1 << 24)) {
    return "row counts out of range";
  }
  if (steps <= 0 || (steps & ~U15H_STEP_ALL) != 0) { return "bad step mask"; }
  if (tier != U15H_TIER_BF16 && tier != U15H_TIER_I8) { return "bad tier"; }
  if ((flags & ~U15H_FUSED_SWIGLU) != 0) { return "unknown flags"; }
  if (tier == U15H_TIER_I8 && (flags & U15H_FUSED_SWIGLU)) {
    return "the fused SwiGLU epilogue is a bf16-tier option";
  }
  if (tier == U15H_TIER_I8) {
    if (const char* why = i8_widths_error(st)) { return why; }
  }
  if (M_und + M_gen > 0 && !io_ok(io, steps, tier, flags)) {
    return "an io buffer the steps need is null or not 16-byte aligned";
  }
  return nullptr;
}

// "language_model.model.layers.<i>." with <i> a decimal layer index as
// std::to_string writes it: no sign, no leading zero (except "0"), at most
// 9 digits.
bool
eat_layer(const char** sp, long long* li)
{
  const char* s = *sp;
  if (!eat(&s, "language_model.model.layers.")) { return false; }
  if (*s < '0' || *s > '9' || (s[0] == '0' && s[1] >= '0' && s[1] <= '9')) {
    return false;
  }
  long long v = 0;
  int nd = 0;
  while (*s >= '0' && *s <= '9') {
    v = v * 10 + (*s - '0');
    ++s;
    if (++nd > 9) { return false; }
  }
  if (!eat(&s, ".")) { return false; }
  *sp = s;
  *li = v;
  return true;
}

bool
is_pow2(int v)
{
  return v > 0 && (v & (v - 1)) == 0;
}

// Arguments of a whole-layer call; nullptr if acceptable, else why not.
const char*
check_full_call(const u15h_stack* st, int layer, const u15h_layer_full_io* io,
                int M_und, int M_gen, int tier)
{
  if (st == nullptr || io == nullptr) { return "null stack or io"; }
  if (layer < 0 || layer >= st->n_layers) { return "layer index outside the stack"; }
  if (M_und < 0 || M_gen < 0 || (long long)M_und + M_gen > (1 << 24)) {
    return "row counts out of range";
  }
  if (tier != U15H_TIER_BF16 && tier != U15H_TIER_I8) { return "bad tier"; }
  const int M = M_und + M_gen;
  if (M == 0) { return nullptr; }
  if (tier == U15H_TIER_I8) {
    if (const char* why = i8_widths_error(st)) { return why; }
  }
  const int hd = st->head_dim;
  if (hd != 32 && hd != 64 && hd != 128) {
    return "whole layer: head_dim must be 32, 64 or 128 (the attention kernel's)";
  }
  if (io->d_t <= 0 || io->d_h <= 0 || io->d_t + 2 * io->d_h != hd ||
      io->d_t % 16 || io->d_h % 16 || !is_pow2(io->d_t / 16) ||
      !is_pow2(io->d_h / 16) || io->d_t % io->d_h) {
    return "whole layer: the RoPE ranges must split head_dim as [t | h | w] with "
           "d_t/16 and d_h/16 powers of two and d_h dividing d_t";
  }
  if (st->hidden > 16384 || (tier == U15H_TIER_I8 && st->inter > 16384)) {
    return "whole layer: the norms take rows of at most 16384";
  }
  if (!(io->eps >= 0.0f)) { return "whole layer: eps must be >= 0"; }
  if (io->mode < 0 || io->mode > 2) { return "whole layer: bad attention mode"; }
  if (io->cap <= 0 || io->kv_off < 0 || (long long)io->kv_off + M > io->kv_len ||
      io->kv_len > io->cap) {
    return "whole layer: needs kv_off + M <= kv_len <= cap";
  }
  if ((long long)io->cap * hd * 2 >= (1LL << 31)) {
    return "whole layer: one kv head's cache must stay below 2 GiB";
  }
  auto ok = [](const void* p) { return p != nullptr && aligned16(p); };
  if (!(ok(io->x) && ok(io->q) && ok(io->k) && ok(io->v) && ok(io->attn) &&
        ok(io->proj) && ok(io->h) && ok(io->k_cache) && ok(io->v_cache) &&
        ok(io->cos_tab) && ok(io->sin_tab))) {
    return "whole layer: an io buffer is null or not 16-byte aligned";
  }
  if (tier == U15H_TIER_BF16 ? !ok(io->normed)
                             : !(ok(io->up) && ok(io->xq) && ok(io->sx))) {
    return "whole layer: a tier buffer is null or not 16-byte aligned";
  }
  if (io->mode == 2 && io->t_index == nullptr) {
    return "whole layer: block-causal attention needs t_index";
  }
  // the residual stream keeps its sum: no scratch buffer may be x (the
  // post-attention norm would refuse it after the layer's first launches)
  for (const void* p : {(const void*)io->normed, (const void*)io->q, (const void*)io->k,
                        (const void*)io->v, (const void*)io->attn, (const void*)io->proj,
                        (const void*)io->h, (const void*)io->up}) {
    if (p == io->x) { return "whole layer: a scratch buffer is x"; }
  }
  if (!step_weights_ok(st, layer, U15H_STEP_ALL, tier, M_und > 0, M_gen > 0)) {
    return "a matrix the layer needs is not bound (u15h_stack_check_full names it)";
  }
  for (int e = 0; e < 2; ++e) {
    if ((e == U15H_UND ? M_und : M_gen) == 0) { continue; }
    for (int w = 0; w < U15H_NNORM; ++w) {
      if (st->norm(layer, e, w) == nullptr) {
        return "a norm the layer needs is not bound (u15h_stack_check_full names it)";
      }
    }
  }
  return nullptr;
}

// One whole layer, its arguments already checked (check_full_call) and M >
// 0.  `input_normed`: the input norm's output (normed, or xq and sx for
// the int8 tier) is already in io, written by the previous layer's last
// pass.  `next` >= 0: instead of the residual add, that pass is the add
// and layer `next`'s input norm together (u15h_mot_rms_norm with the down
// output as delta), the same bits as u15h_add then the norm.
u15h_status
run_full_layer(u15h_ctx* ctx, u15h_stream stream, const u15h_stack* st, int layer,
               const u15h_layer_full_io* io, int M_und, int M_gen, int tier,
               bool input_normed, int next)
{
  const int M = M_und + M_gen;
  const bool i8 = tier == U15H_TIER_I8;
  const u15h_bf16* const* nu = &st->norms[((size_t)layer * 2 + U15H_UND) * U15H_NNORM];
  const u15h_bf16* const* ng = &st->norms[((size_t)layer * 2 + U15H_GEN) * U15H_NNORM];
  const int H = st->hidden, I = st->inter;
  u15h_status r = U15H_OK;
#define U15H_RUN(call)                     \
  do {                                     \
    r = (call);                            \
    if (r != U15H_OK) { return r; }        \
  } while (0)
  auto proj = [&](const u15h_bf16* in, int K, std::initializer_list<int> ids,
                  std::initializer_list<u15h_bf16*> outs) {
    u15h_mot_proj p[3];
    int n = 0;
    auto o = outs.begin();
    for (int id : ids) { p[n++] = bf16_proj(st, layer, id, *o++); }
    return u15h_mot_linear(ctx, stream, in, M_und, M_gen, K, p, n);
  };
  auto proj8 = [&](int K, std::initializer_list<int> ids,
                   std::initializer_list<u15h_bf16*> outs) {
    u15h_mot_proj_i8 p[3];
    int n = 0;
    auto o = outs.begin();
    for (int id : ids) { p[n++] = i8_proj(st, layer, id, *o++); }
    return u15h_mot_gemm_i8(ctx, stream, io->xq, io->sx, M_und, M_gen, K, p, n);
  };
  // attention: the input norm, q|k|v, the prologue, attention, o
  if (!input_normed) {
    U15H_RUN(u15h_mot_rms_norm(ctx, stream, io->x, nullptr, M_und, M_gen, H,
                               nu[U15H_NORM_INPUT], ng[U15H_NORM_INPUT], io->eps,
                               i8 ? nullptr : io->normed, i8 ? io->xq : nullptr,
                               i8 ? io->sx : nullptr));
  }
  if (i8) {
    U15H_RUN(proj8(H, {U15H_PROJ_Q, U15H_PROJ_K, U15H_PROJ_V}, {io->q, io->k, io->v}));
  } else {
    U15H_RUN(proj(io->normed, H, {U15H_PROJ_Q, U15H_PROJ_K, U15H_PROJ_V},
                  {io->q, io->k, io->v}));
  }
  const u15h_qk_norm qn_u = {nu[U15H_NORM_Q], nu[U15H_NORM_Q_HW], nu[U15H_NORM_K],
                             nu[U15H_NORM_K_HW]};
  const u15h_qk_norm qn_g = {ng[U15H_NORM_Q], ng[U15H_NORM_Q_HW], ng[U15H_NORM_K],
                             ng[U15H_NORM_K_HW]};
  U15H_RUN(u15h_mot_attention_prologue(ctx, stream, io->q, io->k, io->v,
                                       M_und > 0 ? &qn_u : nullptr,
                                       M_gen > 0 ? &qn_g : nullptr, io->cos_tab,
                                       io->sin_tab, M_und, M_gen, st->heads,
                                       st->kv_heads, st->head_dim, io->d_t, io->d_h,
                                       io->eps, io->k_cache, io->v_cache, io->cap,
                                       io->kv_off));
  U15H_RUN(u15h_attention_token_major(ctx, stream, io->q, io->k_cache, io->v_cache,
                                      io->attn, io->t_index, st->heads, st->kv_heads,
                                      M, io->kv_len, st->head_dim, io->cap,
                                      io->kv_off, io->mode));
  if (i8) {
    U15H_RUN(u15h_quant_rows_i8(ctx, stream, io->attn, M, st->qdim, io->xq, io->sx));
    U15H_RUN(proj8(st->qdim, {U15H_PROJ_O}, {io->proj}));
    // x += o; the post norm's codes
    U15H_RUN(u15h_mot_rms_norm(ctx, stream, io->x, io->proj, M_und, M_gen, H,
                               nu[U15H_NORM_POST], ng[U15H_NORM_POST], io->eps,
                               nullptr, io->xq, io->sx));
    U15H_RUN(proj8(H, {U15H_PROJ_GATE, U15H_PROJ_UP}, {io->h, io->up}));
    U15H_RUN(u15h_swiglu_quant_i8(ctx, stream, io->h, io->up, M, I, nullptr, io->xq,
                                  io->sx));
    U15H_RUN(proj8(I, {U15H_PROJ_DOWN}, {io->proj}));
  } else {
    U15H_RUN(proj(io->attn, st->qdim, {U15H_PROJ_O}, {io->proj}));
    // x += o; normed = the post norm
    U15H_RUN(u15h_mot_rms_norm(ctx, stream, io->x, io->proj, M_und, M_gen, H,
                               nu[U15H_NORM_POST], ng[U15H_NORM_POST], io->eps,
                               io->normed, nullptr, nullptr));
    const auto& gu = st->at(layer, U15H_UND, U15H_PROJ_GATE);
    const auto& uu = st->at(layer, U15H_UND, U15H_PROJ_UP);
    const auto& gg = st->at(layer, U15H_GEN, U15H_PROJ_GATE);
    const auto& ug = st->at(layer, U15H_GEN, U15H_PROJ_UP);
    U15H_RUN(u15h_mot_gate_up_swiglu(ctx, stream, io->normed, M_und, M_gen, H, gu.w,
                                     uu.w, gg.w, ug.w, io->h, I));
    U15H_RUN(proj(io->h, I, {U15H_PROJ_DOWN}, {io->proj}));
  }
  if (next < 0) {
    U15H_RUN(u15h_add(ctx, stream, io->x, io->proj, (int64_t)M * H));
  } else {
    // x += down; the next layer's input norm (its codes for the int8 tier)
    const u15h_bf16* const* xu = &st->norms[((size_t)next * 2 + U15H_UND) * U15H_NNORM];
    const u15h_bf16* const* xg = &st->norms[((size_t)next * 2 + U15H_GEN) * U15H_NNORM];
    U15H_RUN(u15h_mot_rms_norm(ctx, stream, io->x, io->proj, M_und, M_gen, H,
                               xu[U15H_NORM_INPUT], xg[U15H_NORM_INPUT], io->eps,
                               i8 ? nullptr : io->normed, i8 ? io->xq : nullptr,
                               i8 ? io->sx : nullptr));
  }
#undef U15H_RUN
  return U15H_OK;
}


}  // namespace

extern "C" {

u15h_status
u15h_stack_create(int n_layers, int hidden, int heads, int kv_heads,
                  int head_dim, int inter, u15h_stack** out)
{
  if (out == nullptr) { return U15H_EINVAL; }
  *out = nullptr;
  if (n_layers <= 0 || n_layers > 4096 || hidden <= 0 || heads <= 0 ||
      kv_heads <= 0 || head_dim <= 0 || inter <= 0 || heads % kv_heads != 0) {
    return U15H_EINVAL;
  }
  const long long qd = (long long)heads * head_dim;
  const long long kvd = (long long)kv_heads * head_dim;
  // Every width is both some projection's K (bf16: % 8; int8: % 128 is
  // checked per call) and some projection's N (% 8).
  if (hidden % 8 || qd % 8 || kvd % 8 || inter % 8 || qd > (1 << 20) ||
      hidden > (1 << 20) || inter > (1 << 20)) {
    return U15H_EINVAL;
  }
  u15h_stack* st = new u15h_stack;
  st->n_layers = n_layers;
  st->hidden = hidden;
  st->qdim = (int)qd;
  st->kvdim = (int)kvd;
  st->inter = inter;
  st->heads = heads;
  st->kv_heads = kv_heads;
  st->head_dim = head_dim;
  st->slots.resize((size_t)n_layers * 2 * U15H_NPROJ);
  st->norms.assign((size_t)n_layers * 2 * U15H_NNORM, nullptr);
  *out = st;
  return U15H_OK;
}

void
u15h_stack_destroy(u15h_stack* st)
{
  delete st;
}

u15h_status
u15h_weight_slot(const char* name, int* layer, int* expert, int* proj)
{
  if (name == nullptr || layer == nullptr || expert == nullptr || proj == nullptr) {
    return U15H_EINVAL;
  }
  const char* s = name;
  long long li = 0;
  if (!eat_layer(&s, &li)) { return U15H_EINVAL; }
  int e = U15H_UND, p = -1;
  if (eat(&s, "self_attn.")) {
    // The attention suffixes the TENSOR: q_proj_mot_gen.
    for (int i = U15H_PROJ_Q; i <= U15H_PROJ_O; ++i) {
      const char* t = s;
      if (eat(&t, kProjName[i]) && eat(&t, "_proj")) { p = i; s = t; break; }
    }
    if (p < 0) { return U15H_EINVAL; }
    if (eat(&s, "_mot_gen")) { e = U15H_GEN; }
  } else if (eat(&s, "mlp")) {
    // The MLP suffixes the MODULE: mlp_mot_gen.gate_proj.
    if (eat(&s, "_mot_gen")) { e = U15H_GEN; }
    if (!eat(&s, ".")) { return U15H_EINVAL; }
    for (int i = U15H_PROJ_GATE; i <= U15H_PROJ_DOWN; ++i) {
      const char* t = s;
      if (eat(&t, kProjName[i]) && eat(&t, "_proj")) { p = i; s = t; break; }
    }
    if (p < 0) { return U15H_EINVAL; }
  } else {
    return U15H_EINVAL;
  }
  (void)eat(&s, ".weight");
  if (*s != '\0') { return U15H_EINVAL; }
  *layer = (int)li;
  *expert = e;
  *proj = p;
  return U15H_OK;
}

u15h_status
u15h_stack_set(u15h_stack* st, int layer, int expert, int proj,
               const u15h_bf16* w, const int8_t* wq, const float* sw)
{
  if (st == nullptr || layer < 0 || layer >= st->n_layers ||
      (expert != U15H_UND && expert != U15H_GEN) || proj < 0 ||
      proj >= U15H_NPROJ || ((wq == nullptr) != (sw == nullptr))) {
    return U15H_EINVAL;
  }
  if ((w != nullptr && !aligned16(w)) || (wq != nullptr && !aligned16(wq)) ||
      (sw != nullptr && !aligned16(sw))) {
    return U15H_EINVAL;
  }
  auto& s = st->at(layer, expert, proj);
  if (w != nullptr) { s.w = w; }
  if (wq != nullptr) {
    s.wq = wq;
    s.sw = sw;
  }
  return U15H_OK;
}

u15h_status
u15h_stack_bind(u15h_stack* st, const char* name, const u15h_bf16* w)
{
  int l = 0, e = 0, p = 0;
  if (st == nullptr || w == nullptr) { return U15H_EINVAL; }
  u15h_status r = u15h_weight_slot(name, &l, &e, &p);
  if (r != U15H_OK) { return r; }
  return u15h_stack_set(st, l, e, p, w, nullptr, nullptr);
}

u15h_status
u15h_stack_bind_i8(u15h_stack* st, const char* name, const int8_t* wq,
                   const float* sw)
{
  int l = 0, e = 0, p = 0;
  if (st == nullptr || wq == nullptr || sw == nullptr) { return U15H_EINVAL; }
  u15h_status r = u15h_weight_slot(name, &l, &e, &p);
  if (r != U15H_OK) { return r; }
  return u15h_stack_set(st, l, e, p, nullptr, wq, sw);
}

u15h_status
u15h_stack_check(const u15h_stack* st, int need_und, int need_gen, int tier,
                 char* missing, size_t missing_cap)
{
  if (st == nullptr || (tier != U15H_TIER_BF16 && tier != U15H_TIER_I8)) {
    return U15H_EINVAL;
  }
  if (tier == U15H_TIER_I8) {
    if (const char* why = i8_widths_error(st)) {
      if (missing != nullptr && missing_cap > 0) {
        std::snprintf(missing, missing_cap, "%s", why);
      }
      return U15H_EINVAL;
    }
  }
  for (int l = 0; l < st->n_layers; ++l) {
    for (int e = 0; e < 2; ++e) {
      if ((e == U15H_UND && !need_und) || (e == U15H_GEN && !need_gen)) { continue; }
      for (int p = 0; p < U15H_NPROJ; ++p) {
        const auto& s = st->at(l, e, p);
        const bool bound = tier == U15H_TIER_I8 ? s.wq != nullptr && s.sw != nullptr
                                                : s.w != nullptr;
        if (!bound) {
          if (missing != nullptr && missing_cap > 0) {
            std::snprintf(missing, missing_cap, "%s%s", slot_name(l, e, p).c_str(),
                          tier == U15H_TIER_I8 ? " (int8)" : "");
          }
          return U15H_EINVAL;
        }
      }
    }
  }
  if (missing != nullptr && missing_cap > 0) { missing[0] = '\0'; }
  return U15H_OK;
}

u15h_status
u15h_stack_layer(u15h_ctx* ctx, u15h_stream stream, const u15h_stack* st,
                 int layer, const u15h_layer_io* io, int M_und, int M_gen,
                 int steps, int tier, int flags)
{
  if (ctx == nullptr) { return U15H_EINVAL; }
  if (const char* why = check_call(st, io, M_und, M_gen, steps, tier, flags)) {
    return u15h::set_error(ctx, U15H_EINVAL, why);
  }
  if (layer < 0 || layer >= st->n_layers) {
    return u15h::set_error(ctx, U15H_EINVAL, "layer index outside the stack");
  }
  if (M_und + M_gen == 0) { return u15h::set_error(ctx, U15H_OK, ""); }
  if (!step_weights_ok(st, layer, steps, tier, M_und > 0, M_gen > 0)) {
    return u15h::set_error(ctx, U15H_EINVAL,
                           "a matrix the steps need is not bound (u15h_stack_check names it)");
  }
  u15h_status r = U15H_OK;
  for (int b = 0; b < 4; ++b) {
    const int step = 1 << b;
    if ((steps & step) == 0) { continue; }
    r = run_step(ctx, stream, st, layer, io, M_und, M_gen, step, tier, flags);
    if (r != U15H_OK) { return r; }
  }
  return U15H_OK;
}

u15h_status
u15h_stack_forward(u15h_ctx* ctx, u15h_stream stream, const u15h_stack* st,
                   const u15h_layer_io* io, int M_und, int M_gen, int tier,
                   int flags)
{
  if (ctx == nullptr) { return U15H_EINVAL; }
  if (const char* why = check_call(st, io, M_und, M_gen, U15H_STEP_ALL, tier, flags)) {
    return u15h::set_error(ctx, U15H_EINVAL, why);
  }
  if (M_und + M_gen == 0) { return u15h::set_error(ctx, U15H_OK, ""); }
  for (int l = 0; l < st->n_layers; ++l) {
    if (!step_weights_ok(st, l, U15H_STEP_ALL, tier, M_und > 0, M_gen > 0)) {
      return u15h::set_error(ctx, U15H_EINVAL,
                             "a matrix the pass needs is not bound (u15h_stack_check names it)");
    }
  }
  u15h_status r = U15H_OK;
  for (int l = 0; l < st->n_layers; ++l) {
    for (int b = 0; b < 4; ++b) {
      r = run_step(ctx, stream, st, l, io, M_und, M_gen, 1 << b, tier, flags);
      if (r != U15H_OK) { return r; }
    }
  }
  return U15H_OK;
}

u15h_status
u15h_norm_slot(const char* name, int* layer, int* expert, int* which)
{
  if (name == nullptr || layer == nullptr || expert == nullptr || which == nullptr) {
    return U15H_EINVAL;
  }
  const char* s = name;
  long long li = 0;
  if (!eat_layer(&s, &li)) { return U15H_EINVAL; }
  int e = U15H_UND, w = -1;
  if (eat(&s, "input_layernorm")) {
    w = U15H_NORM_INPUT;          // the layernorms suffix the MODULE
  } else if (eat(&s, "post_attention_layernorm")) {
    w = U15H_NORM_POST;
  } else if (eat(&s, "self_attn.")) {
    // the head norms suffix the TENSOR: q_norm_hw_mot_gen (longest first)
    if (eat(&s, "q_norm_hw")) {
      w = U15H_NORM_Q_HW;
    } else if (eat(&s, "k_norm_hw")) {
      w = U15H_NORM_K_HW;
    } else if (eat(&s, "q_norm")) {
      w = U15H_NORM_Q;
    } else if (eat(&s, "k_norm")) {
      w = U15H_NORM_K;
    } else {
      return U15H_EINVAL;
    }
  } else {
    return U15H_EINVAL;
  }
  if (eat(&s, "_mot_gen")) { e = U15H_GEN; }
  (void)eat(&s, ".weight");
  if (*s != '\0') { return U15H_EINVAL; }
  *layer = (int)li;
  *expert = e;
  *which = w;
  return U15H_OK;
}

u15h_status
u15h_stack_set_norm(u15h_stack* st, int layer, int expert, int which,
                    const u15h_bf16* w)
{
  if (st == nullptr || layer < 0 || layer >= st->n_layers ||
      (expert != U15H_UND && expert != U15H_GEN) || which < 0 ||
      which >= U15H_NNORM || w == nullptr || !aligned16(w)) {
    return U15H_EINVAL;
  }
  st->norm(layer, expert, which) = w;
  return U15H_OK;
}

u15h_status
u15h_stack_bind_norm(u15h_stack* st, const char* name, const u15h_bf16* w)
{
  int l = 0, e = 0, k = 0;
  if (st == nullptr || w == nullptr) { return U15H_EINVAL; }
  u15h_status r = u15h_norm_slot(name, &l, &e, &k);
  if (r != U15H_OK) { return r; }
  return u15h_stack_set_norm(st, l, e, k, w);
}

u15h_status
u15h_stack_check_full(const u15h_stack* st, int need_und, int need_gen,
                      int tier, char* missing, size_t missing_cap)
{
  u15h_status r = u15h_stack_check(st, need_und, need_gen, tier, missing,
                                   missing_cap);
  if (r != U15H_OK) { return r; }
  for (int l = 0; l < st->n_layers; ++l) {
    for (int e = 0; e < 2; ++e) {
      if ((e == U15H_UND && !need_und) || (e == U15H_GEN && !need_gen)) { continue; }
      for (int w = 0; w < U15H_NNORM; ++w) {
        if (st->norm(l, e, w) == nullptr) {
          if (missing != nullptr && missing_cap > 0) {
            std::snprintf(missing, missing_cap, "%s", norm_name(l, w, e).c_str());
          }
          return U15H_EINVAL;
        }
      }
    }
  }
  return U15H_OK;
}

u15h_status
u15h_stack_layer_full(u15h_ctx* ctx, u15h_stream stream, const u15h_stack* st,
                      int layer, const u15h_layer_full_io* io, int M_und,
                      int M_gen, int tier)
{
  if (ctx == nullptr) { return U15H_EINVAL; }
  if (const char* why = check_full_call(st, layer, io, M_und, M_gen, tier)) {
    return u15h::set_error(ctx, U15H_EINVAL, why);
  }
  if (M_und + M_gen == 0) { return u15h::set_error(ctx, U15H_OK, ""); }
  return run_full_layer(ctx, stream, st, layer, io, M_und, M_gen, tier, false, -1);
}

u15h_status
u15h_stack_forward_full(u15h_ctx* ctx, u15h_stream stream, const u15h_stack* st,
                        int first, int count, const u15h_layer_full_io* io,
                        u15h_bf16* const* k_caches, u15h_bf16* const* v_caches,
                        int M_und, int M_gen, int tier)
{
  if (ctx == nullptr) { return U15H_EINVAL; }
  if (st == nullptr || io == nullptr || k_caches == nullptr || v_caches == nullptr) {
    return u15h::set_error(ctx, U15H_EINVAL, "null stack, io or cache array");
  }
  if (count < 1 || first < 0 || (long long)first + count > st->n_layers) {
    return u15h::set_error(ctx, U15H_EINVAL, "layers [first, first + count) outside the stack");
  }
  // every layer's call is checked before the first launch
  for (int i = 0; i < count; ++i) {
    u15h_layer_full_io li = *io;
    li.k_cache = k_caches[i];
    li.v_cache = v_caches[i];
    if (const char* why = check_full_call(st, first + i, &li, M_und, M_gen, tier)) {
      char msg[320];
      std::snprintf(msg, sizeof msg, "layer %d: %s", first + i, why);
      return u15h::set_error(ctx, U15H_EINVAL, msg);
    }
  }
  if (M_und + M_gen == 0) { return u15h::set_error(ctx, U15H_OK, ""); }
  for (int i = 0; i < count; ++i) {
    u15h_layer_full_io li = *io;
    li.k_cache = k_caches[i];
    li.v_cache = v_caches[i];
    const int next = i + 1 < count ? first + i + 1 : -1;
    const u15h_status r =
        run_full_layer(ctx, stream, st, first + i, &li, M_und, M_gen, tier, i > 0, next);
    if (r != U15H_OK) { return r; }
  }
  return U15H_OK;
}

}  // extern "C"
