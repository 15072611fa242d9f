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
#include <string>
#include <vector>

#include "u15h_internal.h"

struct u15h_stack {
  int n_layers = 0;
  int hidden = 0, qdim = 0, kvdim = 0, inter = 0;
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
  st->slots.resize((size_t)n_layers * 2 * U15H_NPROJ);
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
  if (!eat(&s, "language_model.model.layers.")) { return U15H_EINVAL; }
  // A decimal layer index as std::to_string writes it: no sign, no
  // leading zero (except "0"), at most 9 digits.
  if (*s < '0' || *s > '9' || (s[0] == '0' && s[1] >= '0' && s[1] <= '9')) {
    return U15H_EINVAL;
  }
  long long li = 0;
  int nd = 0;
  while (*s >= '0' && *s <= '9') {
    li = li * 10 + (*s - '0');
    ++s;
    if (++nd > 9) { return U15H_EINVAL; }
  }
  if (!eat(&s, ".")) { return U15H_EINVAL; }
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

}  // extern "C"
