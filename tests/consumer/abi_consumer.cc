// abi_consumer.cc -- TEST PROGRAM: a C++ caller of include/u15h.h, linked
// against libu15h.so the way a reference build would link it (the
// reference's layer step calling the C ABI in place of MetalOps), with the
// CPU oracle (liboracle.so) as the checker.
//
// It runs, on config 1's split (64 und + 192 gen rows, hidden 4096):
//   1. the grouped call a layer step makes: q, k and v of both experts in
//      ONE u15h_mot_linear launch;
//   2. MetalOps::linear's replacement, u15h_linear, on the o projection of
//      the gen expert;
//   3. the layer stack: all 14 matrices of each of two layers bound by the
//      reference's tensor names, u15h_stack_layer over the four steps;
// and checks sampled rows of every output against the oracle's restatement
// of ref::linear (max-rel <= 1e-2, rel-L2 < 4e-3); then
//   4. the whole layer: the 12 norm vectors bound by their names too, one
//      u15h_stack_layer_full call (both groups, block-causal attention over
//      the layer's cache), checked bit for bit against the same layer made
//      of the public calls (u15h_mot_rms_norm, u15h_mot_linear,
//      u15h_mot_attention_prologue, u15h_attention_token_major,
//      u15h_mot_gate_up_swiglu, u15h_add);
//   5. forward_many's loop: both layers of the stack (the second bound to
//      the first's tensors) in one u15h_stack_forward_full call, checked
//      bit for bit against two u15h_stack_layer_full calls (output and
//      each layer's caches).
// Exit status 0 = pass.
#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "u15h.h"
#include "u15_oracle.h"

namespace {

int g_fail = 0;

void
check(bool ok, const std::string& what)
{
  std::printf("%s %s\n", ok ? "ok  " : "FAIL", what.c_str());
  if (!ok) { ++g_fail; }
}

#define HIP_OK(e)                                                        \
  do {                                                                   \
    hipError_t r_ = (e);                                                 \
    if (r_ != hipSuccess) {                                              \
      std::printf("FAIL %s: %s\n", #e, hipGetErrorString(r_));           \
      std::exit(2);                                                      \
    }                                                                    \
  } while (0)

// Host bf16 bits ~N(0, std), seeded (the reference tests' generator).
std::vector<uint16_t>
randn_bf16(uint32_t seed, size_t n, float stddev)
{
  std::vector<float> f(n);
  u15o_randn_mt(seed, stddev, n, f.data());
  std::vector<uint16_t> b(n);
  u15o_f32_to_bf16_n(f.data(), n, b.data());
  return b;
}

// Host bf16 bits ~N(mean, std): the norm gains.
std::vector<uint16_t>
randn_bf16_mean(uint32_t seed, size_t n, float mean, float stddev)
{
  std::vector<float> f(n);
  u15o_randn_mt(seed, stddev, n, f.data());
  for (float& v : f) { v += mean; }
  std::vector<uint16_t> b(n);
  u15o_f32_to_bf16_n(f.data(), n, b.data());
  return b;
}

struct Dev {
  void* p = nullptr;
  size_t bytes = 0;
  explicit Dev(size_t n) : bytes(n) { HIP_OK(hipMalloc(&p, n)); }
  ~Dev() { (void)hipFree(p); }
  template <class T> T* as() const { return static_cast<T*>(p); }
};

Dev*
upload(const std::vector<uint16_t>& h)
{
  Dev* d = new Dev(h.size() * 2);
  HIP_OK(hipMemcpy(d->p, h.data(), d->bytes, hipMemcpyHostToDevice));
  return d;
}

std::vector<uint16_t>
download(const Dev& d, size_t n)
{
  std::vector<uint16_t> h(n);
  HIP_OK(hipMemcpy(h.data(), d.p, n * 2, hipMemcpyDeviceToHost));
  return h;
}

// Sampled rows of y [M][N] (bf16) against the oracle's linear of x [M][K]
// with the row's expert's weights.
void
check_rows(const std::string& what, const std::vector<uint16_t>& y,
           const std::vector<uint16_t>& x, const std::vector<uint16_t>& w_und,
           const std::vector<uint16_t>& w_gen, int M_und, int M, int K, int N)
{
  const int rows[] = {0, M_und / 2, M_und - 1, M_und, M_und + 77, M - 1};
  std::vector<float> got, exp;
  for (int r : rows) {
    if (r < 0 || r >= M) { continue; }
    const std::vector<uint16_t>& w = r < M_und ? w_und : w_gen;
    std::vector<float> e((size_t)N);
    const int32_t id = r;
    u15o_linear_bf16(x.data(), w.data(), nullptr, &id, 1, (size_t)K, (size_t)N,
                     e.data());
    for (int n = 0; n < N; ++n) {
      got.push_back(u15o_bf16_to_f32(y[(size_t)r * N + n]));
      exp.push_back(e[(size_t)n]);
    }
  }
  const double mr = u15o_max_rel(got.data(), exp.data(), got.size());
  const double rl = u15o_rel_l2(got.data(), exp.data(), got.size());
  char buf[160];
  std::snprintf(buf, sizeof buf, "%s: max-rel %.2e, rel-L2 %.2e", what.c_str(),
                mr, rl);
  check(mr <= 1e-2 && rl < 4e-3, buf);
}

}  // namespace

int
main()
{
  const int Mu = 64, Mg = 192, M = Mu + Mg;
  const int H = 4096, NH = 32, KV = 8, HD = 128, I = 12288;
  u15h_ctx* ctx = nullptr;
  u15h_status st = u15h_create(0, &ctx);
  if (st != U15H_OK) {
    std::printf("FAIL u15h_create: %s\n", u15h_status_str(st));
    return 2;
  }
  check(u15h_abi_version() == U15H_ABI_VERSION, "ABI version");
  hipStream_t stream = nullptr;
  HIP_OK(hipStreamCreate(&stream));

  // ---- weights of one MoT layer, both experts, bf16 ~N(0, 0.02) ----------
  const int Ns[U15H_NPROJ] = {NH * HD, KV * HD, KV * HD, H, I, I, H};
  const int Ks[U15H_NPROJ] = {H, H, H, NH * HD, H, H, I};
  std::vector<uint16_t> wh[2][U15H_NPROJ];
  Dev* wd[2][U15H_NPROJ];
  for (int e = 0; e < 2; ++e) {
    for (int p = 0; p < U15H_NPROJ; ++p) {
      wh[e][p] = randn_bf16(100u + 10u * e + p, (size_t)Ns[p] * Ks[p], 0.02f);
      wd[e][p] = upload(wh[e][p]);
    }
  }
  const std::vector<uint16_t> xh = randn_bf16(7u, (size_t)M * H, 1.0f);
  const std::vector<uint16_t> ah = randn_bf16(8u, (size_t)M * NH * HD, 1.0f);
  const std::vector<uint16_t> x2h = randn_bf16(9u, (size_t)M * H, 1.0f);
  const std::vector<uint16_t> hh = randn_bf16(10u, (size_t)M * I, 1.0f);
  Dev* x = upload(xh);
  Dev* attn = upload(ah);
  Dev* x2 = upload(x2h);
  Dev* h = upload(hh);
  Dev q((size_t)M * NH * HD * 2), k((size_t)M * KV * HD * 2),
      v((size_t)M * KV * HD * 2), o((size_t)M * H * 2), gate((size_t)M * I * 2),
      up((size_t)M * I * 2), down((size_t)M * H * 2);
  auto W = [&](int e, int p) { return wd[e][p]->as<const u15h_bf16>(); };

  // ---- 1. q, k, v of both experts in one grouped launch -----------------
  u15h_mot_proj qkv[3] = {
      {W(0, 0), W(1, 0), nullptr, nullptr, q.as<u15h_bf16>(), NH * HD},
      {W(0, 1), W(1, 1), nullptr, nullptr, k.as<u15h_bf16>(), KV * HD},
      {W(0, 2), W(1, 2), nullptr, nullptr, v.as<u15h_bf16>(), KV * HD}};
  st = u15h_mot_linear(ctx, stream, x->as<u15h_bf16>(), Mu, Mg, H, qkv, 3);
  check(st == U15H_OK, std::string("u15h_mot_linear q|k|v: ") + u15h_last_error(ctx));
  HIP_OK(hipStreamSynchronize(stream));
  check_rows("grouped q", download(q, (size_t)M * NH * HD), xh, wh[0][0], wh[1][0],
             Mu, M, H, NH * HD);
  check_rows("grouped k", download(k, (size_t)M * KV * HD), xh, wh[0][1], wh[1][1],
             Mu, M, H, KV * HD);
  check_rows("grouped v", download(v, (size_t)M * KV * HD), xh, wh[0][2], wh[1][2],
             Mu, M, H, KV * HD);

  // ---- 2. MetalOps::linear's replacement: one expert's o projection -----
  st = u15h_linear(ctx, stream, attn->as<u15h_bf16>(), W(1, 3), nullptr,
                   o.as<u15h_bf16>(), M, NH * HD, H);
  check(st == U15H_OK, "u15h_linear o (gen weights on every row)");
  HIP_OK(hipStreamSynchronize(stream));
  check_rows("linear o", download(o, (size_t)M * H), ah, wh[1][3], wh[1][3], 0, M,
             NH * HD, H);
  // a refused call launches nothing and says why
  st = u15h_linear(ctx, stream, attn->as<u15h_bf16>(), W(1, 3), nullptr,
                   o.as<u15h_bf16>(), M, NH * HD + 4, H);
  check(st == U15H_EINVAL && u15h_last_error(ctx)[0] != '\0',
        std::string("K % 8 != 0 refused: ") + u15h_last_error(ctx));

  // ---- 3. the layer stack, bound by the reference's tensor names -------
  u15h_stack* stk = nullptr;
  check(u15h_stack_create(2, H, NH, KV, HD, I, &stk) == U15H_OK, "stack create");
  static const char* kAttn[4] = {"q", "k", "v", "o"};
  static const char* kMlp[3] = {"gate", "up", "down"};
  // two layers, the second bound to the first's tensors
  for (int layer = 0; layer < 2; ++layer) {
    const std::string pre = "language_model.model.layers." + std::to_string(layer) + ".";
    for (int e = 0; e < 2; ++e) {
      const std::string sfx = e ? "_mot_gen" : "";
      for (int p = 0; p < U15H_NPROJ; ++p) {
        const std::string name =
            p < 4 ? pre + "self_attn." + std::string(kAttn[p]) + "_proj" + sfx + ".weight"
                  : pre + "mlp" + sfx + "." + std::string(kMlp[p - 4]) + "_proj.weight";
        if (u15h_stack_bind(stk, name.c_str(), W(e, p)) != U15H_OK) {
          check(false, "bind " + name);
        }
      }
    }
  }
  char missing[256];
  check(u15h_stack_check(stk, 1, 1, U15H_TIER_BF16, missing, sizeof missing) ==
            U15H_OK, "every matrix bound");
  u15h_layer_io io = {};
  io.x = x->as<u15h_bf16>();
  io.q = q.as<u15h_bf16>();
  io.k = k.as<u15h_bf16>();
  io.v = v.as<u15h_bf16>();
  io.attn = attn->as<u15h_bf16>();
  io.o = o.as<u15h_bf16>();
  io.x2 = x2->as<u15h_bf16>();
  io.gate = gate.as<u15h_bf16>();
  io.up = up.as<u15h_bf16>();
  io.h = h->as<u15h_bf16>();
  io.down = down.as<u15h_bf16>();
  st = u15h_stack_layer(ctx, stream, stk, 0, &io, Mu, Mg, U15H_STEP_ALL,
                        U15H_TIER_BF16, 0);
  check(st == U15H_OK, std::string("u15h_stack_layer: ") + u15h_last_error(ctx));
  HIP_OK(hipStreamSynchronize(stream));
  check_rows("stack o", download(o, (size_t)M * H), ah, wh[0][3], wh[1][3], Mu, M,
             NH * HD, H);
  check_rows("stack gate", download(gate, (size_t)M * I), x2h, wh[0][4], wh[1][4],
             Mu, M, H, I);
  check_rows("stack up", download(up, (size_t)M * I), x2h, wh[0][5], wh[1][5], Mu,
             M, H, I);
  check_rows("stack down", download(down, (size_t)M * H), hh, wh[0][6], wh[1][6],
             Mu, M, I, H);

  // ---- 4. the whole layer: norms bound by name, one call --------------
  static const char* kNorm[U15H_NNORM] = {"input_layernorm", "post_attention_layernorm",
                                          "self_attn.q_norm", "self_attn.k_norm",
                                          "self_attn.q_norm_hw", "self_attn.k_norm_hw"};
  Dev* nd[2][U15H_NNORM];
  for (int e = 0; e < 2; ++e) {
    const std::string sfx = e ? "_mot_gen" : "";
    for (int n = 0; n < U15H_NNORM; ++n) {
      const size_t len = n < 2 ? (size_t)H : (size_t)HD / 2;
      nd[e][n] = upload(randn_bf16_mean(300u + 10u * e + n, len, 1.0f, 0.2f));
      for (int layer = 0; layer < 2; ++layer) {
        const std::string name = "language_model.model.layers." + std::to_string(layer) +
                                 "." + std::string(kNorm[n]) + sfx + ".weight";
        if (u15h_stack_bind_norm(stk, name.c_str(), nd[e][n]->as<const u15h_bf16>()) !=
            U15H_OK) {
          check(false, "bind " + name);
        }
      }
    }
  }
  check(u15h_stack_check_full(stk, 1, 1, U15H_TIER_BF16, missing, sizeof missing) ==
            U15H_OK, "ExpertLayer complete: 13 tensors per expert bound");
  // positions: 64 text tokens, then a 12 x 16 image block on one t
  std::vector<int32_t> pt(M), ph(M), pw(M);
  for (int i = 0; i < M; ++i) {
    pt[i] = i < Mu ? i : Mu;
    ph[i] = i < Mu ? 0 : (i - Mu) / 16;
    pw[i] = i < Mu ? 0 : (i - Mu) % 16;
  }
  std::vector<float> cs((size_t)M * HD), sn((size_t)M * HD);
  check(u15h_build_rope_tables(pt.data(), ph.data(), pw.data(), M, HD, 64, 32, 5.0e6,
                               1.0e4, cs.data(), sn.data()) == U15H_OK, "rope tables");
  Dev csd(cs.size() * 4), snd(sn.size() * 4), tid((size_t)M * 4);
  HIP_OK(hipMemcpy(csd.p, cs.data(), csd.bytes, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(snd.p, sn.data(), snd.bytes, hipMemcpyHostToDevice));
  HIP_OK(hipMemcpy(tid.p, pt.data(), tid.bytes, hipMemcpyHostToDevice));
  Dev xa((size_t)M * H * 2), xb((size_t)M * H * 2), normed((size_t)M * H * 2),
      proj((size_t)M * H * 2), hh2((size_t)M * I * 2),
      kca((size_t)KV * M * HD * 2), vca((size_t)KV * M * HD * 2),
      kcb((size_t)KV * M * HD * 2), vcb((size_t)KV * M * HD * 2);
  HIP_OK(hipMemcpy(xa.p, x->p, xa.bytes, hipMemcpyDeviceToDevice));
  HIP_OK(hipMemcpy(xb.p, x->p, xb.bytes, hipMemcpyDeviceToDevice));
  u15h_layer_full_io fio = {};
  fio.x = xa.as<u15h_bf16>();
  fio.normed = normed.as<u15h_bf16>();
  fio.q = q.as<u15h_bf16>();
  fio.k = k.as<u15h_bf16>();
  fio.v = v.as<u15h_bf16>();
  fio.attn = o.as<u15h_bf16>();
  fio.proj = proj.as<u15h_bf16>();
  fio.h = hh2.as<u15h_bf16>();
  fio.k_cache = kca.as<u15h_bf16>();
  fio.v_cache = vca.as<u15h_bf16>();
  fio.cap = M;
  fio.kv_off = 0;
  fio.kv_len = M;
  fio.mode = 2;
  fio.t_index = tid.as<const int32_t>();
  fio.cos_tab = csd.as<const float>();
  fio.sin_tab = snd.as<const float>();
  fio.d_t = 64;
  fio.d_h = 32;
  fio.eps = 1e-6f;
  st = u15h_stack_layer_full(ctx, stream, stk, 0, &fio, Mu, Mg, U15H_TIER_BF16);
  check(st == U15H_OK, std::string("u15h_stack_layer_full: ") + u15h_last_error(ctx));
  // the same layer from the public calls, on xb and the second cache pair
  auto N = [&](int e, int n) { return nd[e][n]->as<const u15h_bf16>(); };
  bool calls_ok = true;
  auto run = [&](u15h_status r) { calls_ok = calls_ok && r == U15H_OK; };
  run(u15h_mot_rms_norm(ctx, stream, xb.as<u15h_bf16>(), nullptr, Mu, Mg, H, N(0, 0),
                        N(1, 0), 1e-6f, normed.as<u15h_bf16>(), nullptr, nullptr));
  run(u15h_mot_linear(ctx, stream, normed.as<u15h_bf16>(), Mu, Mg, H, qkv, 3));
  const u15h_qk_norm qn[2] = {{N(0, 2), N(0, 4), N(0, 3), N(0, 5)},
                              {N(1, 2), N(1, 4), N(1, 3), N(1, 5)}};
  run(u15h_mot_attention_prologue(ctx, stream, q.as<u15h_bf16>(), k.as<u15h_bf16>(),
                                  v.as<u15h_bf16>(), &qn[0], &qn[1], csd.as<const float>(),
                                  snd.as<const float>(), Mu, Mg, NH, KV, HD, 64, 32, 1e-6f,
                                  kcb.as<u15h_bf16>(), vcb.as<u15h_bf16>(), M, 0));
  run(u15h_attention_token_major(ctx, stream, q.as<u15h_bf16>(), kcb.as<u15h_bf16>(),
                                 vcb.as<u15h_bf16>(), o.as<u15h_bf16>(),
                                 tid.as<const int32_t>(), NH, KV, M, M, HD, M, 0, 2));
  u15h_mot_proj po = {W(0, 3), W(1, 3), nullptr, nullptr, proj.as<u15h_bf16>(), H};
  run(u15h_mot_linear(ctx, stream, o.as<u15h_bf16>(), Mu, Mg, NH * HD, &po, 1));
  run(u15h_mot_rms_norm(ctx, stream, xb.as<u15h_bf16>(), proj.as<u15h_bf16>(), Mu, Mg, H,
                        N(0, 1), N(1, 1), 1e-6f, normed.as<u15h_bf16>(), nullptr, nullptr));
  run(u15h_mot_gate_up_swiglu(ctx, stream, normed.as<u15h_bf16>(), Mu, Mg, H, W(0, 4),
                              W(0, 5), W(1, 4), W(1, 5), hh2.as<u15h_bf16>(), I));
  u15h_mot_proj pd = {W(0, 6), W(1, 6), nullptr, nullptr, proj.as<u15h_bf16>(), H};
  run(u15h_mot_linear(ctx, stream, hh2.as<u15h_bf16>(), Mu, Mg, I, &pd, 1));
  run(u15h_add(ctx, stream, xb.as<u15h_bf16>(), proj.as<u15h_bf16>(), (int64_t)M * H));
  check(calls_ok, std::string("the layer from the public calls: ") + u15h_last_error(ctx));
  HIP_OK(hipStreamSynchronize(stream));
  const std::vector<uint16_t> ya = download(xa, (size_t)M * H);
  const std::vector<uint16_t> yb = download(xb, (size_t)M * H);
  bool finite = true;
  for (uint16_t b : ya) { finite = finite && (b & 0x7f80u) != 0x7f80u; }
  check(finite && ya != xh, "whole layer: finite output that differs from its input");
  check(ya == yb && download(kca, kca.bytes / 2) == download(kcb, kcb.bytes / 2) &&
            download(vca, vca.bytes / 2) == download(vcb, vcb.bytes / 2),
        "whole layer: bit-equal to the public calls (output and both caches)");

  // ---- 5. both layers in one call: forward_many's loop -----------------
  Dev xc((size_t)M * H * 2), xd((size_t)M * H * 2);
  HIP_OK(hipMemcpy(xc.p, x->p, xc.bytes, hipMemcpyDeviceToDevice));
  HIP_OK(hipMemcpy(xd.p, x->p, xd.bytes, hipMemcpyDeviceToDevice));
  Dev* kv2[4][2];
  for (auto& pair : kv2) {
    for (Dev*& d : pair) { d = new Dev((size_t)KV * M * HD * 2); }
  }
  u15h_bf16* kf[2] = {kv2[0][0]->as<u15h_bf16>(), kv2[1][0]->as<u15h_bf16>()};
  u15h_bf16* vf[2] = {kv2[0][1]->as<u15h_bf16>(), kv2[1][1]->as<u15h_bf16>()};
  fio.x = xc.as<u15h_bf16>();
  st = u15h_stack_forward_full(ctx, stream, stk, 0, 2, &fio, kf, vf, Mu, Mg,
                               U15H_TIER_BF16);
  check(st == U15H_OK, std::string("u15h_stack_forward_full: ") + u15h_last_error(ctx));
  fio.x = xd.as<u15h_bf16>();
  for (int layer = 0; layer < 2; ++layer) {
    fio.k_cache = kv2[2 + layer][0]->as<u15h_bf16>();
    fio.v_cache = kv2[2 + layer][1]->as<u15h_bf16>();
    run(u15h_stack_layer_full(ctx, stream, stk, layer, &fio, Mu, Mg, U15H_TIER_BF16));
  }
  check(calls_ok, std::string("two u15h_stack_layer_full calls: ") + u15h_last_error(ctx));
  HIP_OK(hipStreamSynchronize(stream));
  bool caches_equal = true;
  for (int layer = 0; layer < 2; ++layer) {
    for (int c = 0; c < 2; ++c) {
      caches_equal = caches_equal &&
                     download(*kv2[layer][c], kv2[layer][c]->bytes / 2) ==
                         download(*kv2[2 + layer][c], kv2[2 + layer][c]->bytes / 2);
    }
  }
  const std::vector<uint16_t> yc = download(xc, (size_t)M * H);
  check(yc != ya && yc == download(xd, (size_t)M * H) && caches_equal,
        "two layers in one forward_full call: bit-equal to the per-layer calls");
  for (auto& pair : kv2) {
    for (Dev* d : pair) { delete d; }
  }
  for (auto& row : nd) {
    for (Dev* d : row) { delete d; }
  }
  u15h_stack_destroy(stk);

  for (auto& row : wd) {
    for (Dev* d : row) { delete d; }
  }
  delete x;
  delete attn;
  delete x2;
  delete h;
  HIP_OK(hipStreamDestroy(stream));
  u15h_destroy(ctx);
  std::printf("%s (%d failed)\n", g_fail == 0 ? "PASS" : "FAIL", g_fail);
  return g_fail == 0 ? 0 : 1;
}
