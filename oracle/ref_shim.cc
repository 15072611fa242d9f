// ref_shim.cc -- TEST INFRASTRUCTURE ONLY.
//
// Exposes the reference's own CPU functions, compiled from
// /root/reference/src/u15-ref.cc where it lies (never copied), under C
// names so the oracle tests can call them through ctypes:
//   u15ref_linear -> u15::ref::linear   (src/u15-ref.h:33-36, u15-ref.cc:33-49)
//   u15ref_silu   -> u15::ref::silu     (src/u15-ref.h:38, u15-ref.cc:51-58)
//   u15ref_rms_norm, u15ref_rope_inv_freq, u15ref_rope_half,
//   u15ref_split_rope_project -> the RoPE/norm helpers (src/u15-ref.h:25-95)
//   u15ref_attention, u15ref_block_causal_mask -> src/u15-ref.h:95-110
//   u15ref_decoder_layer -> u15::ref::decoder_layer (src/u15-ref.h:114-147,
//                           u15-ref.cc:242-311), one expert's whole layer
#include "u15-ref.h"

extern "C" void
u15ref_linear(const float* x, const float* w, const float* b,
              std::size_t rows, std::size_t in_dim, std::size_t out_dim,
              float* out)
{
  u15::ref::linear(x, w, b, rows, in_dim, out_dim, out);
}

extern "C" void
u15ref_silu(float* x, std::size_t n)
{
  u15::ref::silu(x, n);
}

extern "C" void
u15ref_rms_norm(const float* x, const float* w, float eps, std::size_t rows,
                std::size_t dim, float* out)
{
  u15::ref::rms_norm(x, w, eps, rows, dim, out);
}

extern "C" void
u15ref_rope_inv_freq(int dim, double theta, float* out)
{
  const std::vector<float> f = u15::ref::rope_inv_freq(dim, theta);
  for (std::size_t i = 0; i < f.size(); ++i) { out[i] = f[i]; }
}

extern "C" void
u15ref_rope_half(float* x, const float* inv, int dim, double pos)
{
  const std::vector<float> f(inv, inv + dim / 2);
  u15::ref::rope_half_inplace(x, f, dim, pos);
}

extern "C" void
u15ref_split_rope_project(const float* x, const float* w_proj,
                          const float* w_norm, const float* w_norm_hw,
                          const int* pos_t, const int* pos_h,
                          const int* pos_w, std::size_t tokens,
                          std::size_t hidden, int heads, int head_dim,
                          double theta_t, double theta_hw, double eps,
                          float* out)
{
  u15::ref::SplitRopeParams p;
  p.heads = heads;
  p.head_dim = head_dim;
  p.theta_t = theta_t;
  p.theta_hw = theta_hw;
  p.rms_eps = eps;
  const std::vector<int> t(pos_t, pos_t + tokens), h(pos_h, pos_h + tokens),
      w(pos_w, pos_w + tokens);
  u15::ref::split_rope_project(x, w_proj, w_norm, w_norm_hw, t, h, w, tokens,
                               hidden, p, out);
}

extern "C" void
u15ref_attention(const float* q, const float* k, const float* v,
                 const float* mask, std::size_t hq, std::size_t hkv,
                 std::size_t tq, std::size_t tk, std::size_t d, float* out)
{
  u15::ref::attention(q, k, v, mask, hq, hkv, tq, tk, d, out);
}

extern "C" void
u15ref_block_causal_mask(const int* t_index, std::size_t n, float* out)
{
  const std::vector<int> t(t_index, t_index + n);
  const std::vector<float> m = u15::ref::block_causal_mask(t);
  for (std::size_t i = 0; i < m.size(); ++i) { out[i] = m[i]; }
}

// w[13]: input_layernorm, post_attention_layernorm, q, k, v, o, q_norm,
// k_norm, q_norm_hw, k_norm_hw, gate, up, down (LayerWeights' order)
extern "C" void
u15ref_decoder_layer(const float* x, const float* const* w, std::size_t hidden,
                     std::size_t heads, std::size_t kv_heads,
                     std::size_t head_dim, std::size_t inter, double eps,
                     double theta_t, double theta_hw, const int* pos_t,
                     const int* pos_h, const int* pos_w, const float* mask,
                     std::size_t tokens, float* out)
{
  u15::ref::LayerWeights lw;
  lw.input_layernorm = w[0];
  lw.post_attention_layernorm = w[1];
  lw.q_proj = w[2];
  lw.k_proj = w[3];
  lw.v_proj = w[4];
  lw.o_proj = w[5];
  lw.q_norm = w[6];
  lw.k_norm = w[7];
  lw.q_norm_hw = w[8];
  lw.k_norm_hw = w[9];
  lw.gate_proj = w[10];
  lw.up_proj = w[11];
  lw.down_proj = w[12];
  u15::ref::LayerDims d;
  d.hidden = hidden;
  d.heads = heads;
  d.kv_heads = kv_heads;
  d.head_dim = head_dim;
  d.intermediate = inter;
  d.rms_eps = eps;
  d.theta_t = theta_t;
  d.theta_hw = theta_hw;
  const std::vector<int> t(pos_t, pos_t + tokens), h(pos_h, pos_h + tokens),
      ww(pos_w, pos_w + tokens);
  u15::ref::decoder_layer(x, lw, d, t, h, ww, mask, tokens, out);
}
