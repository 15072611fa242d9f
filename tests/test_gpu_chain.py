"""The attention half of a MoT layer, chained on the GPU and checked against
the compiled reference.

The chain is the projection half of U15Backbone::layer_step_'s attention
block (src/u15-backbone.cc:193-243) with both experts in each launch:
x -> grouped q|k|v -> split q/k norm + three-way RoPE per expert group
(u15h_split_qk_norm_rope) -> k, v into a head-major cache whose stride is
its capacity (u15h_transpose_into_cache) -> bidirectional GQA attention
over the cache, token-major (u15h_attention_token_major) -> grouped o.
The norm, RoPE and cache steps run either as those calls or as the one
launch that replaces them (u15h_mot_attention_prologue).

The reference runs the same layer half in f32 from the same bf16 inputs:
u15::ref::split_rope_project for q and k, ref::linear for v, ref::attention
and ref::linear for o (src/u15-ref.cc:121-175, 194-236, 33-49), each
expert's rows with that expert's weights.  Bar: the reference's layer test,
rel-L2 < 2e-2 (tests/u15-layer0-test.cc:293-299), and max-rel <= 1e-2.
Negative control: the same chain against a reference whose o projection
takes the other expert's weights must miss the bar.

Split: config 1's 64 understanding + 192 generated-image tokens (a 12 x 16
patch grid sharing one temporal position after 64 text positions).
"""
import numpy as np
import pytest
import torch

import oracle
import u15h
from helpers import host_bits, host_f32, max_rel, rel_l2

pytestmark = pytest.mark.gpu

HID, NH, KV, HD = 4096, 32, 8, 128
D_T, D_H = HD // 2, HD // 4


def _bf16(g, shape, std=1.0, mean=0.0):
    return (torch.randn(*shape, generator=g, device="cuda") * std + mean).to(torch.bfloat16)


def _f32(t):
    return oracle.bf16_to_f32(host_bits(t))


@pytest.mark.parametrize("prologue", ["calls", "fused"])
def test_attention_half_chain_vs_reference(ops, prologue):
    if oracle.ref_lib() is None:
        pytest.skip("the compiled reference (oracle/_ref) is not built")
    Mu, Mg = 64, 192
    T = Mu + Mg
    g = torch.Generator(device="cuda").manual_seed(2193)
    x = _bf16(g, (T, HID))
    W = {}
    for e in ("und", "gen"):
        W[e] = dict(q=_bf16(g, (NH * HD, HID), 0.02), k=_bf16(g, (KV * HD, HID), 0.02),
                    v=_bf16(g, (KV * HD, HID), 0.02), o=_bf16(g, (HID, NH * HD), 0.02),
                    qn_t=_bf16(g, (HD // 2,), 0.2, 1.0), qn_hw=_bf16(g, (HD // 2,), 0.2, 1.0),
                    kn_t=_bf16(g, (HD // 2,), 0.2, 1.0), kn_hw=_bf16(g, (HD // 2,), 0.2, 1.0))
    pos_t = np.array(list(range(Mu)) + [Mu] * Mg, np.int32)
    pos_h = np.array([0] * Mu + [i // 16 for i in range(Mg)], np.int32)
    pos_w = np.array([0] * Mu + [i % 16 for i in range(Mg)], np.int32)
    groups = (("und", slice(0, Mu)), ("gen", slice(Mu, T)))

    # ---- the chain on the GPU ------------------------------------------------
    q = torch.empty(T, NH * HD, dtype=torch.bfloat16, device="cuda")
    k = torch.empty(T, KV * HD, dtype=torch.bfloat16, device="cuda")
    v = torch.empty(T, KV * HD, dtype=torch.bfloat16, device="cuda")
    ops.mot_linear(x, Mu, Mg, HID, [dict(w_und=W["und"][n], w_gen=W["gen"][n], y=y)
                                    for n, y in (("q", q), ("k", k), ("v", v))])
    cs, sn = (torch.from_numpy(a).cuda() for a in
              u15h.build_rope_tables(pos_t, pos_h, pos_w, HD, D_T, D_H))
    cap = T + 40                    # the cache stride is its capacity, not T
    kc = torch.full((KV, cap, HD), float("nan"), dtype=torch.bfloat16, device="cuda")
    vc = torch.full((KV, cap, HD), float("nan"), dtype=torch.bfloat16, device="cuda")
    if prologue == "calls":
        for e, r in groups:
            ops.split_qk_norm_rope(q[r], W[e]["qn_t"], W[e]["qn_hw"], cs[r], sn[r],
                                   NH, HD, D_T, D_H)
            ops.split_qk_norm_rope(k[r], W[e]["kn_t"], W[e]["kn_hw"], cs[r], sn[r],
                                   KV, HD, D_T, D_H)
        ops.transpose_into_cache(k, kc, T, KV, HD, 0)
        ops.transpose_into_cache(v, vc, T, KV, HD, 0)
    else:
        norms = {e: dict(q_t=W[e]["qn_t"], q_hw=W[e]["qn_hw"],
                         k_t=W[e]["kn_t"], k_hw=W[e]["kn_hw"]) for e in ("und", "gen")}
        ops.mot_attention_prologue(q, k, v, norms["und"], norms["gen"], cs, sn,
                                   Mu, Mg, NH, KV, HD, D_T, D_H, kc, vc)
    attn = torch.empty(T, NH * HD, dtype=torch.bfloat16, device="cuda")
    ops.attention_token_major(q, kc, vc, attn, NH, KV, T, mode=0)
    o = torch.empty(T, HID, dtype=torch.bfloat16, device="cuda")
    ops.mot_linear(attn, Mu, Mg, NH * HD, [dict(w_und=W["und"]["o"],
                                                w_gen=W["gen"]["o"], y=o)])
    torch.cuda.synchronize()
    got = host_f32(o)
    assert np.all(np.isfinite(got))

    # ---- the reference, f32 from the same bf16 values ---------------------------
    xf = _f32(x)
    Q = np.empty((NH, T, HD), np.float32)
    K = np.empty((KV, T, HD), np.float32)
    V = np.empty((KV, T, HD), np.float32)
    for e, r in groups:
        w = {n: _f32(t) for n, t in W[e].items()}
        Q[:, r] = oracle.ref_split_rope_project(xf[r], w["q"], w["qn_t"], w["qn_hw"],
                                                pos_t[r], pos_h[r], pos_w[r], NH, HD)
        K[:, r] = oracle.ref_split_rope_project(xf[r], w["k"], w["kn_t"], w["kn_hw"],
                                                pos_t[r], pos_h[r], pos_w[r], KV, HD)
        vv = oracle.ref_linear(xf[r], w["v"])                     # [t][KV*HD]
        V[:, r] = vv.reshape(-1, KV, HD).transpose(1, 0, 2)
    A = oracle.ref_attention(Q, K, V, None, KV)                  # [T][NH*HD]
    ref = np.empty((T, HID), np.float32)
    bad = np.empty((T, HID), np.float32)
    for (e, r), other in zip(groups, ("gen", "und")):
        ref[r] = oracle.ref_linear(A[r], _f32(W[e]["o"]))
        bad[r] = oracle.ref_linear(A[r], _f32(W[other]["o"]))
    assert rel_l2(got, ref) < 2e-2
    assert max_rel(got, ref) <= 1e-2
    # the expert routing of the o projection is load-bearing
    assert rel_l2(got, bad) > 2e-2
