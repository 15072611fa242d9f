"""The attention prologue in one launch (u15h_mot_attention_prologue)
against the separate calls it replaces.

U15Backbone::layer_step_ runs, after the q, k, v projections,
split_qk_norm and split_rope on q and on k, then transpose_into_cache of k
and v (src/u15-backbone.cc:203-216).  Here those are u15h_split_qk_norm_rope
on q and k per expert group (und rows with the base norm weights, gen rows
with the _mot_gen ones) and u15h_transpose_into_cache of k and v; the fused
launch must give the same bits: q in place, both caches (including every
slot it must not touch, NaN-filled beforehand), and k and v unchanged.  The
separate calls are pinned against the compiled reference by
tests/test_gpu_rope.py and tests/test_gpu_chain.py, which also runs the
chain through the fused launch.
"""
import numpy as np
import pytest
import torch

import u15h
from helpers import host_bits

pytestmark = pytest.mark.gpu


def _bf16(g, shape, std=1.0, mean=0.0):
    return (torch.randn(*shape, generator=g, device="cuda") * std + mean).to(torch.bfloat16)


def _norms(g, d):
    return {f: _bf16(g, (d // 2,), 0.2, 1.0) for f in ("q_t", "q_hw", "k_t", "k_hw")}


def _tables(T, d, d_t, d_h, Mu):
    pos_t = np.array(list(range(Mu)) + [Mu] * (T - Mu), np.int32)
    pos_h = np.array([0] * Mu + [i // 16 for i in range(T - Mu)], np.int32)
    pos_w = np.array([0] * Mu + [i % 16 for i in range(T - Mu)], np.int32)
    return [torch.from_numpy(a).cuda() for a in
            u15h.build_rope_tables(pos_t, pos_h, pos_w, d, d_t, d_h)]


# (M_und, M_gen, hq, hkv, d, d_t, d_h, cap extra, offset)
CASES = [
    (64, 192, 32, 8, 128, 64, 32, 40, 0),        # config 1's split
    (128, 4096, 32, 8, 128, 64, 32, 0, 0),       # config 2
    (128, 1024, 32, 8, 128, 64, 32, 77, 128),    # after a 128-token prefix
    (0, 100, 32, 8, 128, 64, 32, 13, 5),         # gen rows only, ragged
    (37, 0, 32, 8, 128, 64, 32, 3, 0),           # und rows only, ragged
    (20, 45, 16, 2, 64, 32, 16, 9, 17),          # another head shape
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{c[0]}+{c[1]}_h{c[2]}x{c[3]}_d{c[4]}_o{c[8]}")
def test_prologue_bit_equal_to_the_separate_calls(ops, case):
    Mu, Mg, HQ, KV, D, D_T, D_H, extra, off = case
    T = Mu + Mg
    cap = off + T + extra
    g = torch.Generator(device="cuda").manual_seed(sum(case))
    q = _bf16(g, (T, HQ * D))
    k = _bf16(g, (T, KV * D))
    v = _bf16(g, (T, KV * D))
    W = {"und": _norms(g, D), "gen": _norms(g, D)}
    cs, sn = _tables(T, D, D_T, D_H, Mu)
    k_in, v_in = host_bits(k), host_bits(v)

    # the separate calls
    q1, k1 = q.clone(), k.clone()
    for e, r in (("und", slice(0, Mu)), ("gen", slice(Mu, T))):
        if r.start == r.stop:
            continue
        w = W[e]
        ops.split_qk_norm_rope(q1[r], w["q_t"], w["q_hw"], cs[r], sn[r], HQ, D, D_T, D_H)
        ops.split_qk_norm_rope(k1[r], w["k_t"], w["k_hw"], cs[r], sn[r], KV, D, D_T, D_H)
    kc1 = torch.full((KV, cap, D), float("nan"), dtype=torch.bfloat16, device="cuda")
    vc1 = torch.full((KV, cap, D), float("nan"), dtype=torch.bfloat16, device="cuda")
    ops.transpose_into_cache(k1, kc1, T, KV, D, off)
    ops.transpose_into_cache(v, vc1, T, KV, D, off)

    # one launch
    q2 = q.clone()
    kc2 = torch.full((KV, cap, D), float("nan"), dtype=torch.bfloat16, device="cuda")
    vc2 = torch.full((KV, cap, D), float("nan"), dtype=torch.bfloat16, device="cuda")
    ops.mot_attention_prologue(q2, k, v, W["und"] if Mu else None,
                               W["gen"] if Mg else None, cs, sn, Mu, Mg, HQ, KV,
                               D, D_T, D_H, kc2, vc2, offset=off)
    torch.cuda.synchronize()

    assert np.array_equal(host_bits(q2), host_bits(q1))
    assert np.array_equal(host_bits(kc2), host_bits(kc1))
    assert np.array_equal(host_bits(vc2), host_bits(vc1))
    assert np.array_equal(host_bits(k), k_in) and np.array_equal(host_bits(v), v_in)
    # the slots outside [off, off + T) are untouched
    kb = host_bits(kc2)
    outside = np.ones(cap, bool)
    outside[off:off + T] = False
    nan_bits = host_bits(torch.full((1,), float("nan"), dtype=torch.bfloat16))[0]
    assert np.all(kb[:, outside] == nan_bits)
    assert np.all(host_bits(vc2)[:, outside] == nan_bits)
    # and the norm weights are routed: the other expert's give other bits
    if Mu and Mg:
        q3 = q.clone()
        kc3 = torch.zeros_like(kc2)
        vc3 = torch.zeros_like(vc2)
        ops.mot_attention_prologue(q3, k, v, W["gen"], W["und"], cs, sn, Mu, Mg,
                                   HQ, KV, D, D_T, D_H, kc3, vc3, offset=off)
        torch.cuda.synchronize()
        assert not np.array_equal(host_bits(q3), host_bits(q1))


def test_prologue_refusals_launch_nothing(ops):
    T, HQ, KV, D = 64, 32, 8, 128
    g = torch.Generator(device="cuda").manual_seed(5)
    q = _bf16(g, (T, HQ * D))
    k = _bf16(g, (T, KV * D))
    v = _bf16(g, (T, KV * D))
    W = _norms(g, D)
    cs, sn = _tables(T, D, 64, 32, T)
    q0 = host_bits(q)
    kc = torch.zeros(KV, T, D, dtype=torch.bfloat16, device="cuda")
    vc = torch.zeros(KV, T, D, dtype=torch.bfloat16, device="cuda")
    # offset + T past the capacity
    with pytest.raises(u15h.U15hError, match="capacity"):
        ops.mot_attention_prologue(q, k, v, W, None, cs, sn, T, 0, HQ, KV, D,
                                   64, 32, kc, vc, offset=1)
    # ranges the one-launch kernel does not take (d_t = 48: not a power of two x 16)
    with pytest.raises(u15h.U15hError, match="separate calls"):
        ops.mot_attention_prologue(q, k, v, W, None, cs, sn, T, 0, HQ, KV, D,
                                   48, 40, kc, vc)
    # a group with rows needs its norm weights
    with pytest.raises(ValueError, match="gen"):
        ops.mot_attention_prologue(q, k, v, W, None, cs, sn, 32, 32, HQ, KV, D,
                                   64, 32, kc, vc)
    torch.cuda.synchronize()
    assert np.array_equal(host_bits(q), q0)
    assert not torch.any(kc.view(torch.int16) != 0).item()
    assert not torch.any(vc.view(torch.int16) != 0).item()
