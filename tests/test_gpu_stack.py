"""GPU parity of the resident layer stack and of every BASELINE config's
launches, through the C ABI.

  * The stack (u15h_stack_layer / u15h_stack_forward) with weights bound by
    the reference's tensor names: a reduced-depth config-5 stack (3 layers
    x 2 weight sets at 128 + 4096 rows) and the 128 + 1024 point, each
    layer's seven outputs sampled against the oracle with that layer's
    weights; the int8 tier bit-exact against the oracle's quantise ->
    int32 GEMM -> dequant on sampled rows.
  * Config 4 (4352 und + 12288 gen): bf16 sampled rows; int8 accumulators
    exact in every row sum and column sum of all four launches, plus
    sampled rows in full.
  * Config 2's launches not covered elsewhere: grouped gate|up (N = 2 x
    12288) at 4224 rows in bf16 and int8, int8 down at K = 12288.
  * The MLP chain gate|up -> SwiGLU -> down against the compiled
    reference's linear and silu composed as u15::ref::decoder_layer does
    (src/u15-ref.cc:294-310; bar of tests/u15-layer0-test.cc:299).

Bars: bf16 max-rel-err <= 1e-2 and rel-L2 < 4e-3 per output (the
reference's kernel-test bar, tests/u15-kernels-test.cc:55); int8 int32
accumulators and the dequantised bf16 BIT-EXACT.
"""
import numpy as np
import pytest
import torch

import oracle
import u15h
from helpers import host_bits, host_f32, max_rel, rel_l2

pytestmark = pytest.mark.gpu

H, I, NQ, NKV = 4096, 12288, 4096, 1024
MAX_REL, KERNEL_BAR = 1e-2, 4e-3


def _gen(seed):
    return torch.Generator(device="cuda").manual_seed(seed)


def _act(g, M, K):
    return torch.randn(M, K, generator=g, device="cuda").to(torch.bfloat16)


def _weights(g, n_layers, stack, want_i8, ops):
    """Random bf16 weights ~N(0, 0.02) for every slot, bound by name."""
    W = {}
    for layer in range(n_layers):
        for e in (u15h.UND, u15h.GEN):
            for p in range(7):
                N, K = stack.shape(p)
                w = (torch.randn(N, K, generator=g, device="cuda") * 0.02).to(torch.bfloat16)
                name = u15h.slot_name(layer, e, p)
                stack.bind(name, w)
                if want_i8:
                    wq = torch.empty(N, K, dtype=torch.int8, device="cuda")
                    sw = torch.empty(N, dtype=torch.float32, device="cuda")
                    ops.quant_rows_i8(w, wq, sw)
                    stack.bind_i8(name, wq, sw)
                    W[(layer, e, p)] = (w, wq, sw)
                else:
                    W[(layer, e, p)] = (w, None, None)
    return W


def _io(g, M):
    t = dict(x=_act(g, M, H), attn=_act(g, M, NQ), x2=_act(g, M, H),
             h=_act(g, M, I))
    for name, n in (("q", NQ), ("k", NKV), ("v", NKV), ("o", H),
                    ("gate", I), ("up", I), ("down", H)):
        t[name] = torch.full((M, n), float("nan"), dtype=torch.bfloat16, device="cuda")
    t["xq"] = torch.empty(M, I, dtype=torch.int8, device="cuda")
    t["sx"] = torch.empty(M, dtype=torch.float32, device="cuda")
    return t


# (output, input, projection) of the four steps
OUTS = (("q", "x", 0), ("k", "x", 1), ("v", "x", 2), ("o", "attn", 3),
        ("gate", "x2", 4), ("up", "x2", 5), ("down", "h", 6))


def _rows(Mu, Mg):
    M = Mu + Mg
    r = [0, Mu // 2, Mu - 1, Mu, Mu + Mg // 3, M - 1] if Mu else [0, Mg // 2, M - 1]
    return np.unique(np.array([x for x in r if 0 <= x < M], np.int32))


def _check_bf16_layer(t, W, layer, Mu, Mg, rows):
    """Sampled rows of each output against the oracle's linear with the
    row's expert's weights of `layer`."""
    for out, inp, p in OUTS:
        xb = host_bits(t[inp])
        got = host_f32(t[out])[rows]
        assert np.all(np.isfinite(got)), out
        exp = np.empty_like(got)
        for e, sel in ((u15h.UND, rows < Mu), (u15h.GEN, rows >= Mu)):
            if not sel.any():
                continue
            wb = host_bits(W[(layer, e, p)][0])
            exp[sel] = oracle.linear_bf16(xb, wb, row_ids=rows[sel])
        assert max_rel(got, exp) <= MAX_REL, (layer, out)
        assert rel_l2(got, exp) < KERNEL_BAR, (layer, out)


def _check_i8_layer(t, W, layer, Mu, Mg, rows):
    """The int8 tier's bf16 outputs on sampled rows, bit-exact against the
    oracle's quantise -> exact int32 GEMM -> dequant with the device's
    weight codes (themselves checked against the oracle's quantiser)."""
    for out, inp, p in OUTS:
        xb = host_bits(t[inp])
        xq, sx = oracle.quant_rows_i8(xb[rows])
        got = host_bits(t[out])[rows]
        for e, sel in ((u15h.UND, rows < Mu), (u15h.GEN, rows >= Mu)):
            if not sel.any():
                continue
            w, wq, sw = W[(layer, e, p)]
            wq_h, sw_h = wq.cpu().numpy(), sw.cpu().numpy()
            qo, so = oracle.quant_rows_i8(host_bits(w[::97]))
            assert np.array_equal(wq_h[::97], qo) and np.array_equal(sw_h[::97], so)
            acc = oracle.gemm_i8_i32(xq[sel], wq_h)
            exp = oracle.dequant_bf16(acc, sx[sel], sw_h)
            assert np.array_equal(got[sel], exp), (layer, out, e)


def test_stack_reduced_depth_bf16(ops):
    """A 3-layer stack (6 weight sets) at config 5's 128 + 4096 rows: each
    layer's outputs through u15h_stack_layer, then one u15h_stack_forward
    pass, whose outputs are the last layer's bit for bit."""
    Mu, Mg, L = 128, 4096, 3
    g = _gen(300)
    st = u15h.Stack(L)
    W = _weights(g, L, st, False, ops)
    assert st.check() is None
    t = _io(g, Mu + Mg)
    io = u15h.layer_io(**t)
    rows = _rows(Mu, Mg)
    per_layer = []
    for layer in range(L):
        ops.stack_layer(st, layer, io, Mu, Mg)
        torch.cuda.synchronize()
        _check_bf16_layer(t, W, layer, Mu, Mg, rows)
        per_layer.append({k: t[k].clone() for k, _, _ in OUTS})
    for k, _, _ in OUTS:
        t[k].fill_(float("nan"))
    ops.stack_forward(st, io, Mu, Mg)
    torch.cuda.synchronize()
    for k, _, _ in OUTS:
        assert torch.equal(t[k].view(torch.int16), per_layer[-1][k].view(torch.int16)), k
        # the layers' weights really differ: layer 1's output is not layer 2's
        assert not torch.equal(per_layer[1][k].view(torch.int16),
                               per_layer[2][k].view(torch.int16)), k
    st.close()


def test_stack_exchange_control(ops):
    """Binding the gen matrices into the und slots (and the reverse) must
    change the result: both weight sets are really in use, row by group
    (the reference's expert-gap check, tests/u15-ref-test.cc:321-332)."""
    Mu, Mg = 64, 192
    g = _gen(301)
    st = u15h.Stack(1)
    W = _weights(g, 1, st, False, ops)
    t = _io(g, Mu + Mg)
    io = u15h.layer_io(**t)
    ops.stack_layer(st, 0, io, Mu, Mg, steps=u15h.STEP_QKV)
    torch.cuda.synchronize()
    good = t["q"].clone()
    for p in range(7):
        st.bind(u15h.slot_name(0, u15h.UND, p), W[(0, u15h.GEN, p)][0])
        st.bind(u15h.slot_name(0, u15h.GEN, p), W[(0, u15h.UND, p)][0])
    ops.stack_layer(st, 0, io, Mu, Mg, steps=u15h.STEP_QKV)
    torch.cuda.synchronize()
    swapped = t["q"]
    assert not torch.equal(good[:Mu], swapped[:Mu])
    assert not torch.equal(good[Mu:], swapped[Mu:])
    # a refused call (int8 tier with nothing int8 bound) launches nothing
    t["q"].fill_(0.0)
    with pytest.raises(u15h.U15hError):
        ops.stack_layer(st, 0, io, Mu, Mg, steps=u15h.STEP_QKV, tier=u15h.TIER_I8)
    torch.cuda.synchronize()
    assert int(torch.count_nonzero(t["q"].float())) == 0
    st.close()


def test_stack_reduced_depth_int8(ops):
    """The int8 tier of a 3-layer stack at 128 + 4096 rows: every layer's
    seven outputs bit-exact on sampled rows."""
    Mu, Mg, L = 128, 4096, 3
    g = _gen(302)
    st = u15h.Stack(L)
    W = _weights(g, L, st, True, ops)
    assert st.check(tier=u15h.TIER_I8) is None
    t = _io(g, Mu + Mg)
    io = u15h.layer_io(**t)
    rows = _rows(Mu, Mg)
    for layer in range(L):
        ops.stack_layer(st, layer, io, Mu, Mg, tier=u15h.TIER_I8)
        torch.cuda.synchronize()
        _check_i8_layer(t, W, layer, Mu, Mg, rows)
    ops.stack_forward(st, io, Mu, Mg, tier=u15h.TIER_I8)
    torch.cuda.synchronize()
    _check_i8_layer(t, W, L - 1, Mu, Mg, rows)
    st.close()


def test_stack_small_m_point(ops):
    """Config 5's second point, 128 + 1024 rows, both tiers, and the fused
    SwiGLU form of the gate|up step (h = silu(gate) * up, bit-equal to the
    unfused GEMMs followed by u15h_swiglu)."""
    Mu, Mg = 128, 1024
    g = _gen(303)
    st = u15h.Stack(2)
    W = _weights(g, 2, st, True, ops)
    t = _io(g, Mu + Mg)
    io = u15h.layer_io(**t)
    rows = _rows(Mu, Mg)
    ops.stack_forward(st, io, Mu, Mg)
    torch.cuda.synchronize()
    _check_bf16_layer(t, W, 1, Mu, Mg, rows)
    ops.stack_forward(st, io, Mu, Mg, tier=u15h.TIER_I8)
    torch.cuda.synchronize()
    _check_i8_layer(t, W, 1, Mu, Mg, rows)
    # fused SwiGLU: compare with the unfused sequence
    ops.stack_layer(st, 0, io, Mu, Mg, steps=u15h.STEP_GATE_UP)
    h_ref = torch.empty_like(t["h"])
    ops.swiglu(t["gate"], t["up"], h_ref)
    h_in = t["h"].clone()
    ops.stack_layer(st, 0, io, Mu, Mg, steps=u15h.STEP_GATE_UP,
                    flags=u15h.FUSED_SWIGLU)
    torch.cuda.synchronize()
    assert torch.equal(t["h"].view(torch.int16), h_ref.view(torch.int16))
    assert not torch.equal(t["h"], h_in)
    st.close()


def test_c4_bf16(ops):
    """Config 4: 4352 und + 12288 gen rows (edit + CFG), one layer's seven
    projections through the stack, sampled rows against the oracle."""
    Mu, Mg = 4352, 12288
    g = _gen(304)
    st = u15h.Stack(1)
    W = _weights(g, 1, st, False, ops)
    t = _io(g, Mu + Mg)
    io = u15h.layer_io(**t)
    ops.stack_layer(st, 0, io, Mu, Mg)
    torch.cuda.synchronize()
    rows = np.array([0, 255, 256, 4351, 4352, 8000, 16383, 16639], np.int32)
    _check_bf16_layer(t, W, 0, Mu, Mg, rows)
    st.close()


def _i8_exact(xq_h, Mu, accs, wqs):
    """Every row sum and column sum of each launch's int32 accumulators,
    per group, against exact integer identities; then sampled rows."""
    M = xq_h.shape[0]
    for acc, (wq_u, wq_g) in zip(accs, wqs):
        for lo, hi, wq in ((0, Mu, wq_u), (Mu, M, wq_g)):
            if hi <= lo:
                continue
            a = acc[lo:hi]
            rs, cs = oracle.i8_product_sums(xq_h[lo:hi], wq)
            assert np.array_equal(a.sum(axis=1, dtype=np.int64), rs)
            assert np.array_equal(a.sum(axis=0, dtype=np.int64), cs)
        for r in (0, Mu - 1, Mu, M - 1):
            if 0 <= r < M:
                wq = wq_u if r < Mu else wq_g
                assert np.array_equal(acc[r:r + 1], oracle.gemm_i8_i32(xq_h[r:r + 1], wq))


def _i8_launches(ops, g, Mu, Mg, launches):
    """Random int8 codes for each launch's input and weights, the raw int32
    grouped GEMM, and the exact checks.  launches: (K, [N, ...])."""
    M = Mu + Mg
    for K, Ns in launches:
        xq = torch.randint(-127, 128, (M, K), generator=g, device="cuda", dtype=torch.int8)
        accs, wqs, projs = [], [], []
        for N in Ns:
            wu = torch.randint(-127, 128, (N, K), generator=g, device="cuda", dtype=torch.int8)
            wg = torch.randint(-127, 128, (N, K), generator=g, device="cuda", dtype=torch.int8)
            y = torch.empty(M, N, dtype=torch.int32, device="cuda")
            projs.append(dict(wq_und=wu, wq_gen=wg, y=y))
            wqs.append((wu.cpu().numpy(), wg.cpu().numpy()))
        ops.mot_gemm_i8_i32(xq, Mu, Mg, K, projs)
        torch.cuda.synchronize()
        accs = [p["y"].cpu().numpy() for p in projs]
        _i8_exact(xq.cpu().numpy(), Mu, accs, wqs)
        del projs, accs


def test_c4_int8_exact(ops):
    """Config 4 in the int8 tier: the four launches' raw int32 accumulators
    (q|k|v, o, gate|up, down) exact in every row and column sum, sampled
    rows in full; then the stack's int8 tier bit-exact on sampled rows."""
    Mu, Mg = 4352, 12288
    g = _gen(305)
    _i8_launches(ops, g, Mu, Mg, [(H, [NQ, NKV, NKV]), (NQ, [H]), (H, [I, I]), (I, [H])])
    st = u15h.Stack(1)
    W = _weights(g, 1, st, True, ops)
    t = _io(g, Mu + Mg)
    io = u15h.layer_io(**t)
    ops.stack_layer(st, 0, io, Mu, Mg, tier=u15h.TIER_I8)
    torch.cuda.synchronize()
    _check_i8_layer(t, W, 0, Mu, Mg, np.array([0, 4351, 4352, 16639], np.int32))
    st.close()


def test_c2_gate_up_grouped(ops):
    """Config 2's gate|up as one grouped launch (two projections of N =
    12288 over both weight sets, 4224 rows): bf16 sampled rows against the
    oracle; int8 accumulators exact."""
    Mu, Mg = 128, 4096
    g = _gen(306)
    x = _act(g, Mu + Mg, H)
    ws = {(e, n): (torch.randn(I, H, generator=g, device="cuda") * 0.02).to(torch.bfloat16)
          for e in ("und", "gen") for n in ("gate", "up")}
    ys = {n: torch.empty(Mu + Mg, I, dtype=torch.bfloat16, device="cuda") for n in ("gate", "up")}
    ops.mot_linear(x, Mu, Mg, H, [dict(w_und=ws[("und", n)], w_gen=ws[("gen", n)], y=ys[n])
                                  for n in ("gate", "up")])
    torch.cuda.synchronize()
    rows = _rows(Mu, Mg)
    xb = host_bits(x)
    for n in ("gate", "up"):
        got = host_f32(ys[n])[rows]
        exp = np.empty_like(got)
        for e, sel in (("und", rows < Mu), ("gen", rows >= Mu)):
            exp[sel] = oracle.linear_bf16(xb, host_bits(ws[(e, n)]), row_ids=rows[sel])
        assert max_rel(got, exp) <= MAX_REL and rel_l2(got, exp) < KERNEL_BAR
    _i8_launches(ops, g, Mu, Mg, [(H, [I, I])])


def test_c2_int8_down_full(ops):
    """Config 2's int8 down launch at full size: K = 12288, N = 4096, 4224
    rows over both weight sets, exact accumulators."""
    g = _gen(307)
    _i8_launches(ops, g, 128, 4096, [(I, [H])])


def test_mlp_chain_vs_reference(ops):
    """gate|up -> SwiGLU -> down on the GPU (unfused and fused SwiGLU)
    against the compiled reference's ref::linear and ref::silu composed as
    decoder_layer's MLP (src/u15-ref.cc:294-310), f32 throughout, on
    sampled rows of both groups: rel-L2 < 2e-2 (tests/u15-layer0-test.cc:
    299) and max-rel <= 1e-2."""
    if oracle.ref_lib() is None:
        pytest.skip("the compiled reference (oracle/_ref) is not built")
    Mu, Mg = 128, 4096
    g = _gen(308)
    st = u15h.Stack(1)
    W = _weights(g, 1, st, False, ops)
    t = _io(g, Mu + Mg)
    io = u15h.layer_io(**t)
    rows = np.array([0, 127, 128, 2100, 4223], np.int32)
    x2 = oracle.bf16_to_f32(host_bits(t["x2"])[rows])
    exp = np.empty((rows.size, H), np.float32)
    for e, sel in ((u15h.UND, rows < Mu), (u15h.GEN, rows >= Mu)):
        wg, wu, wd = (oracle.bf16_to_f32(host_bits(W[(0, e, p)][0])) for p in (4, 5, 6))
        gg = oracle.ref_linear(x2[sel], wg)
        uu = oracle.ref_linear(x2[sel], wu)
        hh = oracle.ref_silu(gg) * uu
        exp[sel] = oracle.ref_linear(hh, wd)
    for fused in (False, True):
        if fused:
            ops.stack_layer(st, 0, io, Mu, Mg, steps=u15h.STEP_GATE_UP,
                            flags=u15h.FUSED_SWIGLU)
        else:
            ops.stack_layer(st, 0, io, Mu, Mg, steps=u15h.STEP_GATE_UP)
            ops.swiglu(t["gate"], t["up"], t["h"])
        ops.stack_layer(st, 0, io, Mu, Mg, steps=u15h.STEP_DOWN)
        torch.cuda.synchronize()
        got = host_f32(t["down"])[rows]
        assert rel_l2(got, exp) < 2e-2, fused
        assert max_rel(got, exp) <= MAX_REL, fused
    st.close()
