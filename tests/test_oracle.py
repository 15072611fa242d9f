"""Pins the CPU oracle (oracle/) to things other than itself.

Each check is chosen so a plausible mistake in the oracle (a dropped term,
a swapped operand, a wrong rounding rule) fails it:
  * the reference's own compiled CPU path (oracle/_ref, from
    src/u15-ref.cc) on the reference test's own inputs;
  * committed golden fixtures written from that reference path;
  * closed forms and brute force with independent arithmetic
    (numpy int64, Python fractions, torch's bf16 rounding).
"""
import math
from fractions import Fraction

import numpy as np
import pytest
import torch

import oracle

REF = oracle.ref_lib() is not None


def torch_bf16_bits(a):
    t = torch.from_numpy(np.ascontiguousarray(a, np.float32))
    return t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


# ---- bf16 conversion ---------------------------------------------------------
def test_bf16_rne_matches_torch_over_bit_sweep():
    rng = np.random.default_rng(0)
    u = rng.integers(0, 2**32, size=400_000, dtype=np.uint64).astype(np.uint32)
    # every low-half pattern that decides a tie, on a spread of exponents
    ties = (np.arange(0, 2**16, dtype=np.uint32) | (0x3F81 << 16))
    u = np.concatenate([u, ties, ties | 0x80000000,
                        np.array([0x3F808000, 0x3F818000, 0x7F7FFFFF],
                                 np.uint32)])
    f = u.view(np.float32)
    f = f[np.isfinite(f)]
    assert np.array_equal(oracle.f32_to_bf16(f), torch_bf16_bits(f))


def test_bf16_widen_is_exact():
    h = np.arange(0, 2**16, dtype=np.uint16)
    f = oracle.bf16_to_f32(h)
    t = torch.from_numpy(h.view(np.int16)).view(torch.bfloat16).float().numpy()
    fin = np.isfinite(t)
    assert np.array_equal(f[fin].view(np.uint32), t[fin].view(np.uint32))


# ---- linear ------------------------------------------------------------------
@pytest.mark.skipif(not REF, reason="oracle/_ref not built (no reference)")
def test_linear_equals_reference_on_its_test_inputs():
    # tests/u15-kernels-test.cc:433-455: M=9 K=64 N=48, seeds 31/32.
    x = oracle.randn_mt(31, 9 * 64).reshape(9, 64)
    w = oracle.randn_mt(32, 48 * 64).reshape(48, 64)
    ours = oracle.linear(x, w)
    ref = oracle.ref_linear(x, w)
    assert np.array_equal(ours, ref)          # same double accumulation
    b = oracle.randn_mt(5, 48)
    assert np.array_equal(oracle.linear(x, w, b), oracle.ref_linear(x, w, b))


@pytest.mark.skipif(not REF, reason="oracle/_ref not built (no reference)")
def test_linear_equals_reference_random_shapes():
    rng = np.random.default_rng(1)
    for (M, K, N) in [(1, 1, 8), (7, 130, 24), (33, 512, 40)]:
        x = rng.standard_normal((M, K), dtype=np.float32)
        w = rng.standard_normal((N, K), dtype=np.float32)
        assert np.array_equal(oracle.linear(x, w), oracle.ref_linear(x, w))


def test_golden_linear_case(golden):
    g = golden("linear_test_case.npz")
    # the generator reproduces the reference test's inputs exactly
    assert np.array_equal(oracle.randn_mt(31, 9 * 64).reshape(9, 64), g["x"])
    assert np.array_equal(oracle.linear(g["x"], g["w"]), g["y_ref"])
    assert np.array_equal(oracle.linear_bf16(g["x_bf16"], g["w_bf16"]),
                          g["y_ref_bf16in"])
    assert np.array_equal(
        oracle.linear_bf16(g["x_bf16"], g["w_bf16"], g["bias_bf16"]),
        g["y_ref_bias"])


def test_golden_mot_case(golden):
    g = golden("mot_linear_case.npz")
    mu, mg = (int(v) for v in g["m"])
    y = oracle.mot_linear_bf16(g["x"], g["w_und"], g["w_gen"], mu, mg)
    assert np.array_equal(y, g["y_ref"])
    # exchange control: the two weight sets are not interchangeable
    y_swapped = oracle.mot_linear_bf16(g["x"], g["w_gen"], g["w_und"], mu, mg)
    assert oracle.rel_l2(y_swapped, g["y_ref"]) > 0.5


def test_linear_closed_forms():
    rng = np.random.default_rng(2)
    x = rng.standard_normal((5, 16), dtype=np.float32)
    # identity and permutation weights gather x exactly
    assert np.array_equal(oracle.linear(x, np.eye(16, dtype=np.float32)), x)
    perm = rng.permutation(16)
    assert np.array_equal(oracle.linear(x, np.eye(16, dtype=np.float32)[perm]),
                          x[:, perm])
    # K=1: an outer product, exact in f32 after one rounding
    a = rng.standard_normal((6, 1), dtype=np.float32)
    b = rng.standard_normal((9, 1), dtype=np.float32)
    assert np.array_equal(oracle.linear(a, b),
                          (a.astype(np.float64) @ b.T.astype(np.float64)).astype(np.float32))
    # small integers: exact
    xi = rng.integers(-8, 9, (4, 40)).astype(np.float32)
    wi = rng.integers(-8, 9, (12, 40)).astype(np.float32)
    exact = (xi.astype(np.int64) @ wi.T.astype(np.int64)).astype(np.float32)
    assert np.array_equal(oracle.linear(xi, wi), exact)
    # bias is added once, not per term; a transposed operand would fail
    bias = np.arange(12, dtype=np.float32)
    assert np.array_equal(oracle.linear(xi, wi, bias), exact + bias)
    xr = rng.integers(-8, 9, (3, 5)).astype(np.float32)
    wr = rng.integers(-8, 9, (7, 5)).astype(np.float32)
    assert np.array_equal(oracle.linear(xr, wr),
                          (xr.astype(np.int64) @ wr.T.astype(np.int64)).astype(np.float32))


def test_linear_bf16_row_subset():
    rng = np.random.default_rng(3)
    x = torch_bf16_bits(rng.standard_normal((10, 24), dtype=np.float32))
    w = torch_bf16_bits(rng.standard_normal((8, 24), dtype=np.float32))
    full = oracle.linear_bf16(x, w)
    ids = np.array([9, 0, 4], np.int32)
    assert np.array_equal(oracle.linear_bf16(x, w, row_ids=ids), full[ids])


# ---- silu / swiglu --------------------------------------------------------
@pytest.mark.skipif(not REF, reason="oracle/_ref not built (no reference)")
def test_silu_equals_reference():
    x = np.linspace(-30, 30, 4001, dtype=np.float32)
    assert np.array_equal(oracle.silu(x), oracle.ref_silu(x))


def test_silu_closed_forms():
    assert oracle.silu(np.array([0.0], np.float32))[0] == 0.0
    big = np.array([40.0, 80.0], np.float32)
    assert np.array_equal(oracle.silu(big), big)      # sigmoid -> 1
    x = np.linspace(0.1, 8, 200, dtype=np.float32)
    # silu(x) - silu(-x) = x (to f32 rounding of each term)
    d = oracle.silu(x).astype(np.float64) - oracle.silu(-x).astype(np.float64)
    assert np.max(np.abs(d - x)) < 2e-6 * 8


def test_golden_swiglu(golden):
    g = golden("swiglu_case.npz")
    assert np.array_equal(oracle.swiglu_bf16(g["g_bf16"], g["u_bf16"]),
                          g["h_ref"])


# ---- int8 quantisation -----------------------------------------------------
def _quant_bruteforce(row_f32):
    """Exact-rational restatement: s = f32(absmax/127), q = round-half-away
    of f32(x/s) clamped; f32 divisions are numpy's IEEE divisions."""
    amax = np.float32(np.max(np.abs(row_f32))) if row_f32.size else np.float32(0)
    s = np.float32(amax) / np.float32(127.0)
    q = []
    for v in row_f32:
        if s == 0:
            q.append(0)
            continue
        t = Fraction(float(np.float32(v) / s))
        mag = math.floor(abs(t) + Fraction(1, 2))
        c = mag if t >= 0 else -mag
        q.append(max(-127, min(127, c)))
    return np.array(q, np.int8), np.float32(s)


def test_quant_rows_bruteforce():
    rng = np.random.default_rng(4)
    rows = [rng.standard_normal(37, dtype=np.float32) * 3,
            np.zeros(37, np.float32),
            np.array([0.0] * 36 + [-5.0], np.float32),
            rng.standard_normal(37, dtype=np.float32) * 1e-30]
    # exact ties: absmax 127 -> s = 1, so k + 0.5 is a tie
    rows.append(np.array([127.0, 2.5, -2.5, 0.5, -0.5, 1.5, -126.5] + [0.0] * 30,
                         np.float32))
    x = torch_bf16_bits(np.stack(rows))
    q, s = oracle.quant_rows_i8(x)
    xf = oracle.bf16_to_f32(x)
    for r in range(x.shape[0]):
        qb, sb = _quant_bruteforce(xf[r])
        assert s[r] == sb
        assert np.array_equal(q[r], qb), r
    assert list(q[4][:7]) == [127, 3, -3, 1, -1, 2, -127]
    assert np.all(q[1] == 0) and s[1] == 0


def test_quant_invariants():
    rng = np.random.default_rng(5)
    x = torch_bf16_bits(rng.standard_normal((50, 256), dtype=np.float32))
    q, s = oracle.quant_rows_i8(x)
    xf = oracle.bf16_to_f32(x)
    assert np.all(np.abs(q.astype(np.int32)) <= 127)
    i = np.argmax(np.abs(xf), axis=1)
    assert np.all(np.abs(q[np.arange(50), i].astype(np.int32)) == 127)
    # reconstruction error is at most half a step (plus f32 slack)
    err = np.abs(q.astype(np.float64) * s[:, None] - xf)
    assert np.all(err <= 0.5 * s[:, None] * (1 + 1e-5))


# ---- int8 GEMM ------------------------------------------------------------------
def test_gemm_i8_bruteforce_and_extremes():
    rng = np.random.default_rng(6)
    a = rng.integers(-127, 128, (13, 384), dtype=np.int8)
    w = rng.integers(-127, 128, (24, 384), dtype=np.int8)
    ref = a.astype(np.int64) @ w.T.astype(np.int64)
    assert np.array_equal(oracle.gemm_i8_i32(a, w), ref)
    ext = np.full((2, 4096), 127, np.int8)
    ext[1] = -127
    wext = np.full((3, 4096), 127, np.int8)
    out = oracle.gemm_i8_i32(ext, wext)
    assert out[0, 0] == 127 * 127 * 4096 and out[1, 2] == -127 * 127 * 4096
    ids = np.array([12, 3], np.int32)
    assert np.array_equal(oracle.gemm_i8_i32(a, w, row_ids=ids), ref[ids])


def test_i8_product_sums_identity():
    rng = np.random.default_rng(7)
    a = rng.integers(-127, 128, (9, 200), dtype=np.int8)
    w = rng.integers(-127, 128, (11, 200), dtype=np.int8)
    full = a.astype(np.int64) @ w.T.astype(np.int64)
    rs, cs = oracle.i8_product_sums(a, w)
    assert np.array_equal(rs, full.sum(axis=1))
    assert np.array_equal(cs, full.sum(axis=0))


def test_dequant_against_numpy_f32():
    rng = np.random.default_rng(8)
    acc = rng.integers(-2**27, 2**27, (6, 16), dtype=np.int64).astype(np.int32)
    sa = (rng.random(6, dtype=np.float32) * 0.03).astype(np.float32)
    sw = (rng.random(16, dtype=np.float32) * 0.001).astype(np.float32)
    ours = oracle.dequant_bf16(acc, sa, sw)
    v = (acc.astype(np.float32) * sa[:, None]).astype(np.float32) * sw[None, :]
    assert np.array_equal(ours, torch_bf16_bits(v.astype(np.float32)))
    f64 = oracle.dequant_f64(acc, sa, sw)
    assert np.allclose(f64, acc.astype(np.float64) * sa[:, None] * sw[None, :],
                       rtol=0, atol=0)


def test_quantised_gemm_tracks_bf16_linear():
    """The int8 tier approximates the bf16 product: at K=4096 with N(0,1)
    activations and N(0,0.02) weights the dequantised result stays within a
    few percent rel-L2 of the exact product."""
    rng = np.random.default_rng(9)
    x = torch_bf16_bits(rng.standard_normal((4, 4096), dtype=np.float32))
    w = torch_bf16_bits(rng.standard_normal((32, 4096), dtype=np.float32) * 0.02)
    xq, sx = oracle.quant_rows_i8(x)
    wq, sw = oracle.quant_rows_i8(w)
    y = oracle.dequant_f64(oracle.gemm_i8_i32(xq, wq), sx, sw)
    ref = oracle.linear_bf16(x, w)
    assert oracle.rel_l2(y.astype(np.float32), ref) < 0.03


# ---- affine-quantized packs ------------------------------------------------
def _np_unpack(codes, bits, K):
    """Independent unpack: code k at bits [bits*(k%per), +bits) of word k/per."""
    per = 32 // bits
    N = codes.shape[0]
    sh = (np.arange(K) % per) * bits
    words = codes[:, np.arange(K) // per].astype(np.uint64)
    return ((words >> sh.astype(np.uint64)) & ((1 << bits) - 1)).astype(np.int64)


def _np_dequant_bits(codes, scales, biases, bits, group, K):
    q = _np_unpack(codes, bits, K).astype(np.float32)
    s = oracle.bf16_to_f32(scales).repeat(group, axis=1)
    b = oracle.bf16_to_f32(biases).repeat(group, axis=1)
    with np.errstate(all="ignore"):
        w = (s * q).astype(np.float32) + b           # f32 multiply, then add
    return torch_bf16_bits(w.astype(np.float32))


def test_pack_w8g64_round_trips_on_reference_fixture():
    """tests/u15-m5-test.cc:316-329: K=4096, N=6144, G=64, seed 77, stddev
    0.05; the pack's meaning is within 1.5e-2 rel-L2 of the weights."""
    K, N, G = 4096, 6144, 64
    w = oracle.randn_mt(77, N * K, 0.05).reshape(N, K)
    codes, sc, bi, deq = oracle.pack_affine(w, 8, G)
    e = oracle.rel_l2(deq, w)
    assert e < 1.5e-2
    # A uniform residual of step/sqrt(12), step = range/255: far below the
    # bar, so a packing error (wrong group, wrong byte) cannot hide under it.
    assert e < 8e-3


def test_pack_w4g32_round_trips():
    # 4 bits over 32 normals: step ~ 4.1 sigma / 15, residual ~ step/sqrt(12)
    # ~ 0.08 sigma.  A byte-order or group mix-up gives O(1).
    w = oracle.randn_mt(5, 512 * 256, 1.0).reshape(512, 256)
    codes, sc, bi, deq = oracle.pack_affine(w, 4, 32)
    e = oracle.rel_l2(deq, w)
    assert 0.03 < e < 0.12


@pytest.mark.parametrize("bits,group", [(8, 64), (8, 32), (4, 64), (4, 32)])
def test_pack_codes_follow_the_fixture_rule(bits, group):
    """Recompute every code with numpy from the stored scale/bias
    (tests/u15-m5-test.cc:280-306 generalised to 2^bits-1 levels) and check
    the packed words and the f32 meaning."""
    N, K = 24, 256
    w = oracle.randn_mt(11 + bits + group, N * K, 0.05).reshape(N, K)
    w[3, :group] = 0.25                            # a flat group: scale 0
    codes, sc, bi, deq = oracle.pack_affine(w, bits, group)
    lv = (1 << bits) - 1
    sf = oracle.bf16_to_f32(sc).repeat(group, axis=1)
    bf = oracle.bf16_to_f32(bi).repeat(group, axis=1)
    lo = w.reshape(N, K // group, group).min(axis=2).repeat(group, axis=1)
    hi = w.reshape(N, K // group, group).max(axis=2).repeat(group, axis=1)
    assert np.array_equal(sc.repeat(group, axis=1),
                          torch_bf16_bits((hi - lo) / np.float32(lv)))
    assert np.array_equal(bi.repeat(group, axis=1), torch_bf16_bits(lo))
    with np.errstate(all="ignore"):
        r = np.where(sf > 0, (w - bf) / np.where(sf > 0, sf, 1), 0)
    # lround: half away from zero
    q = np.clip(np.sign(r) * np.floor(np.abs(r).astype(np.float64) + 0.5),
                0, lv).astype(np.int64)
    assert np.array_equal(_np_unpack(codes, bits, K), q)
    assert np.array_equal(deq, (sf * q.astype(np.float32)) + bf)
    assert np.all(q[3, :group] == 0)


@pytest.mark.parametrize("bits,group", [(8, 64), (4, 32), (4, 64), (8, 32)])
def test_dequant_affine_matches_numpy_unpack(bits, group):
    N, K = 40, 512
    rng = np.random.default_rng(bits * 100 + group)
    codes = rng.integers(0, 2**32, size=(N, K * bits // 32),
                         dtype=np.uint64).astype(np.uint32)
    sc = torch_bf16_bits(rng.uniform(-0.02, 0.02, (N, K // group)))
    bi = torch_bf16_bits(rng.normal(0, 0.5, (N, K // group)))
    got = oracle.dequant_affine(codes, sc, bi, bits, group, K)
    assert np.array_equal(got, _np_dequant_bits(codes, sc, bi, bits, group, K))


def test_dequant_affine_closed_forms():
    N, K, G = 2, 64, 32
    # scale 1, bias 0: w = code exactly (codes <= 255 are bf16-exact).
    codes = np.array([[0x03020100 + 0x04040404 * i for i in range(16)]] * N,
                     np.uint32)
    one = torch_bf16_bits(np.ones((N, K // G)))
    zero = np.zeros((N, K // G), np.uint16)
    w = oracle.bf16_to_f32(oracle.dequant_affine(codes, one, zero, 8, G, K))
    assert np.array_equal(w, np.tile(np.arange(64, dtype=np.float32), (N, 1)))
    # all codes 0: w = bias; code 15 (w4 max) with scale 2, bias -1 -> 29.
    b = torch_bf16_bits(np.full((N, K // G), 0.375))
    w = oracle.bf16_to_f32(oracle.dequant_affine(
        np.zeros((N, K // 8), np.uint32), one, b, 4, G, K))
    assert np.all(w == 0.375)
    w = oracle.bf16_to_f32(oracle.dequant_affine(
        np.full((N, K // 8), 0xFFFFFFFF, np.uint32),
        torch_bf16_bits(np.full((N, K // G), 2.0)),
        torch_bf16_bits(np.full((N, K // G), -1.0)), 4, G, K))
    assert np.all(w == 29.0)


def test_dequant_affine_inverts_pack():
    """The pack and the dequant are two readers of one convention: the bf16
    expansion is the RNE of the pack's own f32 meaning."""
    w = oracle.randn_mt(3, 64 * 512, 0.05).reshape(64, 512)
    for bits, group in ((8, 64), (4, 32)):
        codes, sc, bi, deq = oracle.pack_affine(w, bits, group)
        got = oracle.dequant_affine(codes, sc, bi, bits, group, 512)
        assert np.array_equal(got, torch_bf16_bits(deq))


def test_bias_add_matches_f32_add_then_rne():
    rng = np.random.default_rng(9)
    y = torch_bf16_bits(rng.normal(0, 3, (33, 64)))
    b = torch_bf16_bits(rng.normal(0, 1, 64))
    got = oracle.bias_add_bf16(y, b)
    want = torch_bf16_bits(oracle.bf16_to_f32(y) + oracle.bf16_to_f32(b))
    assert np.array_equal(got, want)
    # bias 0 is the identity; y = -bias gives +0.
    assert np.array_equal(oracle.bias_add_bf16(y, np.zeros(64, np.uint16)), y)
    z = oracle.bias_add_bf16(np.tile(b ^ 0x8000, (2, 1)), b)
    assert np.all(oracle.bf16_to_f32(z) == 0)


# ---- split q/k norm + three-way RoPE ------------------------------------------
def _ref_test_case():
    """test_split_head's inputs (tests/u15-kernels-test.cc:124-153):
    H=4, T=12, D=32, x = randn(seed 7), w_t, w_hw ~ N(1, 0.2) from seed 8,
    positions: 5 text tokens then an image block (t = 5, h = i/7, w = i%7)."""
    H, T, D = 4, 12, 32
    x = oracle.randn_mt(7, T * H * D).reshape(T, H * D)
    w = oracle.randn_mt(8, D, 0.2) + np.float32(1.0)
    w_t, w_hw = w[: D // 2], w[D // 2:]
    pt = [i for i in range(5)] + [5] * (T - 5)
    ph = [0] * 5 + [i // 7 for i in range(T - 5)]
    pw = [0] * 5 + [i % 7 for i in range(T - 5)]
    return H, T, D, x, w_t, w_hw, np.array(pt), np.array(ph), np.array(pw)


@pytest.mark.skipif(not REF, reason="reference CPU path not built")
def test_norm_and_rope_pieces_equal_reference():
    rng = np.random.default_rng(3)
    for dim in (16, 32, 64, 128):
        x = rng.standard_normal((7, dim)).astype(np.float32) * 3
        w = rng.normal(1, 0.2, dim).astype(np.float32)
        assert np.array_equal(oracle.rms_norm(x, w, 1e-6),
                              oracle.ref_rms_norm(x, w, 1e-6))
        for theta in (1e4, 5e6):
            inv = oracle.rope_inv_freq(dim, theta)
            assert np.array_equal(inv, oracle.ref_rope_inv_freq(dim, theta))
            for pos in (0, 1, 37, 4095, 100000):
                assert np.array_equal(oracle.rope_half(x[0], inv, dim, pos),
                                      oracle.ref_rope_half(x[0], inv, dim, pos))


@pytest.mark.skipif(not REF, reason="reference CPU path not built")
def test_split_composition_equals_reference_split_rope_project():
    """u15::ref::split_rope_project (u15-ref.cc:121-175): projection, the two
    half norms, the three-way rope, emitted head-major.  The oracle's
    linear + split_qk_norm_rope, re-laid out, is bit-equal."""
    T, hidden, H, D = 9, 64, 3, 32
    rng = np.random.default_rng(11)
    x = rng.standard_normal((T, hidden)).astype(np.float32)
    wp = (rng.standard_normal((H * D, hidden)) * 0.1).astype(np.float32)
    wn = rng.normal(1, 0.2, D // 2).astype(np.float32)
    wh = rng.normal(1, 0.2, D // 2).astype(np.float32)
    pt, ph, pw = np.arange(T), np.arange(T) % 3, np.arange(T) // 3
    ref = oracle.ref_split_rope_project(x, wp, wn, wh, pt, ph, pw, H, D)
    proj = oracle.linear(x, wp)
    ours = oracle.split_qk_norm_rope(proj, wn, wh, pt, ph, pw, H, D, D // 2,
                                     D // 4)
    ours = ours.reshape(T, H, D).transpose(1, 0, 2)
    assert np.array_equal(ours, ref)


def test_split_head_negative_controls():
    """The reference test's two controls (tests/u15-kernels-test.cc:
    208-257): h and w exchanged, and one whole-head norm instead of two
    half norms, must both be more than 1e-2 away."""
    H, T, D, x, w_t, w_hw, pt, ph, pw = _ref_test_case()
    d_t, d_h = D // 2, D // 4
    ref = oracle.split_qk_norm_rope(x, w_t, w_hw, pt, ph, pw, H, D, d_t, d_h)
    swapped = oracle.split_qk_norm_rope(x, w_t, w_hw, pt, pw, ph, H, D, d_t, d_h)
    assert oracle.rel_l2(swapped, ref) > 1e-2
    whole = oracle.rms_norm(x.reshape(T * H, D),
                            np.concatenate([w_t, w_hw]), 1e-6).reshape(T, H * D)
    whole = oracle.split_qk_norm_rope(whole, w_t, w_hw, pt, ph, pw, H, D, d_t,
                                      d_h, norm=False)
    assert oracle.rel_l2(whole, ref) > 1e-2


def test_rope_rotation_closed_forms():
    H, T, D, x, w_t, w_hw, pt, ph, pw = _ref_test_case()
    d_t, d_h = D // 2, D // 4
    normed = oracle.split_qk_norm_rope(x, w_t, w_hw, pt, ph, pw, H, D, d_t,
                                       d_h, rope=False)
    roped = oracle.split_qk_norm_rope(x, w_t, w_hw, pt, ph, pw, H, D, d_t, d_h)
    n3 = normed.reshape(T, H, D).astype(np.float64)
    r3 = roped.reshape(T, H, D).astype(np.float64)
    # each rotated pair keeps its length
    for off, width in ((0, d_t), (d_t, d_h), (d_t + d_h, d_h)):
        h = width // 2
        a = n3[..., off:off + h] ** 2 + n3[..., off + h:off + width] ** 2
        b = r3[..., off:off + h] ** 2 + r3[..., off + h:off + width] ** 2
        assert np.allclose(a, b, rtol=1e-5, atol=1e-6)
    # all positions 0: the rotation is the identity
    z = np.zeros(T, np.int32)
    r0 = oracle.split_qk_norm_rope(x, w_t, w_hw, z, z, z, H, D, d_t, d_h)
    assert np.array_equal(r0, normed)
    # the half norms: unit weights give each half a mean square of 1
    ones = np.ones(D // 2, np.float32)
    u = oracle.split_qk_norm_rope(x, ones, ones, pt, ph, pw, H, D, d_t, d_h,
                                  rope=False).reshape(T * H, D).astype(np.float64)
    assert np.allclose((u[:, : D // 2] ** 2).mean(1), 1, rtol=1e-5)
    assert np.allclose((u[:, D // 2:] ** 2).mean(1), 1, rtol=1e-5)


def test_rope_tables_closed_forms():
    T, D, d_t, d_h = 6, 32, 16, 8
    pt = np.array([0, 1, 2, 3, 4, 1000])
    ph = np.array([0, 5, 0, 7, 1, 2])
    pw = np.array([0, 0, 9, 1, 3, 4])
    cs, sn = oracle.rope_tables(pt, ph, pw, D, d_t, d_h)
    assert np.all(cs[0] == 1) and np.all(sn[0] == 0)
    for off, w, p in ((0, d_t, pt), (d_t, d_h, ph), (d_t + d_h, d_h, pw)):
        h = w // 2
        assert np.array_equal(cs[:, off:off + h], cs[:, off + h:off + w])
        assert np.array_equal(sn[:, off:off + h], sn[:, off + h:off + w])
        # the first pair of every range has frequency 1: angle = position
        assert np.array_equal(cs[:, off], np.cos(p.astype(np.float64)).astype(np.float32))
        assert np.array_equal(sn[:, off], np.sin(p.astype(np.float64)).astype(np.float32))
    # rotating with the tables equals rotate_half with the ladders (f32
    # tables against double angles: within a few f32 ulps)
    x = oracle.randn_mt(5, D)
    got = np.empty(D, np.float64)
    for off, w in ((0, d_t), (d_t, d_h), (d_t + d_h, d_h)):
        h = w // 2
        for j in range(h):
            i = off + j
            a, b = float(x[i]), float(x[i + h])
            got[i] = a * cs[3, i] - b * sn[3, i]
            got[i + h] = b * cs[3, i + h] + a * sn[3, i + h]
    want = x.copy()
    want[:d_t] = oracle.rope_half(want[:d_t], oracle.rope_inv_freq(d_t, 5e6), d_t, 3)
    want[d_t:d_t + d_h] = oracle.rope_half(want[d_t:d_t + d_h],
                                           oracle.rope_inv_freq(d_h, 1e4), d_h, 7)
    want[d_t + d_h:] = oracle.rope_half(want[d_t + d_h:],
                                        oracle.rope_inv_freq(d_h, 1e4), d_h, 1)
    assert np.allclose(got, want, rtol=1e-6, atol=1e-6)


def test_f16_to_bf16_every_pattern():
    """The loader's f16 -> bf16 (u15-weights.cc:66-94) on all 65536 f16
    patterns: every finite and infinite one equals numpy's exact f16 -> f32
    widening rounded by torch's RNE."""
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.f16_to_bf16(h)
    f = h.view(np.float16).astype(np.float32)
    ok = ~np.isnan(f)
    want = torch_bf16_bits(f)
    assert np.array_equal(got[ok], want[ok])
    # subnormals, signed zeros and the largest finite value explicitly
    for bits, val in ((0x0001, 2.0 ** -24), (0x03ff, 1023 * 2.0 ** -24),
                      (0x8000, -0.0), (0x7bff, 65504.0)):
        assert oracle.bf16_to_f32(got[bits]) == np.float32(
            torch.tensor(val).to(torch.bfloat16).float().item())


# ---- attention ------------------------------------------------------------------
def _cache(kk, cap):
    hkv, tk, d = kk.shape
    c = np.zeros((hkv, cap, d), np.float32)
    c[:, :tk] = kk
    return c


def _tm_to_hm(o, hq):
    tq = o.shape[0]
    return o.reshape(tq, hq, -1).transpose(1, 0, 2)


@pytest.mark.skipif(not REF, reason="reference CPU path not built")
def test_attention_equals_reference_all_masks():
    """test_sdpa / test_block_causal inputs (tests/u15-kernels-test.cc:
    510-600, 604-666): GQA, a cache longer than the keys in use."""
    hq, hkv, tq, tk, d, cap = 4, 2, 6, 6, 32, 10
    q = oracle.randn_mt(61, hq * tq * d).reshape(hq, tq, d)
    kk = oracle.randn_mt(62, hkv * tk * d).reshape(hkv, tk, d)
    vv = oracle.randn_mt(63, hkv * tk * d).reshape(hkv, tk, d)
    k, v = _cache(kk, cap), _cache(vv, cap)
    got = oracle.attention(q, k, v, hkv, tk)
    want = _tm_to_hm(oracle.ref_attention(q, kk, vv, None, hkv), hq)
    assert np.array_equal(got, want)
    causal = np.where(np.arange(tk)[None, :] > np.arange(tq)[:, None],
                      -np.inf, 0).astype(np.float32)
    got = oracle.attention(q, k, v, hkv, tk, "causal")
    assert np.array_equal(got, _tm_to_hm(oracle.ref_attention(q, kk, vv, causal, hkv), hq))
    t_idx = np.array([0, 1, 2, 3, 3, 3, 3, 3, 3, 4, 5], np.int32)
    T = t_idx.size
    q = oracle.randn_mt(71, hq * T * d).reshape(hq, T, d)
    kk = oracle.randn_mt(72, hkv * T * d).reshape(hkv, T, d)
    vv = oracle.randn_mt(73, hkv * T * d).reshape(hkv, T, d)
    mask = oracle.ref_block_causal_mask(t_idx)
    got = oracle.attention(q, _cache(kk, T + 4), _cache(vv, T + 4), hkv, T,
                           "block_causal", t_idx)
    assert np.array_equal(got, _tm_to_hm(oracle.ref_attention(q, kk, vv, mask, hkv), hq))


def test_attention_controls_and_closed_forms():
    """The reference tests' controls (u15-kernels-test.cc:672-718, 806-825)
    and closed forms."""
    hq, hkv, d = 4, 2, 32
    t_idx = np.array([0, 1, 2, 3, 3, 3, 3, 3, 3, 4, 5], np.int32)
    T = t_idx.size
    q = oracle.randn_mt(71, hq * T * d).reshape(hq, T, d)
    k = _cache(oracle.randn_mt(72, hkv * T * d).reshape(hkv, T, d), T)
    v = _cache(oracle.randn_mt(73, hkv * T * d).reshape(hkv, T, d), T)
    blk = oracle.attention(q, k, v, hkv, T, "block_causal", t_idx)
    cau = oracle.attention(q, k, v, hkv, T, "causal")
    assert oracle.rel_l2(cau, blk) > 1e-2          # the block rule matters
    text = np.arange(T, dtype=np.int32)
    assert np.array_equal(oracle.attention(q, k, v, hkv, T, "block_causal", text), cau)
    # the GQA group is load-bearing: kv head h // 2 vs h // 1 (a cache with
    # hq heads whose extra heads hold other keys)
    k4 = np.concatenate([k, oracle.randn_mt(74, 2 * T * d).reshape(2, T, d)])
    v4 = np.concatenate([v, oracle.randn_mt(75, 2 * T * d).reshape(2, T, d)])
    good = oracle.attention(q, k, v, hkv, T)
    bad = oracle.attention(q, k4, v4, hq, T)
    assert oracle.rel_l2(bad, good) > 1e-2
    # identical keys: uniform weights, the output is the mean of the values
    kc = np.repeat(k[:, :1], T, axis=1)
    u = oracle.attention(q, kc, v, hkv, T)
    mean = v.mean(axis=1)
    assert np.allclose(u, np.repeat(mean, hq // hkv, axis=0)[:, None, :], atol=1e-6)
    # one key: the output is that key's value row
    one = oracle.attention(q, k, v, hkv, 1)
    assert np.allclose(one, np.repeat(v[:, :1], hq // hkv, axis=0).repeat(T, 1), atol=1e-7)


def _tiny_layer(rng, hidden=64, heads=4, kv=2, hd=16, inter=96):
    w = {"input_layernorm": 1 + 0.2 * rng.standard_normal(hidden),
         "post_attention_layernorm": 1 + 0.2 * rng.standard_normal(hidden),
         "q_proj": 0.1 * rng.standard_normal((heads * hd, hidden)),
         "k_proj": 0.1 * rng.standard_normal((kv * hd, hidden)),
         "v_proj": 0.1 * rng.standard_normal((kv * hd, hidden)),
         "o_proj": 0.1 * rng.standard_normal((hidden, heads * hd)),
         "q_norm": 1 + 0.2 * rng.standard_normal(hd // 2),
         "k_norm": 1 + 0.2 * rng.standard_normal(hd // 2),
         "q_norm_hw": 1 + 0.2 * rng.standard_normal(hd // 2),
         "k_norm_hw": 1 + 0.2 * rng.standard_normal(hd // 2),
         "gate_proj": 0.1 * rng.standard_normal((inter, hidden)),
         "up_proj": 0.1 * rng.standard_normal((inter, hidden)),
         "down_proj": 0.1 * rng.standard_normal((hidden, inter))}
    return {k: v.astype(np.float32) for k, v in w.items()}


@pytest.mark.skipif(not REF, reason="reference CPU path not built")
@pytest.mark.parametrize("masked", [False, True])
def test_decoder_layer_wrapper_is_the_reference_composition(masked):
    """oracle.ref_decoder_layer (the compiled u15::ref::decoder_layer through
    its C shim) against the same layer composed step by step from the
    reference's own pieces (src/u15-ref.cc:242-311): rms_norm, the split
    q/k projection, v, attention, o + residual, rms_norm, SwiGLU MLP +
    residual.  Every step is f32 in the same order, so the two agree bit
    for bit; a wrong argument order in the shim (a swapped weight, head
    count or position array) does not."""
    rng = np.random.default_rng(77)
    T, hidden, heads, kv, hd, inter = 6, 64, 4, 2, 16, 96
    w = _tiny_layer(rng, hidden, heads, kv, hd, inter)
    x = rng.standard_normal((T, hidden)).astype(np.float32)
    pt = np.array([0, 1, 2, 3, 3, 3], np.int32)
    ph = np.array([0, 0, 0, 0, 1, 1], np.int32)
    pw = np.array([0, 0, 0, 0, 0, 1], np.int32)
    mask = oracle.ref_block_causal_mask(pt) if masked else None
    got = oracle.ref_decoder_layer(x, w, heads, kv, hd, pt, ph, pw, mask)

    normed = oracle.ref_rms_norm(x, w["input_layernorm"])
    q = oracle.ref_split_rope_project(normed, w["q_proj"], w["q_norm"], w["q_norm_hw"],
                                      pt, ph, pw, heads, hd)
    k = oracle.ref_split_rope_project(normed, w["k_proj"], w["k_norm"], w["k_norm_hw"],
                                      pt, ph, pw, kv, hd)
    v = oracle.ref_linear(normed, w["v_proj"]).reshape(T, kv, hd).transpose(1, 0, 2)
    att = oracle.ref_attention(q, k, np.ascontiguousarray(v), mask, kv)
    proj = oracle.ref_linear(att, w["o_proj"]) + x
    n2 = oracle.ref_rms_norm(proj, w["post_attention_layernorm"])
    g = oracle.ref_silu(oracle.ref_linear(n2, w["gate_proj"]))
    u = oracle.ref_linear(n2, w["up_proj"])
    want = proj + oracle.ref_linear(g * u, w["down_proj"])
    assert np.array_equal(got, want)
    # the shim's weight order is load-bearing
    w2 = dict(w, q_norm=w["k_norm"], k_norm=w["q_norm"])
    assert not np.array_equal(oracle.ref_decoder_layer(x, w2, heads, kv, hd, pt, ph, pw, mask),
                              got)
