"""GPU parity of the bf16 projection GEMMs against the CPU oracle.

Bars (stated here, used everywhere):
  * BASELINE: max-rel-err <= 1e-2, max|y - ref| / max|ref|, fp32 accumulate;
  * the reference's own: rel-L2 < 4e-3 (tests/u15-kernels-test.cc:55) and
    < 6e-3 at model shapes (tests/u15-m5-test.cc:56).
The GPU output is bf16, so its rounding alone contributes ~2e-3 rel-L2.
"""
import numpy as np
import pytest
import torch

import oracle
import u15h
from helpers import dev_bf16, host_bits, host_f32, max_rel, rand_bf16_bits, rel_l2

pytestmark = pytest.mark.gpu

MAX_REL = 1e-2
REF_BAR = 4e-3       # tests/u15-kernels-test.cc:55
M5_BAR = 6e-3        # tests/u15-m5-test.cc:56


def widen(bits):
    return oracle.bf16_to_f32(bits)


def test_linear_reference_test_case(ops, golden):
    """test_linear (tests/u15-kernels-test.cc:433-455): M=9 K=64 N=48,
    the reference test's inputs; expected output from the reference's own
    CPU linear (golden fixture)."""
    g = golden("linear_test_case.npz")
    x, w = dev_bf16(g["x_bf16"]), dev_bf16(g["w_bf16"])
    y = torch.empty(9, 48, dtype=torch.bfloat16, device="cuda")
    ops.linear(x, w, None, y, 9, 64, 48)
    torch.cuda.synchronize()
    out = host_f32(y)
    print(f"\n  rel-L2 vs reference (f32 inputs) {rel_l2(out, g['y_ref']):.3e}")
    assert rel_l2(out, g["y_ref"]) < REF_BAR
    assert rel_l2(out, g["y_ref_bf16in"]) < REF_BAR
    assert max_rel(out, g["y_ref_bf16in"]) <= MAX_REL
    # with bias
    b = dev_bf16(g["bias_bf16"])
    ops.linear(x, w, b, y, 9, 64, 48)
    torch.cuda.synchronize()
    assert max_rel(host_f32(y), g["y_ref_bias"]) <= MAX_REL
    assert rel_l2(host_f32(y), g["y_ref_bias"]) < REF_BAR


def test_mot_linear_golden_case(ops, golden):
    g = golden("mot_linear_case.npz")
    mu, mg = (int(v) for v in g["m"])
    x = dev_bf16(g["x"])
    y = torch.empty(mu + mg, 40, dtype=torch.bfloat16, device="cuda")
    ops.mot_linear(x, mu, mg, 64, [dict(w_und=dev_bf16(g["w_und"]),
                                        w_gen=dev_bf16(g["w_gen"]), y=y)])
    torch.cuda.synchronize()
    assert rel_l2(host_f32(y), g["y_ref"]) < REF_BAR
    assert max_rel(host_f32(y), g["y_ref"]) <= MAX_REL


M5_SHAPES = [(1, 4096, 6144), (4, 4096, 6144), (16, 4096, 6144),
             (64, 4096, 6144), (256, 4096, 6144), (256, 4096, 4096),
             (256, 4096, 24576), (256, 12288, 4096), (1024, 4096, 6144),
             (1024, 12288, 4096)]


@pytest.mark.parametrize("M,K,N", M5_SHAPES)
def test_linear_model_shapes(ops, M, K, N):
    """The reference's model-shape sweep (tests/u15-m5-test.cc:146-200):
    inputs randn*0.05 with seeds 11 / 22 from the reference tests'
    generator; sampled rows checked against the oracle."""
    xf = oracle.randn_mt(11, M * K, 0.05).reshape(M, K)
    wf = oracle.randn_mt(22, N * K, 0.05).reshape(N, K)
    xb, wb = oracle.f32_to_bf16(xf), oracle.f32_to_bf16(wf)
    y = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    ops.linear(dev_bf16(xb), dev_bf16(wb), None, y, M, K, N)
    torch.cuda.synchronize()
    out = host_f32(y)
    assert np.all(np.isfinite(out))
    rows = np.unique(np.array([0, M // 3, M // 2, M - 1], np.int32))
    ref = oracle.linear_bf16(xb, wb, row_ids=rows)
    e = rel_l2(out[rows], ref)
    print(f"\n  M={M} K={K} N={N} rel-L2 {e:.2e} max-rel {max_rel(out[rows], ref):.2e}")
    assert e < M5_BAR
    assert max_rel(out[rows], ref) <= MAX_REL


def test_mot_qkv_one_launch_c1_shape(ops):
    """Config 1's token split (64 und + 192 gen), q/k/v in one launch;
    each row checked with ITS expert's weights.  Negative control: the
    other expert's weights must fail the same bar."""
    rng = np.random.default_rng(100)
    Mu, Mg, K = 64, 192, 4096
    M = Mu + Mg
    xb = rand_bf16_bits(rng, (M, K))
    Ns = [4096, 1024, 1024]
    W = [(rand_bf16_bits(rng, (n, K), 0.02), rand_bf16_bits(rng, (n, K), 0.02))
         for n in Ns]
    x = dev_bf16(xb)
    ys = [torch.empty(M, n, dtype=torch.bfloat16, device="cuda") for n in Ns]
    projs = [dict(w_und=dev_bf16(wu), w_gen=dev_bf16(wg), y=y)
             for (wu, wg), y in zip(W, ys)]
    ops.mot_linear(x, Mu, Mg, K, projs)
    torch.cuda.synchronize()
    und_rows = np.array([0, 17, 63], np.int32)
    gen_rows = np.array([64, 100, 191, 255], np.int32)
    for (wu, wg), y in zip(W, ys):
        out = host_f32(y)
        ru = oracle.linear_bf16(xb, wu, row_ids=und_rows)
        rg = oracle.linear_bf16(xb, wg, row_ids=gen_rows)
        assert rel_l2(out[und_rows], ru) < REF_BAR
        assert rel_l2(out[gen_rows], rg) < REF_BAR
        assert max_rel(out[und_rows], ru) <= MAX_REL
        assert max_rel(out[gen_rows], rg) <= MAX_REL
        # exchange control
        assert rel_l2(out[und_rows], oracle.linear_bf16(xb, wg, row_ids=und_rows)) > 0.5
        assert rel_l2(out[gen_rows], oracle.linear_bf16(xb, wu, row_ids=gen_rows)) > 0.5


@pytest.mark.parametrize("Mu,Mg,K,N", [(37, 263, 72, 40), (0, 300, 136, 264),
                                       (5, 0, 64, 8), (1, 1, 8, 8),
                                       (257, 511, 200, 520),
                                       # split into K shares, K tail in the last
                                       (37, 263, 1032, 264)])
def test_mot_linear_ragged_full_check(ops, Mu, Mg, K, N):
    """Ragged tails in M (both groups), N and K (K not a multiple of the
    64-element stage); the whole output against the oracle."""
    rng = np.random.default_rng(Mu * 1000 + Mg + K + N)
    M = Mu + Mg
    xb = rand_bf16_bits(rng, (M, K))
    wu = rand_bf16_bits(rng, (N, K), 0.1)
    wg = rand_bf16_bits(rng, (N, K), 0.1)
    y = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
    ops.mot_linear(dev_bf16(xb), Mu, Mg, K,
                   [dict(w_und=dev_bf16(wu), w_gen=dev_bf16(wg), y=y)])
    torch.cuda.synchronize()
    ref = oracle.mot_linear_bf16(xb, wu, wg, Mu, Mg)
    out = host_f32(y)
    assert np.all(np.isfinite(out))
    assert rel_l2(out, ref) < REF_BAR
    assert max_rel(out, ref) <= MAX_REL


def test_identity_weight_is_exact(ops):
    rng = np.random.default_rng(7)
    K = 256
    xb = rand_bf16_bits(rng, (300, K))
    eye = oracle.f32_to_bf16(np.eye(K, dtype=np.float32))
    y = torch.empty(300, K, dtype=torch.bfloat16, device="cuda")
    ops.linear(dev_bf16(xb), dev_bf16(eye), None, y, 300, K, K)
    torch.cuda.synchronize()
    assert np.array_equal(host_bits(y), xb)


def test_row_permutation_is_bit_exact(ops):
    """Each output row depends only on its own input row: permuting the
    rows permutes the output bit for bit."""
    rng = np.random.default_rng(8)
    M, K, N = 512, 1024, 512
    xb = rand_bf16_bits(rng, (M, K))
    wb = rand_bf16_bits(rng, (N, K), 0.05)
    perm = rng.permutation(M)
    w = dev_bf16(wb)
    y1 = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    y2 = torch.empty_like(y1)
    ops.linear(dev_bf16(xb), w, None, y1, M, K, N)
    ops.linear(dev_bf16(xb[perm]), w, None, y2, M, K, N)
    torch.cuda.synchronize()
    assert np.array_equal(host_bits(y1)[perm], host_bits(y2))


def test_swiglu_elementwise(ops, golden):
    g = golden("swiglu_case.npz")
    gt, ut = dev_bf16(g["g_bf16"]), dev_bf16(g["u_bf16"])
    out = torch.empty_like(gt)
    ops.swiglu(gt, ut, out)
    torch.cuda.synchronize()
    assert max_rel(host_f32(out), g["h_ref"]) <= MAX_REL
    assert rel_l2(host_f32(out), g["h_ref"]) < REF_BAR


def test_fused_gate_up_swiglu_matches_unfused(ops):
    """The fused gate/up/SwiGLU launch equals the reference's unfused
    sequence (gate GEMM, up GEMM, swiglu; src/u15-backbone.cc:251-253) bit
    for bit on the GPU, and the oracle to the bar."""
    rng = np.random.default_rng(9)
    Mu, Mg, K, I = 40, 300, 512, 384
    M = Mu + Mg
    xb = rand_bf16_bits(rng, (M, K))
    ws = [rand_bf16_bits(rng, (I, K), 0.05) for _ in range(4)]
    x = dev_bf16(xb)
    wgu, wuu, wgg, wug = (dev_bf16(w) for w in ws)
    h = torch.empty(M, I, dtype=torch.bfloat16, device="cuda")
    ops.mot_gate_up_swiglu(x, Mu, Mg, K, wgu, wuu, wgg, wug, h)
    gate = torch.empty(M, I, dtype=torch.bfloat16, device="cuda")
    up = torch.empty_like(gate)
    ops.mot_linear(x, Mu, Mg, K, [dict(w_und=wgu, w_gen=wgg, y=gate),
                                  dict(w_und=wuu, w_gen=wug, y=up)])
    h2 = torch.empty_like(h)
    ops.swiglu(gate, up, h2)
    torch.cuda.synchronize()
    assert np.array_equal(host_bits(h), host_bits(h2))
    ref_g = oracle.mot_linear_bf16(xb, ws[0], ws[2], Mu, Mg)
    ref_u = oracle.mot_linear_bf16(xb, ws[1], ws[3], Mu, Mg)
    ref = oracle.swiglu_bf16(oracle.f32_to_bf16(ref_g), oracle.f32_to_bf16(ref_u))
    assert max_rel(host_f32(h), ref) <= MAX_REL
    assert rel_l2(host_f32(h), ref) < 1e-2


def test_gather_scatter_roundtrip(ops):
    rng = np.random.default_rng(10)
    expert = rng.integers(0, 2, 333).astype(np.uint8)
    perm, mu, mg = u15h.route_rows(expert)
    src = dev_bf16(rand_bf16_bits(rng, (333, 64)))
    p = torch.from_numpy(perm).cuda()
    grouped = torch.empty_like(src)
    back = torch.empty_like(src)
    ops.gather_rows(src, p, grouped)
    ops.scatter_rows(grouped, p, back)
    torch.cuda.synchronize()
    assert torch.equal(grouped.cpu(), src.cpu()[torch.from_numpy(perm).long()])
    assert torch.equal(back.cpu(), src.cpu())


def test_routed_tokens_use_their_expert(ops):
    """Interleaved token types: route, run the grouped GEMM, scatter back;
    every token's row equals linear with its own expert's weights."""
    rng = np.random.default_rng(11)
    M, K, N = 200, 256, 128
    expert = rng.integers(0, 2, M).astype(np.uint8)
    perm, mu, mg = u15h.route_rows(expert)
    xb = rand_bf16_bits(rng, (M, K))
    wu = rand_bf16_bits(rng, (N, K), 0.05)
    wg = rand_bf16_bits(rng, (N, K), 0.05)
    x = dev_bf16(xb)
    p = torch.from_numpy(perm).cuda()
    xg = torch.empty_like(x)
    ops.gather_rows(x, p, xg)
    yg = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    ops.mot_linear(xg, mu, mg, K, [dict(w_und=dev_bf16(wu), w_gen=dev_bf16(wg), y=yg)])
    y = torch.empty_like(yg)
    ops.scatter_rows(yg, p, y)
    torch.cuda.synchronize()
    out = host_f32(y)
    for t in range(M):
        ref = oracle.linear_bf16(xb[t:t + 1], wg if expert[t] else wu)
        assert max_rel(out[t:t + 1], ref) <= MAX_REL


def test_invalid_shapes_launch_nothing(ops):
    x = torch.zeros(4, 16, dtype=torch.bfloat16, device="cuda")
    w = torch.zeros(12, 16, dtype=torch.bfloat16, device="cuda")
    y = torch.full((4, 12), 7.0, dtype=torch.bfloat16, device="cuda")
    lib, ctx = ops.lib, ops.ctx
    import ctypes
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    st = lib.u15h_linear(ctx, s, ctypes.c_void_p(x.data_ptr()),
                         ctypes.c_void_p(w.data_ptr()), None,
                         ctypes.c_void_p(y.data_ptr()), 4, 16, 12)
    assert st == u15h.EINVAL                     # N % 8 != 0
    assert b"N=12" in lib.u15h_last_error(ctx)
    st = lib.u15h_linear(ctx, s, ctypes.c_void_p(x.data_ptr() + 2),
                         ctypes.c_void_p(w.data_ptr()), None,
                         ctypes.c_void_p(y.data_ptr()), 4, 16, 8)
    assert st == u15h.EINVAL                     # misaligned x
    # N above 2^20: rejected before anything is read (the pointers are the
    # small buffers above; nothing may touch them)
    st = lib.u15h_linear(ctx, s, ctypes.c_void_p(x.data_ptr()),
                         ctypes.c_void_p(w.data_ptr()), None,
                         ctypes.c_void_p(y.data_ptr()), 4, 16, (1 << 20) + 8)
    assert st == u15h.EINVAL
    assert b"too large" in lib.u15h_last_error(ctx)
    torch.cuda.synchronize()
    assert torch.all(y == 7.0)


@pytest.fixture(scope="module")
def ops_nosplit():
    """A second context built with the split-K tail switched off
    (U15H_SPLIT=0 read at creation) -- the in-process A/B the reference's
    model-shape test makes with its kill switches
    (tests/u15-m5-test.cc:391-404)."""
    import os
    old = os.environ.get("U15H_SPLIT")
    os.environ["U15H_SPLIT"] = "0"
    try:
        o = u15h.Ops(0)
    finally:
        if old is None:
            del os.environ["U15H_SPLIT"]
        else:
            os.environ["U15H_SPLIT"] = old
    yield o
    torch.cuda.synchronize()
    o.close()


@pytest.mark.parametrize("Mu,Mg,K,N", [(128, 4096, 4096, 4096),    # o: 272 tiles
                                       (128, 4096, 12288, 4096),   # down
                                       (0, 256, 4096, 6144)])      # one partial round
def test_split_tail_matches_unsplit(ops, ops_nosplit, Mu, Mg, K, N):
    """Split-K tail vs whole tiles on the same inputs: both within the bar
    of the oracle on sampled rows, and of each other everywhere."""
    M = Mu + Mg
    g = torch.Generator(device="cuda").manual_seed(M + K + N)
    x = torch.randn(M, K, generator=g, device="cuda").to(torch.bfloat16)
    wu = (torch.randn(N, K, generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    wg = (torch.randn(N, K, generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    y1 = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    y2 = torch.empty_like(y1)
    ops.mot_linear(x, Mu, Mg, K, [dict(w_und=wu, w_gen=wg, y=y1)])
    ops_nosplit.mot_linear(x, Mu, Mg, K, [dict(w_und=wu, w_gen=wg, y=y2)])
    torch.cuda.synchronize()
    a, b = host_f32(y1), host_f32(y2)
    assert rel_l2(a, b) < 4e-3 and max_rel(a, b) <= MAX_REL
    xb, wub, wgb = host_bits(x), host_bits(wu), host_bits(wg)
    rows = np.array([0, Mu // 2, M - 1, max(Mu, 1) + 7], np.int32)
    for r in rows:
        w = wub if r < Mu else wgb
        ref = oracle.linear_bf16(xb, w, row_ids=np.array([r], np.int32))
        assert max_rel(a[r:r + 1], ref) <= MAX_REL
        assert rel_l2(a[r:r + 1], ref) < REF_BAR


@pytest.fixture(scope="module")
def ops_4waves():
    """A context built with the 4-wave GEMM workgroup (U15H_WAVES=4)."""
    import os
    old = os.environ.get("U15H_WAVES")
    os.environ["U15H_WAVES"] = "4"
    try:
        o = u15h.Ops(0)
    finally:
        if old is None:
            del os.environ["U15H_WAVES"]
        else:
            os.environ["U15H_WAVES"] = old
    yield o
    torch.cuda.synchronize()
    o.close()


@pytest.mark.parametrize("Mu,Mg,K,N", [(37, 263, 1032, 264), (128, 4096, 4096, 1024)])
def test_workgroup_shapes_agree(ops, ops_4waves, Mu, Mg, K, N):
    """The 8-wave workgroup (128x64 per wave) and the 4-wave one (128x128
    per wave, accumulators pinned in AGPRs by inline-asm MFMAs): the f32
    sums may round differently, so the bf16 outputs and the fused SwiGLU
    outputs agree within the bar, and both match the oracle on sampled
    rows."""
    M = Mu + Mg
    g = torch.Generator(device="cuda").manual_seed(K + N)
    x = torch.randn(M, K, generator=g, device="cuda").to(torch.bfloat16)
    ws = [(torch.randn(N, K, generator=g, device="cuda") * 0.02).to(torch.bfloat16)
          for _ in range(4)]
    outs = []
    for o in (ops, ops_4waves):
        y = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
        h = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
        o.mot_linear(x, Mu, Mg, K, [dict(w_und=ws[0], w_gen=ws[1], y=y)])
        o.mot_gate_up_swiglu(x, Mu, Mg, K, ws[0], ws[1], ws[2], ws[3], h)
        outs.append((y, h))
    torch.cuda.synchronize()
    for a, b in ((outs[0][0], outs[1][0]), (outs[0][1], outs[1][1])):
        fa, fb = host_f32(a), host_f32(b)
        assert rel_l2(fa, fb) < 4e-3 and max_rel(fa, fb) <= MAX_REL
    xb = host_bits(x)
    for r in (0, Mu - 1, Mu, M - 1):
        w = host_bits(ws[0] if r < Mu else ws[1])
        ref = oracle.linear_bf16(xb, w, row_ids=np.array([r], np.int32))
        for y in (outs[0][0], outs[1][0]):
            assert max_rel(host_f32(y)[r:r + 1], ref) <= MAX_REL


def _ops_with_env(name, value):
    import os
    old = os.environ.get(name)
    os.environ[name] = value
    try:
        return u15h.Ops(0)
    finally:
        if old is None:
            del os.environ[name]
        else:
            os.environ[name] = old


@pytest.fixture(scope="module")
def ops_per_item():
    """A context that launches one GEMM workgroup per work item
    (U15H_PERSIST=0) instead of one persistent workgroup per CU."""
    o = _ops_with_env("U15H_PERSIST", "0")
    yield o
    torch.cuda.synchronize()
    o.close()


@pytest.mark.parametrize("Mu,Mg,K,N", [(128, 4096, 4096, 4096),
                                       (128, 4096, 12288, 4096),
                                       (37, 263, 1032, 264), (1, 1, 8, 8)])
def test_persistent_launch_bit_identical(ops, ops_per_item, Mu, Mg, K, N):
    """A persistent workgroup computes each of its items exactly as a
    one-item workgroup would: same MFMAs, same K order, same split shares
    (the config-2 down projection has a split tail)."""
    g = torch.Generator(device="cuda").manual_seed(Mu + K)
    M = Mu + Mg
    x = torch.randn(M, K, generator=g, device="cuda").to(torch.bfloat16)
    wu = (torch.randn(N, K, generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    wg = (torch.randn(N, K, generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    outs = []
    for o in (ops, ops_per_item):
        y = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
        o.mot_linear(x, Mu, Mg, K, [dict(w_und=wu, w_gen=wg, y=y)])
        outs.append(y)
    torch.cuda.synchronize()
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))


@pytest.fixture(scope="module")
def ops_mfma32():
    """The 8-wave workgroup running 32x32x16 MFMAs for bf16 (U15H_MFMA16=0;
    the default build runs 16x16x32)."""
    o = _ops_with_env("U15H_MFMA16", "0")
    yield o
    torch.cuda.synchronize()
    o.close()


@pytest.mark.parametrize("Mu,Mg,K,N", [(37, 263, 1032, 264), (128, 4096, 4096, 4096),
                                       (0, 300, 12288, 520)])
def test_mfma32_bf16_agrees(ops, ops_mfma32, Mu, Mg, K, N):
    """bf16 GEMM (with bias) and fused SwiGLU: the default 16x16x32 build
    against the 32x32x16 build, and both against the oracle."""
    M = Mu + Mg
    g = torch.Generator(device="cuda").manual_seed(K + N + 1)
    x = torch.randn(M, K, generator=g, device="cuda").to(torch.bfloat16)
    ws = [(torch.randn(N, K, generator=g, device="cuda") * 0.02).to(torch.bfloat16)
          for _ in range(4)]
    bias = torch.randn(N, generator=g, device="cuda").to(torch.bfloat16)
    outs = []
    for o in (ops, ops_mfma32):
        y = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
        h = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
        o.mot_linear(x, Mu, Mg, K, [dict(w_und=ws[0], w_gen=ws[1], bias_und=bias,
                                         bias_gen=bias, y=y)])
        o.mot_gate_up_swiglu(x, Mu, Mg, K, ws[0], ws[1], ws[2], ws[3], h)
        outs.append((y, h))
    torch.cuda.synchronize()
    for a, b in ((outs[0][0], outs[1][0]), (outs[0][1], outs[1][1])):
        fa, fb = host_f32(a), host_f32(b)
        assert rel_l2(fa, fb) < 4e-3 and max_rel(fa, fb) <= MAX_REL
    xb, bb = host_bits(x), host_bits(bias)
    for r in sorted({0, max(Mu - 1, 0), Mu, M - 1}):
        w = host_bits(ws[0] if r < Mu else ws[1])
        ref = oracle.linear_bf16(xb, w, bb, row_ids=np.array([r], np.int32))
        for y, _ in outs:
            assert max_rel(host_f32(y)[r:r + 1], ref) <= MAX_REL
