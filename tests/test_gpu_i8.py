"""GPU parity of the int8 tier against the CPU oracle.

Bars: quantised codes and scales, and the raw int32 accumulators, are
BIT-EXACT; the fused-dequant bf16 output is bit-exact against the oracle's
dequant of the exact accumulators (same fp32 expression), and within
max-rel-err 1e-2 of the unrounded (double) dequantised value.
"""
import numpy as np
import pytest
import torch

import oracle
from helpers import dev_bf16, host_bits, host_f32, max_rel, rand_bf16_bits, rel_l2

pytestmark = pytest.mark.gpu


def quant_gpu(ops, xb):
    rows, K = xb.shape
    x = dev_bf16(xb)
    q = torch.empty(rows, K, dtype=torch.int8, device="cuda")
    s = torch.empty(rows, dtype=torch.float32, device="cuda")
    ops.quant_rows_i8(x, q, s)
    torch.cuda.synchronize()
    return q, s


def test_quant_rows_bit_exact(ops):
    rng = np.random.default_rng(20)
    rows = [rng.standard_normal(4096, dtype=np.float32) * 3,
            np.zeros(4096, np.float32),
            np.concatenate([np.zeros(4095, np.float32), [-5.0]]).astype(np.float32),
            rng.standard_normal(4096, dtype=np.float32) * 1e-30,
            np.array([127.0, 2.5, -2.5, 0.5, -0.5, 1.5, -126.5] + [0.0] * 4089,
                     np.float32)]
    xb = oracle.f32_to_bf16(np.concatenate([np.stack(rows),
                                            rng.standard_normal((200, 4096)).astype(np.float32)]))
    q, s = quant_gpu(ops, xb)
    qo, so = oracle.quant_rows_i8(xb)
    assert np.array_equal(q.cpu().numpy(), qo)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), so.view(np.uint32))
    assert list(q[4, :7].cpu().numpy()) == [127, 3, -3, 1, -1, 2, -127]


def test_quant_rows_every_tie(ops):
    """Every half-integer quotient from -126.5 to 126.5 at scales 2^-3, 1
    and 2^5 (amax = 127 * scale, so x / s is exact and each element is a
    tie): the codes round half away from zero, as the oracle's division."""
    half = np.arange(-126.5, 127.0, 1.0)
    rows = []
    for e in (-3, 0, 5):
        row = np.zeros(256, np.float32)
        row[0] = 127.0 * 2.0 ** e
        row[1:1 + half.size] = half * 2.0 ** e
        rows.append(row)
    xb = oracle.f32_to_bf16(np.stack(rows))
    assert np.array_equal(oracle.bf16_to_f32(xb), np.stack(rows))   # exact
    q, s = quant_gpu(ops, xb)
    qo, so = oracle.quant_rows_i8(xb)
    assert np.array_equal(q.cpu().numpy(), qo)
    assert np.array_equal(s.cpu().numpy().view(np.uint32), so.view(np.uint32))
    want = np.sign(half) * np.floor(np.abs(half) + 0.5)
    assert np.array_equal(q.cpu().numpy()[:, 1:1 + half.size],
                          np.tile(want.astype(np.int8), (3, 1)))


def test_quant_rows_tiny_absmax(ops):
    """Rows whose scale is subnormal, including rows whose 1/s overflows
    to +inf (absmax below ~3.7e-37), down to the smallest bf16 subnormal:
    codes and scales bit-exact against the oracle's division."""
    rng = np.random.default_rng(21)
    K = 4096
    rows = []
    for amax in (1e-36, 5e-37, 3.7e-37, 1e-37, 1e-38, 2.0 ** -126, 2.0 ** -130):
        r = rng.uniform(-amax, amax, K).astype(np.float32)
        r[int(rng.integers(K))] = -amax
        rows.append(r)
    sub = np.zeros(K, np.float32)
    sub[::7] = np.float32(2.0 ** -133)              # smallest bf16 subnormal
    sub[3::7] = -np.float32(2.0 ** -133)
    rows.append(sub)
    tie = np.zeros(K, np.float32)                   # exact ties at a tiny scale
    tie[0] = 127.0 * 2.0 ** -120
    tie[1:255] = np.arange(-126.5, 127.0, 1.0) * 2.0 ** -120
    rows.append(tie)
    xb = oracle.f32_to_bf16(np.stack(rows))
    q, s = quant_gpu(ops, xb)
    qo, so = oracle.quant_rows_i8(xb)
    with np.errstate(divide="ignore", over="ignore"):
        assert not np.all(np.isfinite(np.float32(1.0) / so))     # the case is present
    assert np.array_equal(s.cpu().numpy().view(np.uint32), so.view(np.uint32))
    assert np.array_equal(q.cpu().numpy(), qo)


def test_quant_rows_codes_stay_in_range(ops):
    """A NaN element (no oracle value) still gives a code in [-127, 127]:
    the redo test selects the division for it, and the row's other codes
    are the oracle's for the same row with the NaN set to zero."""
    rng = np.random.default_rng(22)
    x = rng.standard_normal((2, 512)).astype(np.float32)
    x[0, 5] = np.nan
    xb = oracle.f32_to_bf16(x)
    q, _ = quant_gpu(ops, xb)
    qh = q.cpu().numpy()
    assert qh.min() >= -127 and qh.max() <= 127
    clean = x.copy()
    clean[0, 5] = 0.0
    qo, _ = oracle.quant_rows_i8(oracle.f32_to_bf16(clean))
    keep = np.ones(512, bool)
    keep[5] = False
    assert np.array_equal(qh[0, keep], qo[0, keep])
    assert np.array_equal(qh[1], qo[1])


# The four-wave builds: 8, 136 and 2048 (one chunk per lane: partial and
# full), 2056 and 4096 (two), 4104 and 8192 (four); 8200: past 8192 but
# not a multiple of 16 (the six-chunk row kernel); 8208, 12288 and 16384:
# the 512-thread build (partial, typical, full); 16400: six chunks and a
# second read
@pytest.mark.parametrize("K", [8, 136, 2048, 2056, 4096, 4104, 8192, 8200, 8208, 12288, 16384, 16400])
def test_quant_rows_other_widths(ops, K):
    rng = np.random.default_rng(K)
    xb = rand_bf16_bits(rng, (33, K))
    q, s = quant_gpu(ops, xb)
    qo, so = oracle.quant_rows_i8(xb)
    assert np.array_equal(q.cpu().numpy(), qo)
    assert np.array_equal(s.cpu().numpy(), so)


def _proj(wq_u, sw_u, wq_g, sw_g, y):
    return dict(wq_und=wq_u, sw_und=sw_u, wq_gen=wq_g, sw_gen=sw_g, y=y)


def test_i32_accumulators_bit_exact_c1(ops):
    """Config 1's split (64 und + 192 gen), K=4096; q, k, v in one launch;
    every accumulator of every projection against the exact CPU GEMM."""
    rng = np.random.default_rng(21)
    Mu, Mg, K = 64, 192, 4096
    M = Mu + Mg
    xq = rng.integers(-127, 128, (M, K), dtype=np.int8)
    Ns = [1024, 512, 512]
    W = [(rng.integers(-127, 128, (n, K), dtype=np.int8),
          rng.integers(-127, 128, (n, K), dtype=np.int8)) for n in Ns]
    ys = [torch.empty(M, n, dtype=torch.int32, device="cuda") for n in Ns]
    projs = [_proj(torch.from_numpy(wu).cuda(), None, torch.from_numpy(wg).cuda(),
                   None, y) for (wu, wg), y in zip(W, ys)]
    ops.mot_gemm_i8_i32(torch.from_numpy(xq).cuda(), Mu, Mg, K, projs)
    torch.cuda.synchronize()
    for (wu, wg), y in zip(W, ys):
        out = y.cpu().numpy()
        assert np.array_equal(out[:Mu], oracle.gemm_i8_i32(xq[:Mu], wu))
        assert np.array_equal(out[Mu:], oracle.gemm_i8_i32(xq[Mu:], wg))


def test_i32_extremes_and_ragged(ops):
    """+-127 everywhere (the largest magnitudes int32 must hold), ragged M
    and N, both groups."""
    Mu, Mg, K, N = 3, 300, 12288, 264
    M = Mu + Mg
    rng = np.random.default_rng(22)
    xq = np.where(rng.random((M, K)) < 0.5, -127, 127).astype(np.int8)
    xq[0] = 127
    wu = np.full((N, K), 127, np.int8)
    wg = np.where(rng.random((N, K)) < 0.5, -127, 127).astype(np.int8)
    wg[5] = -127
    y = torch.empty(M, N, dtype=torch.int32, device="cuda")
    ops.mot_gemm_i8_i32(torch.from_numpy(xq).cuda(), Mu, Mg, K,
                        [_proj(torch.from_numpy(wu).cuda(), None,
                               torch.from_numpy(wg).cuda(), None, y)])
    torch.cuda.synchronize()
    out = y.cpu().numpy()
    assert out[0, 0] == 127 * 127 * K
    assert np.array_equal(out[:Mu], oracle.gemm_i8_i32(xq[:Mu], wu))
    rows = np.array([0, 1, 150, 299], np.int32)
    assert np.array_equal(out[Mu:][rows], oracle.gemm_i8_i32(xq[Mu:], wg, row_ids=rows))
    rs, cs = oracle.i8_product_sums(xq[Mu:], wg)
    assert np.array_equal(out[Mu:].astype(np.int64).sum(axis=1), rs)
    assert np.array_equal(out[Mu:].astype(np.int64).sum(axis=0), cs)


def test_i8_full_pipeline_c2_shape_q_proj(ops):
    """Config 3 at full size for the q projection (128 und + 4096 gen,
    K=N=4096): per-token activation quantisation, per-channel weight
    quantisation, int32 GEMM and fused dequant.  Whole-output int32 check by
    exact row and column sums; sampled rows bit-exact; dequant bit-exact."""
    rng = np.random.default_rng(23)
    Mu, Mg, K, N = 128, 4096, 4096, 4096
    M = Mu + Mg
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(1)).to(torch.bfloat16)
    wu = (torch.randn(N, K, generator=torch.Generator().manual_seed(2)) * 0.02).to(torch.bfloat16)
    wg = (torch.randn(N, K, generator=torch.Generator().manual_seed(3)) * 0.02).to(torch.bfloat16)
    xbits = x.view(torch.int16).numpy().view(np.uint16)
    wubits = wu.view(torch.int16).numpy().view(np.uint16)
    wgbits = wg.view(torch.int16).numpy().view(np.uint16)
    xq, sx = quant_gpu(ops, xbits)
    wqu, swu = quant_gpu(ops, wubits)
    wqg, swg = quant_gpu(ops, wgbits)
    acc = torch.empty(M, N, dtype=torch.int32, device="cuda")
    y = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    ops.mot_gemm_i8_i32(xq, Mu, Mg, K, [_proj(wqu, None, wqg, None, acc)])
    ops.mot_gemm_i8(xq, sx, Mu, Mg, K, [_proj(wqu, swu, wqg, swg, y)])
    torch.cuda.synchronize()
    # quantisers bit-exact against the oracle (sampled rows for speed)
    xq_h, sx_h = xq.cpu().numpy(), sx.cpu().numpy()
    qo, so = oracle.quant_rows_i8(xbits[::97])
    assert np.array_equal(xq_h[::97], qo) and np.array_equal(sx_h[::97], so)
    wqg_h, swg_h = wqg.cpu().numpy(), swg.cpu().numpy()
    wqu_h, swu_h = wqu.cpu().numpy(), swu.cpu().numpy()
    qo, so = oracle.quant_rows_i8(wgbits[::61])
    assert np.array_equal(wqg_h[::61], qo) and np.array_equal(swg_h[::61], so)
    # int32: exact sums over every accumulator, then sampled rows
    acc_h = acc.cpu().numpy()
    for (lo, hi, wq) in ((0, Mu, wqu_h), (Mu, M, wqg_h)):
        rs, cs = oracle.i8_product_sums(xq_h[lo:hi], wq)
        assert np.array_equal(acc_h[lo:hi].astype(np.int64).sum(axis=1), rs)
        assert np.array_equal(acc_h[lo:hi].astype(np.int64).sum(axis=0), cs)
    rows = np.array([0, 77, 127, 128, 2000, 4223], np.int32)
    for r in rows:
        wq = wqu_h if r < Mu else wqg_h
        assert np.array_equal(acc_h[r:r + 1], oracle.gemm_i8_i32(xq_h[r:r + 1], wq))
    # dequant epilogue: bit-exact vs the oracle's expression, 1e-2 vs double
    y_h = host_bits(y)
    for (lo, hi, sw) in ((0, Mu, swu_h), (Mu, M, swg_h)):
        exp = oracle.dequant_bf16(acc_h[lo:hi], sx_h[lo:hi], sw)
        assert np.array_equal(y_h[lo:hi], exp)
        f64 = oracle.dequant_f64(acc_h[lo:hi], sx_h[lo:hi], sw)
        assert max_rel(oracle.bf16_to_f32(y_h[lo:hi]), f64) <= 1e-2
    # and the tier approximates the bf16 product (quantisation error only)
    ref = oracle.linear_bf16(xbits, wgbits,
                             row_ids=np.array([Mu + 200, Mu + 3000], np.int32))
    assert rel_l2(host_f32(y)[[Mu + 200, Mu + 3000]], ref) < 0.03


def test_linear_int8_route_on_and_decline(ops):
    """u15h_linear with the tier ON: qualifying shapes take the int8 route
    (== quantise + int8 GEMM + dequant, bit for bit); small M declines to
    the bf16 path unchanged (src/u15-metal-ops.cc:291-306)."""
    rng = np.random.default_rng(24)
    K, N = 1024, 256
    Mbig = max(ops.i8_min_m(), 1024)
    xb = rand_bf16_bits(rng, (Mbig, K))
    wb = rand_bf16_bits(rng, (N, K), 0.02)
    x, w = dev_bf16(xb), dev_bf16(wb)
    y_bf16 = torch.empty(Mbig, N, dtype=torch.bfloat16, device="cuda")
    ops.enable_i8_gemm(False)
    ops.linear(x, w, None, y_bf16, Mbig, K, N)
    try:
        on = ops.enable_i8_gemm(True)
        import os
        if os.environ.get("U15H_I8_GEMM", "") == "0":
            assert not on
            return
        assert on
        y_i8 = torch.empty_like(y_bf16)
        ops.linear(x, w, None, y_i8, Mbig, K, N)
        small = torch.empty(8, N, dtype=torch.bfloat16, device="cuda")
        ops.linear(x[:8], w, None, small, 8, K, N)
        torch.cuda.synchronize()
        # explicit pipeline
        xq, sx = quant_gpu(ops, xb)
        wq, sw = quant_gpu(ops, wb)
        y_ref = torch.empty_like(y_bf16)
        ops.mot_gemm_i8(xq, sx, 0, Mbig, K, [_proj(None, None, wq, sw, y_ref)])
        torch.cuda.synchronize()
        assert torch.equal(y_i8.cpu(), y_ref.cpu())
        assert not torch.equal(y_i8.cpu(), y_bf16.cpu())
        assert torch.equal(small.cpu(), y_bf16[:8].cpu())   # declined
        assert rel_l2(host_f32(y_i8), host_f32(y_bf16)) < 0.03
    finally:
        ops.enable_i8_gemm(False)
        ops.release_i8_scratch()


def test_linear_q_int8_interception(ops):
    """u15h_linear_q with the tier ON: the dequant-once expansion takes
    u15h_linear's route, so at M >= the row floor the result equals
    quantise(x) + quantise(expansion) + int8 GEMM + dequant bit for bit
    (the reference's linear_mma_q_ re-enters linear_mma_'s interception,
    src/u15-metal-ops.cc:291-300, 393-399); below the floor it is the dense
    bf16 result on the expansion."""
    import os
    rng = np.random.default_rng(27)
    K, N, G = 1024, 264, 64
    Mbig = max(ops.i8_min_m(), 1024)
    w = oracle.randn_mt(91, N * K, 0.05).reshape(N, K)
    codes, sc, bi, _ = oracle.pack_affine(w, 8, G)
    wd = oracle.dequant_affine(codes, sc, bi, 8, G, K)
    qw = (torch.from_numpy(codes.view(np.int32)).cuda(), dev_bf16(sc), dev_bf16(bi), 8, G)
    xb = rand_bf16_bits(rng, (Mbig, K))
    x, wd_dev = dev_bf16(xb), dev_bf16(wd)
    y_dense = torch.empty(Mbig, N, dtype=torch.bfloat16, device="cuda")
    ops.enable_i8_gemm(False)
    ops.linear_q(x, qw, None, y_dense, Mbig, K, N)
    try:
        on = ops.enable_i8_gemm(True)
        if os.environ.get("U15H_I8_GEMM", "") == "0":
            assert not on
            return
        assert on
        y_q = torch.empty_like(y_dense)
        ops.linear_q(x, qw, None, y_q, Mbig, K, N)
        small = torch.empty(8, N, dtype=torch.bfloat16, device="cuda")
        ops.linear_q(x[:8], qw, None, small, 8, K, N)
        small_dense = torch.empty_like(small)
        ops.linear(x[:8], wd_dev, None, small_dense, 8, K, N)
        torch.cuda.synchronize()
        xq, sx = quant_gpu(ops, xb)
        wq, sw = quant_gpu(ops, wd)
        y_ref = torch.empty_like(y_dense)
        ops.mot_gemm_i8(xq, sx, 0, Mbig, K, [_proj(None, None, wq, sw, y_ref)])
        y_lin = torch.empty_like(y_dense)
        ops.linear(x, wd_dev, None, y_lin, Mbig, K, N)     # the same route
        torch.cuda.synchronize()
        assert torch.equal(y_q.cpu(), y_ref.cpu())
        assert torch.equal(y_q.cpu(), y_lin.cpu())
        assert not torch.equal(y_q.cpu(), y_dense.cpu())
        # declined (below the int8 floor): the dense route on the expansion
        assert torch.equal(small.cpu(), small_dense.cpu())
        # the int32 accumulators behind it are the oracle's, exactly
        qo, so = oracle.quant_rows_i8(wd)
        assert np.array_equal(wq.cpu().numpy(), qo)
        rows = np.array([0, 511, Mbig - 1], np.int32)
        xq_h = xq.cpu().numpy()
        acc = oracle.gemm_i8_i32(xq_h, qo, row_ids=rows)
        exp = oracle.dequant_bf16(acc, sx.cpu().numpy()[rows], so)
        assert np.array_equal(host_bits(y_q)[rows], exp)
    finally:
        ops.enable_i8_gemm(False)
        ops.release_i8_scratch()


def test_i32_split_tail_bit_exact(ops):
    """An int8 launch whose tiles are split into K shares (6 tiles of a
    12288-deep K): the shares' int32 sums are exact, so the result equals
    the exact CPU GEMM bit for bit."""
    rng = np.random.default_rng(25)
    Mu, Mg, K, N = 37, 263, 12288, 264
    M = Mu + Mg
    xq = rng.integers(-127, 128, (M, K), dtype=np.int8)
    wu = rng.integers(-127, 128, (N, K), dtype=np.int8)
    wg = rng.integers(-127, 128, (N, K), dtype=np.int8)
    y = torch.empty(M, N, dtype=torch.int32, device="cuda")
    ops.mot_gemm_i8_i32(torch.from_numpy(xq).cuda(), Mu, Mg, K,
                        [_proj(torch.from_numpy(wu).cuda(), None,
                               torch.from_numpy(wg).cuda(), None, y)])
    torch.cuda.synchronize()
    out = y.cpu().numpy()
    assert np.array_equal(out[:Mu], oracle.gemm_i8_i32(xq[:Mu], wu))
    rows = np.array([0, 100, 262], np.int32)
    assert np.array_equal(out[Mu:][rows], oracle.gemm_i8_i32(xq[Mu:], wg, row_ids=rows))
    rs, cs = oracle.i8_product_sums(xq[Mu:], wg)
    assert np.array_equal(out[Mu:].astype(np.int64).sum(axis=1), rs)
    assert np.array_equal(out[Mu:].astype(np.int64).sum(axis=0), cs)


def test_i32_per_item_launch_bit_exact():
    """One workgroup per work item (U15H_PERSIST=0) on the int8 path: exact
    accumulators, split shares included, equal to the persistent launch."""
    import os
    old = os.environ.get("U15H_PERSIST")
    os.environ["U15H_PERSIST"] = "0"
    try:
        import u15h
        ops_pi = u15h.Ops(0)
    finally:
        if old is None:
            del os.environ["U15H_PERSIST"]
        else:
            os.environ["U15H_PERSIST"] = old
    rng = np.random.default_rng(26)
    Mu, Mg, K, N = 37, 263, 12288, 264
    M = Mu + Mg
    xq = rng.integers(-127, 128, (M, K), dtype=np.int8)
    wu = rng.integers(-127, 128, (N, K), dtype=np.int8)
    wg = rng.integers(-127, 128, (N, K), dtype=np.int8)
    y = torch.empty(M, N, dtype=torch.int32, device="cuda")
    ops_pi.mot_gemm_i8_i32(torch.from_numpy(xq).cuda(), Mu, Mg, K,
                           [_proj(torch.from_numpy(wu).cuda(), None,
                                  torch.from_numpy(wg).cuda(), None, y)])
    torch.cuda.synchronize()
    out = y.cpu().numpy()
    assert np.array_equal(out[:Mu], oracle.gemm_i8_i32(xq[:Mu], wu))
    rs, cs = oracle.i8_product_sums(xq[Mu:], wg)
    assert np.array_equal(out[Mu:].astype(np.int64).sum(axis=1), rs)
    assert np.array_equal(out[Mu:].astype(np.int64).sum(axis=0), cs)
    ops_pi.close()


@pytest.mark.parametrize("Mu,Mg,K,N", [(128, 4096, 4096, 4096), (37, 263, 12288, 264)])
def test_i32_four_wave_workgroup_bit_exact(Mu, Mg, K, N):
    """The 4-wave GEMM workgroup (U15H_WAVES=4: 16x16x64 MFMAs, 128x128
    per wave): exact accumulators -- every row sum and column sum, sampled
    rows in full, split-K tail included."""
    import os
    import u15h
    old = os.environ.get("U15H_WAVES")
    os.environ["U15H_WAVES"] = "4"
    try:
        o4 = u15h.Ops(0)
    finally:
        if old is None:
            del os.environ["U15H_WAVES"]
        else:
            os.environ["U15H_WAVES"] = old
    rng = np.random.default_rng(K + N)
    M = Mu + Mg
    xq = rng.integers(-127, 128, (M, K), dtype=np.int8)
    wu = rng.integers(-127, 128, (N, K), dtype=np.int8)
    wg = rng.integers(-127, 128, (N, K), dtype=np.int8)
    y = torch.empty(M, N, dtype=torch.int32, device="cuda")
    o4.mot_gemm_i8_i32(torch.from_numpy(xq).cuda(), Mu, Mg, K,
                       [_proj(torch.from_numpy(wu).cuda(), None,
                              torch.from_numpy(wg).cuda(), None, y)])
    torch.cuda.synchronize()
    out = y.cpu().numpy()
    for lo, hi, w in ((0, Mu, wu), (Mu, M, wg)):
        rs, cs = oracle.i8_product_sums(xq[lo:hi], w)
        assert np.array_equal(out[lo:hi].astype(np.int64).sum(axis=1), rs)
        assert np.array_equal(out[lo:hi].astype(np.int64).sum(axis=0), cs)
    for r in (0, Mu - 1, Mu, M // 2, M - 1):
        w = wu if r < Mu else wg
        assert np.array_equal(out[r:r + 1], oracle.gemm_i8_i32(xq[r:r + 1], w))
    # the fused dequant epilogue of the same workgroup, on the checked
    # accumulators: bit-exact against the oracle's expression
    sx = (rng.random(M, dtype=np.float32) * 0.01 + 1e-4).astype(np.float32)
    swu = (rng.random(N, dtype=np.float32) * 0.01 + 1e-4).astype(np.float32)
    swg = (rng.random(N, dtype=np.float32) * 0.01 + 1e-4).astype(np.float32)
    yb = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    o4.mot_gemm_i8(torch.from_numpy(xq).cuda(), torch.from_numpy(sx).cuda(), Mu, Mg,
                   K, [_proj(torch.from_numpy(wu).cuda(), torch.from_numpy(swu).cuda(),
                             torch.from_numpy(wg).cuda(), torch.from_numpy(swg).cuda(),
                             yb)])
    torch.cuda.synchronize()
    yb_h = host_bits(yb)
    for lo, hi, sw in ((0, Mu, swu), (Mu, M, swg)):
        assert np.array_equal(yb_h[lo:hi], oracle.dequant_bf16(out[lo:hi], sx[lo:hi], sw))
    o4.close()
