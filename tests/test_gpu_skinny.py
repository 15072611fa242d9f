"""The skinny GEMM route: a bf16 batch whose problems all have at most 128
rows and K a multiple of 64 runs on skinny_reg_kernel (<= 16 rows, 16
output columns per workgroup) or skinny_lds_kernel (64 columns), weights
streamed into registers, K shares summed in order by skinny_reduce_kernel.
Checked against the oracle at the reference's bars (max-rel <= 1e-2,
rel-L2 < 4e-3, tests/u15-kernels-test.cc:55) and against the tiled GEMM of
a context built with U15H_SKINNY=0, over the share counts the planner
picks (1 to 16), the four row-group builds (<= 16, 32, 64, 128 rows),
column counts that leave waves or lanes of a block past N, bias, and
grouped und + gen batches; and u15h_linear_q's direct route below the row
floor, which reads 4- and 8-bit affine packs in the same kernels."""
import os

import numpy as np
import pytest
import torch

import oracle
import u15h
from helpers import dev_bf16, host_bits, host_f32, max_rel, rand_bf16_bits, rel_l2

pytestmark = pytest.mark.gpu

MAX_REL = 1e-2
REF_BAR = 4e-3


@pytest.fixture(scope="module")
def ops_tiled():
    old = os.environ.get("U15H_SKINNY")
    os.environ["U15H_SKINNY"] = "0"
    try:
        o = u15h.Ops(0)
    finally:
        if old is None:
            del os.environ["U15H_SKINNY"]
        else:
            os.environ["U15H_SKINNY"] = old
    yield o
    torch.cuda.synchronize()
    o.close()


# (M, K, N): shares S picked by the planner in the comment
CASES = [
    (1, 4096, 6144),     # S=4, one row (the <=16-row build)
    (5, 1024, 264),      # S=2, N leaves waves 1..3 of the last block idle
    (16, 4096, 4096),    # S=8
    (17, 128, 72),       # S=1 (two K-blocks), the <=32-row build
    (64, 12288, 512),    # S=16, the <=64-row build
    (65, 4096, 1032),    # the <=96-row build, ragged rows, N % 64 = 8
    (96, 4096, 6144),    # the <=96-row build, full, S=4
    (100, 4096, 1000),   # the <=128-row build, ragged rows, N % 64 = 40
    (128, 4096, 6144),   # config-5 und rows at q|k|v width, S=4
    (128, 12288, 4096),  # config-5 und rows at the down projection, S=8
]


@pytest.mark.parametrize("M,K,N", CASES)
def test_skinny_linear_vs_oracle_and_tiled(ops, ops_tiled, M, K, N):
    rng = np.random.default_rng(M * 7 + K + N)
    xb = rand_bf16_bits(rng, (M, K))
    wb = rand_bf16_bits(rng, (N, K), 0.02)
    bb = rand_bf16_bits(rng, (N,), 0.5)
    x, w, b = dev_bf16(xb), dev_bf16(wb), dev_bf16(bb)
    y = torch.full((M, N), 7.0, dtype=torch.bfloat16, device="cuda")
    y2 = torch.empty_like(y)
    ops.linear(x, w, b, y, M, K, N)
    ops_tiled.linear(x, w, b, y2, M, K, N)
    torch.cuda.synchronize()
    a, t = host_f32(y), host_f32(y2)
    assert np.all(np.isfinite(a))
    assert rel_l2(a, t) < REF_BAR and max_rel(a, t) <= MAX_REL
    rows = np.unique(np.array([0, M // 2, M - 1], np.int32))
    ref = oracle.linear_bf16(xb, wb, bb, row_ids=rows)
    assert max_rel(a[rows], ref) <= MAX_REL
    assert rel_l2(a[rows], ref) < REF_BAR


def test_skinny_zero_weights_give_the_bias(ops):
    """Every output column is written, and only the bias survives a zero
    weight: a share or a wave that misses its columns would leave 7.0 or
    add garbage."""
    M, K, N = 77, 2048, 328
    rng = np.random.default_rng(3)
    x = dev_bf16(rand_bf16_bits(rng, (M, K)))
    w = torch.zeros(N, K, dtype=torch.bfloat16, device="cuda")
    bb = rand_bf16_bits(rng, (N,), 1.0)
    y = torch.full((M, N), 7.0, dtype=torch.bfloat16, device="cuda")
    ops.linear(x, w, dev_bf16(bb), y, M, K, N)
    torch.cuda.synchronize()
    assert np.array_equal(host_bits(y), np.broadcast_to(bb, (M, N)))


def test_skinny_identity_is_exact(ops):
    """One nonzero product per output: the K order cannot round it."""
    M, K = 50, 256
    rng = np.random.default_rng(4)
    xb = rand_bf16_bits(rng, (M, K))
    eye = oracle.f32_to_bf16(np.eye(K, dtype=np.float32))
    y = torch.empty(M, K, dtype=torch.bfloat16, device="cuda")
    ops.linear(dev_bf16(xb), dev_bf16(eye), None, y, M, K, K)
    torch.cuda.synchronize()
    assert np.array_equal(host_bits(y), xb)


@pytest.mark.parametrize("Mu,Mg", [(128, 0), (0, 128), (3, 100), (128, 128)])
def test_skinny_mot_linear_grouped(ops, ops_tiled, Mu, Mg):
    """q | k | v of both weight sets in one skinny batch (up to six problems
    of three widths), each row against its own weight set."""
    K = 4096
    M = Mu + Mg
    rng = np.random.default_rng(Mu * 3 + Mg)
    xb = rand_bf16_bits(rng, (M, K))
    x = dev_bf16(xb)
    projs, projs2, host = [], [], []
    for N in (4096, 1024, 1024):
        wu = rand_bf16_bits(rng, (N, K), 0.02)
        wg = rand_bf16_bits(rng, (N, K), 0.02)
        y = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
        y2 = torch.empty_like(y)
        projs.append(dict(w_und=dev_bf16(wu), w_gen=dev_bf16(wg), y=y))
        projs2.append(dict(projs[-1], y=y2))
        host.append((wu, wg, y, y2))
    ops.mot_linear(x, Mu, Mg, K, projs)
    ops_tiled.mot_linear(x, Mu, Mg, K, projs2)
    torch.cuda.synchronize()
    rows = np.unique(np.array([0, max(Mu - 1, 0), Mu, M - 1], np.int32))
    rows = rows[rows < M]
    for wu, wg, y, y2 in host:
        a = host_f32(y)
        assert rel_l2(a, host_f32(y2)) < REF_BAR
        for r in rows:
            w = wu if r < Mu else wg
            ref = oracle.linear_bf16(xb, w, row_ids=np.array([r], np.int32))
            assert max_rel(a[r:r + 1], ref) <= MAX_REL
            assert rel_l2(a[r:r + 1], ref) < REF_BAR


def test_skinny_repeat_is_bit_identical(ops):
    """The shares are summed in a fixed order: two calls agree bit for bit
    (the second after another shape has used the same workspace)."""
    M, K, N = 128, 4096, 6144
    g = torch.Generator(device="cuda").manual_seed(11)
    x = torch.randn(M, K, generator=g, device="cuda").to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g, device="cuda") * 0.02).to(torch.bfloat16)
    y1 = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    y2 = torch.empty_like(y1)
    ops.linear(x, w, None, y1, M, K, N)
    xs = torch.randn(16, K, generator=g, device="cuda").to(torch.bfloat16)
    ys = torch.empty(16, N, dtype=torch.bfloat16, device="cuda")
    ops.linear(xs, w, None, ys, 16, K, N)
    ops.linear(x, w, None, y2, M, K, N)
    torch.cuda.synchronize()
    assert torch.equal(y1.view(torch.int16), y2.view(torch.int16))


def _pack_dev(codes, sc, bi, bits, group):
    return (torch.from_numpy(np.ascontiguousarray(codes, np.uint32).view(np.int32)).cuda(),
            dev_bf16(sc), dev_bf16(bi), bits, group)


@pytest.mark.parametrize("bits,group", [(8, 64), (8, 32), (4, 64), (4, 32)])
@pytest.mark.parametrize("M", [1, 16, 17, 64, 95, 96])
def test_linear_q_direct_route(ops, bits, group, M):
    """Below the row floor (96, the reference's _mma_q_min_m) u15h_linear_q
    reads the affine pack directly (the reference's steel qmm route,
    src/u15-metal-ops.cc:402-431), dequantising in registers to the
    expansion's bf16 weights: bit-equal to u15h_linear on the expansion
    (which at these rows runs the same skinny kernel), and within the bars
    of the oracle.  At 96 rows it is dequant-once + the dense route."""
    K, N = 2048, 328
    w = oracle.randn_mt(bits * 100 + group + M, N * K, 0.05).reshape(N, K)
    codes, sc, bi, _ = oracle.pack_affine(w, bits, group)
    wd = oracle.dequant_affine(codes, sc, bi, bits, group, K)
    rng = np.random.default_rng(M * 11 + bits)
    xb = rand_bf16_bits(rng, (M, K))
    bb = rand_bf16_bits(rng, (N,), 0.5)
    x, b = dev_bf16(xb), dev_bf16(bb)
    y = torch.full((M, N), 7.0, dtype=torch.bfloat16, device="cuda")
    y2 = torch.empty_like(y)
    ops.linear_q(x, _pack_dev(codes, sc, bi, bits, group), b, y, M, K, N)
    ops.linear(x, dev_bf16(wd), b, y2, M, K, N)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), y2.view(torch.int16))
    rows = np.unique(np.array([0, M // 2, M - 1], np.int32))
    ref = oracle.linear_bf16(xb, wd, bb, row_ids=rows)
    a = host_f32(y)[rows]
    assert max_rel(a, ref) <= MAX_REL and rel_l2(a, ref) < REF_BAR
