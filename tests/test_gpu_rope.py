"""GPU parity of the split q/k norm and the three-way split RoPE.

Bar: the reference's bf16 bar, rel-L2 < 4e-3 (tests/u15-kernels-test.cc:55,
used by its test_split_head), against the oracle on the same bf16 inputs;
max-rel <= 1e-2 on top.  The tables come from u15h_build_rope_tables (host
code), pinned bit-equal to the oracle in tests/test_abi.py.
"""
import numpy as np
import pytest
import torch

import oracle
import u15h
from helpers import dev_bf16, host_f32, max_rel, rel_l2

pytestmark = pytest.mark.gpu

BAR = 4e-3
MAX_REL = 1e-2


def widen(bits):
    return oracle.bf16_to_f32(bits)


def ref_case():
    """test_split_head (tests/u15-kernels-test.cc:124-153)."""
    H, T, D = 4, 12, 32
    x = oracle.randn_mt(7, T * H * D).reshape(T, H * D)
    w = oracle.randn_mt(8, D, 0.2) + np.float32(1.0)
    pt = np.array(list(range(5)) + [5] * (T - 5))
    ph = np.array([0] * 5 + [i // 7 for i in range(T - 5)])
    pw = np.array([0] * 5 + [i % 7 for i in range(T - 5)])
    return H, T, D, x, w[: D // 2], w[D // 2:], pt, ph, pw


def dev_f32(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()


def run(ops, xb, wtb, whb, tabs, H, D, d_t, d_h, fused):
    x = dev_bf16(xb)
    cs, sn = (dev_f32(t) for t in tabs)
    if fused:
        ops.split_qk_norm_rope(x, dev_bf16(wtb), dev_bf16(whb), cs, sn, H, D,
                               d_t, d_h)
    else:
        ops.split_qk_norm(x, dev_bf16(wtb), dev_bf16(whb), H, D)
        ops.split_rope(x, cs, sn, H, D, d_t, d_h)
    torch.cuda.synchronize()
    return host_f32(x)


@pytest.mark.parametrize("fused", [False, True])
def test_reference_split_head_case(ops, fused):
    H, T, D, x, w_t, w_hw, pt, ph, pw = ref_case()
    d_t, d_h = D // 2, D // 4
    xb, wtb, whb = (oracle.f32_to_bf16(a) for a in (x, w_t, w_hw))
    tabs = u15h.build_rope_tables(pt, ph, pw, D, d_t, d_h)
    got = run(ops, xb, wtb, whb, tabs, H, D, d_t, d_h, fused)
    # the reference's own comparison: its CPU path on the f32 inputs
    ref32 = oracle.split_qk_norm_rope(x, w_t, w_hw, pt, ph, pw, H, D, d_t, d_h)
    assert rel_l2(got, ref32) < BAR
    # and on the same bf16 inputs
    ref = oracle.split_qk_norm_rope(widen(xb), widen(wtb), widen(whb), pt, ph,
                                    pw, H, D, d_t, d_h)
    assert rel_l2(got, ref) < BAR
    assert max_rel(got, ref) <= MAX_REL
    # negative controls (tests/u15-kernels-test.cc:208-257): the GPU output
    # must be far from the h/w-swapped and the whole-head-norm answers
    swapped = oracle.split_qk_norm_rope(widen(xb), widen(wtb), widen(whb), pt,
                                        pw, ph, H, D, d_t, d_h)
    assert rel_l2(got, swapped) > 1e-2
    whole = oracle.rms_norm(widen(xb).reshape(T * H, D),
                            np.concatenate([widen(wtb), widen(whb)]),
                            1e-6).reshape(T, H * D)
    whole = oracle.split_qk_norm_rope(whole, w_t, w_hw, pt, ph, pw, H, D, d_t,
                                      d_h, norm=False)
    assert rel_l2(got, whole) > 1e-2


def test_swapped_tables_are_detected(ops):
    """The kernel really reads the h and w ranges from their own positions."""
    H, T, D, x, w_t, w_hw, pt, ph, pw = ref_case()
    d_t, d_h = D // 2, D // 4
    xb, wtb, whb = (oracle.f32_to_bf16(a) for a in (x, w_t, w_hw))
    bad = u15h.build_rope_tables(pt, pw, ph, D, d_t, d_h)
    got = run(ops, xb, wtb, whb, bad, H, D, d_t, d_h, True)
    ref = oracle.split_qk_norm_rope(widen(xb), widen(wtb), widen(whb), pt, ph,
                                    pw, H, D, d_t, d_h)
    assert rel_l2(got, ref) > 1e-2


@pytest.mark.parametrize("H", [32, 8])
@pytest.mark.parametrize("fused", [False, True])
def test_model_shape_q_and_k(ops, H, fused):
    """Config 2's q (32 heads) and k (8 heads) at head_dim 128 = [64 | 32 |
    32]: 128 text tokens then a 64x64 image block sharing t = 128."""
    T, D, d_t, d_h = 4224, 128, 64, 32
    rng = np.random.default_rng(H)
    xb = oracle.f32_to_bf16(rng.standard_normal((T, H * D)).astype(np.float32))
    wtb = oracle.f32_to_bf16(rng.normal(1, 0.2, D // 2).astype(np.float32))
    whb = oracle.f32_to_bf16(rng.normal(1, 0.2, D // 2).astype(np.float32))
    i = np.arange(T - 128)
    pt = np.concatenate([np.arange(128), np.full(T - 128, 128)])
    ph = np.concatenate([np.zeros(128, int), i // 64])
    pw = np.concatenate([np.zeros(128, int), i % 64])
    tabs = u15h.build_rope_tables(pt, ph, pw, D, d_t, d_h)
    got = run(ops, xb, wtb, whb, tabs, H, D, d_t, d_h, fused)
    rows = np.array([0, 1, 127, 128, 129, 2000, 4223])
    ref = oracle.split_qk_norm_rope(widen(xb)[rows], widen(wtb), widen(whb),
                                    pt[rows], ph[rows], pw[rows], H, D, d_t,
                                    d_h)
    assert rel_l2(got[rows], ref) < BAR
    assert max_rel(got[rows], ref) <= MAX_REL


def test_fused_is_at_least_as_close(ops):
    """The fused pass keeps the normalised row in f32; the two-step pass
    rounds it to bf16 in between, as the reference's two kernels do."""
    H, T, D = 16, 300, 128
    rng = np.random.default_rng(2)
    xb = oracle.f32_to_bf16(rng.standard_normal((T, H * D)).astype(np.float32))
    wtb = oracle.f32_to_bf16(rng.normal(1, 0.2, D // 2).astype(np.float32))
    whb = oracle.f32_to_bf16(rng.normal(1, 0.2, D // 2).astype(np.float32))
    pt = rng.integers(0, 5000, T)
    ph = rng.integers(0, 64, T)
    pw = rng.integers(0, 64, T)
    tabs = u15h.build_rope_tables(pt, ph, pw, D, 64, 32)
    ref = oracle.split_qk_norm_rope(widen(xb), widen(wtb), widen(whb), pt, ph,
                                    pw, H, D, 64, 32)
    two = run(ops, xb, wtb, whb, tabs, H, D, 64, 32, False)
    one = run(ops, xb, wtb, whb, tabs, H, D, 64, 32, True)
    assert rel_l2(one, ref) < BAR and rel_l2(two, ref) < BAR
    assert rel_l2(one, ref) <= rel_l2(two, ref) * 1.05


def test_norm_rope_rejects_bad_shapes(ops):
    x = torch.zeros(4, 2 * 128, dtype=torch.bfloat16, device="cuda")
    cs = torch.zeros(4, 128, dtype=torch.float32, device="cuda")
    import ctypes
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    L, c = ops.lib, ops.ctx
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    assert L.u15h_split_rope(c, s, p(x), p(cs), p(cs), 2, 4, 128, 64, 30) == u15h.EINVAL
    assert L.u15h_split_rope(c, s, p(x), p(cs), p(cs), 2, 4, 128, 63, 32) == u15h.EINVAL
    assert L.u15h_split_rope(c, s, p(x), None, p(cs), 2, 4, 128, 64, 32) == u15h.EINVAL
    assert L.u15h_split_qk_norm(c, s, p(x), None, None, 2, 4, 128, 1e-6) == u15h.EINVAL
    assert L.u15h_split_qk_norm(c, s, p(x), p(x), p(x), 1, 1, 1024, 1e-6) == u15h.EINVAL
    # zero tokens is a no-op
    assert L.u15h_split_rope(c, s, None, None, None, 2, 0, 128, 64, 32) == u15h.OK


@pytest.mark.parametrize("D,d_t,d_h", [(64, 32, 16), (128, 64, 32), (256, 128, 64)])
@pytest.mark.parametrize("misaligned", [False, True])
def test_chunked_and_row_kernels(ops, D, d_t, d_h, misaligned):
    """Two kernels serve these entry points: one 16-byte chunk per thread
    (16-byte-aligned operands, power-of-two ranges) and one row per wave
    (everything else).  A row view 8 bytes off alignment takes the second;
    both match the oracle, fused and two-step."""
    H, T = 8, 97
    rng = np.random.default_rng(D + misaligned)
    xb = oracle.f32_to_bf16(rng.standard_normal((T, H * D)).astype(np.float32))
    wtb = oracle.f32_to_bf16(rng.normal(1, 0.2, D // 2).astype(np.float32))
    whb = oracle.f32_to_bf16(rng.normal(1, 0.2, D // 2).astype(np.float32))
    pt = rng.integers(0, 3000, T)
    ph = rng.integers(0, 64, T)
    pw = rng.integers(0, 64, T)
    cs, sn = (dev_f32(t) for t in u15h.build_rope_tables(pt, ph, pw, D, d_t, d_h))
    ref = oracle.split_qk_norm_rope(widen(xb), widen(wtb), widen(whb), pt, ph,
                                    pw, H, D, d_t, d_h)
    for fused in (True, False):
        flat = torch.zeros(T * H * D + 4, dtype=torch.bfloat16, device="cuda")
        x = flat[4:] if misaligned else flat[:-4]
        x.view(T, H * D).copy_(dev_bf16(xb))
        x2 = x.view(T, H * D)
        assert (x2.data_ptr() % 16 != 0) == misaligned
        if fused:
            ops.split_qk_norm_rope(x2, dev_bf16(wtb), dev_bf16(whb), cs, sn, H, D,
                                   d_t, d_h)
        else:
            ops.split_qk_norm(x2, dev_bf16(wtb), dev_bf16(whb), H, D)
            ops.split_rope(x2, cs, sn, H, D, d_t, d_h)
        torch.cuda.synchronize()
        got = host_f32(x2)
        assert rel_l2(got, ref) < BAR
        assert max_rel(got, ref) <= MAX_REL
