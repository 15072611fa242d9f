"""Full-output parity at the BASELINE sizes, and the whole resident stack.

  * Every element of every output of config 2's and config 4's four
    grouped launches, bit-exact.  The operands are drawn so that the exact
    product is representable at every step of any fp32 summation: x holds
    integers in [-3, 3] and w integers in [-7, 7] times 2^-8, so each
    partial sum is a multiple of 2^-8 below 2^10 in magnitude (K <= 12288)
    and no fp32 addition rounds, in any order, in the MFMAs, across split-K
    shares or in the reductions.  The only rounding left is the epilogue's
    bf16 RNE, so each output must equal RNE(exact sum) bit for bit; a wrong
    tile anywhere (stale, zero, the other expert's weights, a shifted K
    range) fails.  The exact sums come from an integer GEMM on the host
    (float32 matmul of integer-valued arrays is exact under the same
    bound), itself cross-checked against the oracle's int32 GEMM on a
    slice.  The kernels, tiles, split tails and epilogues are the ones the
    random-data runs take: nothing in the GEMM branches on values.
  * The config-5 stack: all 42 layers x 2 weight sets bound by name and
    resident (32.4 GB bf16 + 16.2 GB int8), each layer run through
    u15h_stack_layer, each layer's seven outputs checked on sampled rows
    and sampled output columns before the next layer overwrites them: bf16
    against the oracle (max-rel <= 1e-2, rel-L2 < 4e-3), the int8 tier
    bit-exact against the oracle's quantise -> int32 GEMM -> dequant.
    Reference: forward_many's layer loop, src/u15-backbone.cc:386-426.
"""
import numpy as np
import pytest
import torch

import oracle
import u15h
from helpers import host_bits, max_rel, rel_l2

pytestmark = pytest.mark.gpu

H, I, NQ, NKV = 4096, 12288, 4096, 1024
# (input width K, [output widths]) of the four grouped launches of a layer
LAUNCHES = {"qkv": (H, [NQ, NKV, NKV]), "o": (NQ, [H]),
            "gate_up": (H, [I, I]), "down": (I, [H])}
CONFIGS = {"c2": (128, 4096), "c4": (4352, 12288)}


def _ints(g, shape, lo, hi):
    return torch.randint(lo, hi + 1, shape, generator=g, device="cuda",
                         dtype=torch.int32)


def _rne_bits(y):
    """bf16 RNE bit patterns of exact f32 values (the oracle's rule)."""
    return oracle.f32_to_bf16(y)


@pytest.mark.parametrize("launch", list(LAUNCHES))
@pytest.mark.parametrize("cfg", list(CONFIGS))
def test_every_output_bit_exact_on_exact_data(ops, cfg, launch):
    Mu, Mg = CONFIGS[cfg]
    K, Ns = LAUNCHES[launch]
    M = Mu + Mg
    seed = 1000 * list(CONFIGS).index(cfg) + list(LAUNCHES).index(launch)
    g = torch.Generator(device="cuda").manual_seed(seed)
    xi = _ints(g, (M, K), -3, 3)
    x = xi.to(torch.bfloat16)
    projs, wints = [], []
    for N in Ns:
        ku = _ints(g, (N, K), -7, 7)
        kg = _ints(g, (N, K), -7, 7)
        wints.append((ku, kg))
        projs.append(dict(w_und=(ku.float() / 256).to(torch.bfloat16),
                          w_gen=(kg.float() / 256).to(torch.bfloat16),
                          y=torch.full((M, N), float("nan"), dtype=torch.bfloat16,
                                       device="cuda")))
    ops.mot_linear(x, Mu, Mg, K, projs)
    torch.cuda.synchronize()
    xh = xi.cpu().numpy().astype(np.float32)
    for (ku, kg), p in zip(wints, projs):
        got = host_bits(p["y"])
        for k_, rows in ((ku, slice(0, Mu)), (kg, slice(Mu, M))):
            if rows.start == rows.stop:
                continue
            kh = k_.cpu().numpy()
            # exact: integer-valued operands, every partial sum < 2^24
            exact = xh[rows] @ kh.astype(np.float32).T
            # pin the host product against the oracle's exact int32 GEMM
            acc = oracle.gemm_i8_i32(xh[rows][:5].astype(np.int8),
                                     kh[:: max(1, kh.shape[0] // 37)].astype(np.int8))
            assert np.array_equal(acc, exact[:5, :: max(1, kh.shape[0] // 37)].astype(np.int32))
            want = _rne_bits(exact * np.float32(1.0 / 256))
            bad = np.argwhere(got[rows] != want)
            assert bad.size == 0, (cfg, launch, rows, bad[:5].tolist(), bad.shape[0])


# ---- the whole config-5 stack ------------------------------------------------

def _sample_cols(N, rng):
    """64 output columns of an N-wide projection: the first and last, both
    sides of the first 256-column tile boundary, the middle, and random
    ones."""
    c = {0, N - 1, 255, 256, N // 2}
    c |= set(rng.choice(N, 59, replace=False).tolist())
    return np.array(sorted(c), np.int64)[:64]


def test_stack_42_layers_resident_both_tiers(ops):
    """All 42 layers x 2 weight sets resident; every layer's seven outputs
    checked at 128 + 4096 rows in both tiers."""
    L, Mu, Mg = 42, 128, 4096
    M = Mu + Mg
    g = torch.Generator(device="cuda").manual_seed(4242)
    st = u15h.Stack(L)
    W = {}
    for layer in range(L):
        for e in (u15h.UND, u15h.GEN):
            for p in range(7):
                N, K = st.shape(p)
                w = (torch.randn(N, K, generator=g, device="cuda") * 0.02).to(torch.bfloat16)
                wq = torch.empty(N, K, dtype=torch.int8, device="cuda")
                sw = torch.empty(N, dtype=torch.float32, device="cuda")
                ops.quant_rows_i8(w, wq, sw)
                name = u15h.slot_name(layer, e, p)
                st.bind(name, w)
                st.bind_i8(name, wq, sw)
                W[(layer, e, p)] = (w, wq, sw)
    assert st.check() is None and st.check(tier=u15h.TIER_I8) is None

    def act(K):
        return torch.randn(M, K, generator=g, device="cuda").to(torch.bfloat16)

    t = dict(x=act(H), attn=act(NQ), x2=act(H), h=act(I),
             xq=torch.empty(M, I, dtype=torch.int8, device="cuda"),
             sx=torch.empty(M, dtype=torch.float32, device="cuda"))
    for name, n in (("q", NQ), ("k", NKV), ("v", NKV), ("o", H),
                    ("gate", I), ("up", I), ("down", H)):
        t[name] = torch.empty(M, n, dtype=torch.bfloat16, device="cuda")
    io = u15h.layer_io(**t)
    outs = (("q", "x", 0), ("k", "x", 1), ("v", "x", 2), ("o", "attn", 3),
            ("gate", "x2", 4), ("up", "x2", 5), ("down", "h", 6))
    rows = np.array([0, 77, 127, 128, 1500, 3333, M - 1], np.int32)
    rows_dev = torch.from_numpy(rows.astype(np.int64)).cuda()
    rng = np.random.default_rng(42)
    xin = {n: host_bits(t[n]) for n in ("x", "attn", "x2", "h")}
    qin = {n: oracle.quant_rows_i8(xin[n][rows]) for n in xin}
    for tier in (u15h.TIER_BF16, u15h.TIER_I8):
        for layer in range(L):
            for name, _, _ in outs:
                t[name].fill_(float("nan"))
            ops.stack_layer(st, layer, io, Mu, Mg, tier=tier)
            torch.cuda.synchronize()
            for name, inp, p in outs:
                N = t[name].shape[1]
                cols = _sample_cols(N, rng)
                got = host_bits(t[name][rows_dev])[:, cols]
                for e, sel in ((u15h.UND, rows < Mu), (u15h.GEN, rows >= Mu)):
                    w, wq, sw = W[(layer, e, p)]
                    if tier == u15h.TIER_BF16:
                        wb = host_bits(w[torch.from_numpy(cols).cuda()])
                        exp = oracle.linear_bf16(xin[inp], wb, row_ids=rows[sel])
                        gf = oracle.bf16_to_f32(got[sel])
                        assert max_rel(gf, exp) <= 1e-2, (layer, name, e)
                        assert rel_l2(gf, exp) < 4e-3, (layer, name, e)
                    else:
                        ci = torch.from_numpy(cols).cuda()
                        wq_h = wq[ci].cpu().numpy()
                        sw_h = sw[ci].cpu().numpy()
                        # the device's weight codes are the oracle's
                        qo, so = oracle.quant_rows_i8(host_bits(w[ci]))
                        assert np.array_equal(wq_h, qo) and np.array_equal(sw_h, so)
                        xq, sx = qin[inp]
                        acc = oracle.gemm_i8_i32(xq[sel], wq_h)
                        exp = oracle.dequant_bf16(acc, sx[sel], sw_h)
                        assert np.array_equal(got[sel], exp), (layer, name, e)
    st.close()
