"""u15h_mot_linear_noalloc (the entry point that allocates nothing) against
u15h_mot_linear, through the C ABI: bit-identical outputs on two calls in
a row, the second with a smaller input, both with split-K tails (so the
static scratch is really used), and the first call's outputs against the
oracle on sampled rows."""
import numpy as np
import pytest
import torch

import oracle
from helpers import host_bits, host_f32, max_rel, rel_l2

pytestmark = pytest.mark.gpu


def _case(g, Mu, Mg, K, Ns):
    M = Mu + Mg
    x = torch.randn(M, K, generator=g, device="cuda").to(torch.bfloat16)
    projs = []
    for N in Ns:
        wu = (torch.randn(N, K, generator=g, device="cuda") * 0.02).to(torch.bfloat16)
        wg = (torch.randn(N, K, generator=g, device="cuda") * 0.02).to(torch.bfloat16)
        projs.append((wu, wg, N))
    return x, projs


def _run(ops, x, Mu, Mg, K, projs, noalloc):
    ys = [torch.full((Mu + Mg, N), float("nan"), dtype=torch.bfloat16, device="cuda")
          for _, _, N in projs]
    ops.mot_linear(x, Mu, Mg, K,
                   [dict(w_und=wu, w_gen=wg, y=y) for (wu, wg, _), y in zip(projs, ys)],
                   noalloc=noalloc)
    return ys


def test_noalloc_matches_mot_linear_twice(ops):
    g = torch.Generator(device="cuda").manual_seed(777)
    # call 1: config 2's o projection (272 tiles on 256 CUs: a 16-tile
    # split-K tail); call 2, smaller: 300 rows at K = 12288 (6 tiles, each
    # split into 24 K shares)
    cases = [(128, 4096, 4096, [4096]), (37, 263, 12288, [264])]
    for i, (Mu, Mg, K, Ns) in enumerate(cases):
        x, projs = _case(g, Mu, Mg, K, Ns)
        y_na = _run(ops, x, Mu, Mg, K, projs, True)
        y_ref = _run(ops, x, Mu, Mg, K, projs, False)
        torch.cuda.synchronize()
        for a, b in zip(y_na, y_ref):
            assert torch.equal(a.view(torch.int16), b.view(torch.int16)), i
        if i == 0:
            rows = np.array([0, 127, 128, 3000, Mu + Mg - 1], np.int32)
            xb = host_bits(x)
            (wu, wg, _), = projs
            got = host_f32(y_na[0])[rows]
            exp = np.empty_like(got)
            exp[rows < Mu] = oracle.linear_bf16(xb, host_bits(wu), row_ids=rows[rows < Mu])
            exp[rows >= Mu] = oracle.linear_bf16(xb, host_bits(wg), row_ids=rows[rows >= Mu])
            assert max_rel(got, exp) <= 1e-2 and rel_l2(got, exp) < 4e-3


def test_noalloc_skinny_route_allocates_nothing_on_a_fresh_context():
    """The skinny route's K shares (every group at most 128 rows), through
    the static scratch: on a context that has never allocated its split-K
    workspace, two calls in a row (the second smaller) are bit-identical
    to u15h_mot_linear and leave the device's free memory unchanged, while
    u15h_mot_linear on the same context then allocates its workspace."""
    import u15h
    g = torch.Generator(device="cuda").manual_seed(778)
    # (Mu, Mg, K, Ns): 64 + 64 rows at K = 12288 split into 4 K shares;
    # then 16 + 48 rows at K = 4096, also 4 shares
    cases = [(64, 64, 12288, [4096]), (16, 48, 4096, [1024, 512])]
    fresh = u15h.Ops(0)
    try:
        data, refs = [], []
        for Mu, Mg, K, Ns in cases:
            x, projs = _case(g, Mu, Mg, K, Ns)
            ys, rs = ([torch.full((Mu + Mg, N), float("nan"), dtype=torch.bfloat16,
                                  device="cuda") for N in Ns] for _ in range(2))
            data.append((Mu, Mg, K, x, projs, ys))
            refs.append(rs)
        args = lambda Mu, Mg, K, x, projs, ys: (
            x, Mu, Mg, K,
            [dict(w_und=wu, w_gen=wg, y=y) for (wu, wg, _), y in zip(projs, ys)])
        # one call first, so that anything the HIP runtime sets up lazily
        # on a first launch in this process is in place before measuring
        fresh.mot_linear(*args(*data[0]), noalloc=True)
        torch.cuda.synchronize()
        free0, _ = torch.cuda.mem_get_info()
        for d in data:
            fresh.mot_linear(*args(*d), noalloc=True)
        torch.cuda.synchronize()
        free1, _ = torch.cuda.mem_get_info()
        assert free1 == free0, (free0, free1)
        for i, ((Mu, Mg, K, x, projs, ys), rs) in enumerate(zip(data, refs)):
            fresh.mot_linear(*args(Mu, Mg, K, x, projs, rs), noalloc=False)
            torch.cuda.synchronize()
            for a, b in zip(ys, rs):
                assert torch.equal(a.view(torch.int16), b.view(torch.int16)), i
        # the allocating entry point did allocate its workspace (num_cu x
        # 256 KiB: 64 MiB on 256 CUs), which shows the measurement sees
        # an allocation; every tensor was allocated before free0
        free2, _ = torch.cuda.mem_get_info()
        assert free0 - free2 >= 32 << 20, (free0, free2)
        # the first case's outputs against the oracle on sampled rows
        Mu, Mg, K, x, projs, ys = data[0]
        rows = np.array([0, 31, 63, 64, 100, 127], np.int32)
        xb = host_bits(x)
        (wu, wg, _), = projs
        got = host_f32(ys[0])[rows]
        exp = np.empty_like(got)
        exp[rows < Mu] = oracle.linear_bf16(xb, host_bits(wu), row_ids=rows[rows < Mu])
        exp[rows >= Mu] = oracle.linear_bf16(xb, host_bits(wg), row_ids=rows[rows >= Mu])
        assert max_rel(got, exp) <= 1e-2 and rel_l2(got, exp) < 4e-3
    finally:
        torch.cuda.synchronize()
        fresh.close()
