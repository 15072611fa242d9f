"""Writes the golden fixtures under tests/golden/ from the reference's own
CPU path.

Run in the container that has /root/reference:
    make -C oracle && python tests/golden/make_golden.py

Inputs are the reference tests' own: std::mt19937 + normal_distribution
(tests/u15-kernels-test.cc:110-118) with the seeds of test_linear
(M=9, K=64, N=48, seeds 31/32; tests/u15-kernels-test.cc:433-455).  The
expected outputs come from u15::ref::linear and u15::ref::silu compiled
from src/u15-ref.cc (oracle/_ref/libu15ref.so), not from this repository's
oracle.  Each fixture is an .npz of plain arrays (no pickles).
"""
import pathlib
import sys

import numpy as np
import torch

HERE = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))
import oracle  # noqa: E402


def bf16_round(a):
    # Inputs are rounded to bf16 by torch (an implementation independent of
    # the oracle under test), as the reference's upload path rounds them.
    t = torch.from_numpy(np.ascontiguousarray(a, np.float32))
    return t.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)


def widen(bits):
    return (bits.astype(np.uint32) << 16).view(np.float32)


def main():
    if oracle.ref_lib() is None:
        raise SystemExit("oracle/_ref/libu15ref.so is not built")

    # 1. test_linear's case, exactly as the reference test draws it.
    M, K, N = 9, 64, 48
    x = oracle.randn_mt(31, M * K).reshape(M, K)
    w = oracle.randn_mt(32, N * K).reshape(N, K)
    y_ref = oracle.ref_linear(x, w)
    xb, wb = bf16_round(x), bf16_round(w)
    y_ref_bf16in = oracle.ref_linear(widen(xb), widen(wb))
    b = oracle.randn_mt(33, N) * 0.5
    bb = bf16_round(b)
    y_ref_bias = oracle.ref_linear(widen(xb), widen(wb), widen(bb))
    np.savez(HERE / "linear_test_case.npz", x=x, w=w, y_ref=y_ref,
             x_bf16=xb, w_bf16=wb, y_ref_bf16in=y_ref_bf16in, bias_bf16=bb,
             y_ref_bias=y_ref_bias, seeds=np.array([31, 32, 33], np.int32))

    # 2. a two-group MoT case: und rows use w_und, gen rows use w_gen --
    #    the reference runs each group as its own linear (one expert per
    #    pass, src/u15-backbone.cc:189).
    Mu, Mg, K2, N2 = 5, 11, 64, 40
    x2 = bf16_round(oracle.randn_mt(41, (Mu + Mg) * K2).reshape(Mu + Mg, K2))
    wu = bf16_round(oracle.randn_mt(42, N2 * K2, 0.05).reshape(N2, K2))
    wg = bf16_round(oracle.randn_mt(43, N2 * K2, 0.05).reshape(N2, K2))
    yu = oracle.ref_linear(widen(x2[:Mu]), widen(wu))
    yg = oracle.ref_linear(widen(x2[Mu:]), widen(wg))
    np.savez(HERE / "mot_linear_case.npz", x=x2, w_und=wu, w_gen=wg,
             y_ref=np.concatenate([yu, yg]), m=np.array([Mu, Mg], np.int32))

    # 3. silu + the SwiGLU product, src/u15-ref.cc:51-58 and :303-304.
    g = oracle.randn_mt(51, 256) * 4.0
    u = oracle.randn_mt(52, 256)
    gb, ub = bf16_round(g), bf16_round(u)
    s = oracle.ref_silu(widen(gb))
    h = (s * widen(ub)).astype(np.float32)
    np.savez(HERE / "swiglu_case.npz", g_bf16=gb, u_bf16=ub, silu_ref=s,
             h_ref=h)
    print("wrote", sorted(p.name for p in HERE.glob("*.npz")))


if __name__ == "__main__":
    main()
