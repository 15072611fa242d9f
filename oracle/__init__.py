"""CPU oracle for the MoT projection GEMMs -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package.  It is the checker, never the thing measured or
shipped: the product library (libu15h.so) neither links nor calls it.

numpy wrappers over liboracle.so (u15_oracle.c, u15_refrand.cc) and, when
built, over _ref/libu15ref.so -- the reference's own CPU path compiled
from /root/reference/src/u15-ref.cc where it lies.
"""
from __future__ import annotations

import ctypes
import pathlib
import subprocess

import numpy as np

ORACLE_DIR = pathlib.Path(__file__).resolve().parent
LIB_PATH = ORACLE_DIR / "liboracle.so"
REF_LIB_PATH = ORACLE_DIR / "_ref" / "libu15ref.so"

_lib = None
_ref = None


def build(quiet: bool = True) -> None:
    """Compile liboracle.so (and _ref/ when the reference is present)."""
    out = subprocess.run(["make", "-C", str(ORACLE_DIR), "-B", "all"],
                         capture_output=True, text=True)
    if out.returncode != 0:
        raise RuntimeError("oracle build failed:\n" + out.stdout + out.stderr)
    if not quiet:
        print(out.stdout)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        vp, sz = ctypes.c_void_p, ctypes.c_size_t
        L.u15o_f32_to_bf16.restype = ctypes.c_uint16
        L.u15o_f32_to_bf16.argtypes = [ctypes.c_float]
        L.u15o_bf16_to_f32.restype = ctypes.c_float
        L.u15o_bf16_to_f32.argtypes = [ctypes.c_uint16]
        for n, a in {
            "u15o_f32_to_bf16_n": [vp, sz, vp],
            "u15o_bf16_to_f32_n": [vp, sz, vp],
            "u15o_linear": [vp, vp, vp, sz, sz, sz, vp],
            "u15o_linear_bf16": [vp, vp, vp, vp, sz, sz, sz, vp],
            "u15o_mot_linear_bf16": [vp, vp, vp, sz, sz, sz, sz, vp],
            "u15o_silu": [vp, sz],
            "u15o_swiglu_bf16": [vp, vp, sz, vp],
            "u15o_quant_rows_i8": [vp, sz, sz, vp, vp],
            "u15o_i8_product_sums": [vp, vp, sz, sz, sz, vp, vp],
            "u15o_dequant_bf16": [vp, vp, vp, sz, sz, vp],
            "u15o_dequant_f64": [vp, vp, vp, sz, sz, vp],
            "u15o_randn_mt": [ctypes.c_uint32, ctypes.c_float, sz, vp],
            "u15o_dequant_affine": [vp, vp, vp, ctypes.c_int, ctypes.c_int, sz, sz, vp],
            "u15o_pack_affine": [vp, ctypes.c_int, ctypes.c_int, sz, sz, vp, vp, vp, vp],
            "u15o_bias_add_bf16": [vp, vp, sz, sz],
            "u15o_rms_norm": [vp, vp, ctypes.c_float, sz, sz, vp],
            "u15o_f16_to_bf16_n": [vp, sz, vp],
            "u15o_attention": [vp, vp, vp, ctypes.c_int, vp, sz, sz, sz, sz,
                               sz, sz, sz, vp],
            "u15o_rope_inv_freq": [ctypes.c_int, ctypes.c_double, vp],
            "u15o_rope_half": [vp, vp, ctypes.c_int, ctypes.c_double],
            "u15o_rope_tables": [vp, vp, vp, sz, ctypes.c_int, ctypes.c_int,
                                 ctypes.c_int, ctypes.c_double, ctypes.c_double,
                                 vp, vp],
            "u15o_split_qk_norm_rope": [vp, vp, vp, vp, vp, vp, sz, sz,
                                        ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                        ctypes.c_double, ctypes.c_double,
                                        ctypes.c_float, ctypes.c_int,
                                        ctypes.c_int],
        }.items():
            getattr(L, n).restype = None
            getattr(L, n).argtypes = a
        L.u15o_gemm_i8_i32.restype = ctypes.c_int
        L.u15o_gemm_i8_i32.argtypes = [vp, vp, vp, sz, sz, sz, vp]
        for n in ("u15o_rel_l2", "u15o_max_rel"):
            getattr(L, n).restype = ctypes.c_double
            getattr(L, n).argtypes = [vp, vp, sz]
        _lib = L
    return _lib


def ref_lib():
    """The reference's own u15::ref functions, or None if not built."""
    global _ref
    if _ref is None and REF_LIB_PATH.exists():
        R = ctypes.CDLL(str(REF_LIB_PATH))
        vp, sz = ctypes.c_void_p, ctypes.c_size_t
        R.u15ref_linear.restype = None
        R.u15ref_linear.argtypes = [vp, vp, vp, sz, sz, sz, vp]
        R.u15ref_silu.restype = None
        R.u15ref_silu.argtypes = [vp, sz]
        for n, a in {
            "u15ref_rms_norm": [vp, vp, ctypes.c_float, sz, sz, vp],
            "u15ref_attention": [vp, vp, vp, vp, sz, sz, sz, sz, sz, vp],
            "u15ref_block_causal_mask": [vp, sz, vp],
            "u15ref_rope_inv_freq": [ctypes.c_int, ctypes.c_double, vp],
            "u15ref_rope_half": [vp, vp, ctypes.c_int, ctypes.c_double],
            "u15ref_split_rope_project": [vp, vp, vp, vp, vp, vp, vp, sz, sz,
                                          ctypes.c_int, ctypes.c_int,
                                          ctypes.c_double, ctypes.c_double,
                                          ctypes.c_double, vp],
            "u15ref_decoder_layer": [vp, ctypes.POINTER(vp), sz, sz, sz, sz, sz,
                                     ctypes.c_double, ctypes.c_double,
                                     ctypes.c_double, vp, vp, vp, vp, sz, vp],
        }.items():
            getattr(R, n).restype = None
            getattr(R, n).argtypes = a
        _ref = R
    return _ref


def _c(a, dtype):
    a = np.ascontiguousarray(a, dtype=dtype)
    return a, a.ctypes.data


# ---- conversions -----------------------------------------------------
def f32_to_bf16(x) -> np.ndarray:
    """RNE f32 -> bf16 bit patterns (uint16)."""
    x, p = _c(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().u15o_f32_to_bf16_n(p, x.size, out.ctypes.data)
    return out


def f16_to_bf16(h) -> np.ndarray:
    """f16 bit patterns (uint16) -> bf16 bit patterns, the loader's rule."""
    h, p = _c(h, np.uint16)
    out = np.empty(h.shape, np.uint16)
    lib().u15o_f16_to_bf16_n(p, h.size, out.ctypes.data)
    return out


def bf16_to_f32(h) -> np.ndarray:
    h, p = _c(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().u15o_bf16_to_f32_n(p, h.size, out.ctypes.data)
    return out


# ---- GEMMs ---------------------------------------------------------------
def linear(x, w, b=None) -> np.ndarray:
    """ref::linear restated: f32 operands, double accumulation."""
    x, px = _c(x, np.float32)
    w, pw = _c(w, np.float32)
    rows, K = x.shape
    N = w.shape[0]
    pb = None
    if b is not None:
        b, pb = _c(b, np.float32)
    y = np.empty((rows, N), np.float32)
    lib().u15o_linear(px, pw, pb, rows, K, N, y.ctypes.data)
    return y


def linear_bf16(x_bits, w_bits, b_bits=None, row_ids=None) -> np.ndarray:
    """linear on bf16 bit patterns; optional subset of rows (f32 out)."""
    x, px = _c(x_bits, np.uint16)
    w, pw = _c(w_bits, np.uint16)
    K = x.shape[1]
    N = w.shape[0]
    pb = None
    if b_bits is not None:
        b_bits, pb = _c(b_bits, np.uint16)
    pr = None
    rows = x.shape[0]
    if row_ids is not None:
        row_ids, pr = _c(row_ids, np.int32)
        rows = row_ids.size
    y = np.empty((rows, N), np.float32)
    lib().u15o_linear_bf16(px, pw, pb, pr, rows, K, N, y.ctypes.data)
    return y


def mot_linear_bf16(x_bits, w_und, w_gen, M_und, M_gen) -> np.ndarray:
    x, px = _c(x_bits, np.uint16)
    wu, pu = _c(w_und, np.uint16)
    wg, pg = _c(w_gen, np.uint16)
    K = x.shape[1]
    N = wu.shape[0]
    y = np.empty((M_und + M_gen, N), np.float32)
    lib().u15o_mot_linear_bf16(px, pu, pg, M_und, M_gen, K, N, y.ctypes.data)
    return y


def silu(x) -> np.ndarray:
    x = np.array(x, dtype=np.float32, copy=True)
    lib().u15o_silu(x.ctypes.data, x.size)
    return x


def swiglu_bf16(g_bits, u_bits) -> np.ndarray:
    g, pg = _c(g_bits, np.uint16)
    u, pu = _c(u_bits, np.uint16)
    out = np.empty(g.shape, np.float32)
    lib().u15o_swiglu_bf16(pg, pu, g.size, out.ctypes.data)
    return out


# ---- int8 ------------------------------------------------------------------
def quant_rows_i8(x_bits):
    x, px = _c(x_bits, np.uint16)
    rows, K = x.shape
    q = np.empty((rows, K), np.int8)
    s = np.empty(rows, np.float32)
    lib().u15o_quant_rows_i8(px, rows, K, q.ctypes.data, s.ctypes.data)
    return q, s


def gemm_i8_i32(a, w, row_ids=None) -> np.ndarray:
    a, pa = _c(a, np.int8)
    w, pw = _c(w, np.int8)
    K = a.shape[1]
    N = w.shape[0]
    pr = None
    rows = a.shape[0]
    if row_ids is not None:
        row_ids, pr = _c(row_ids, np.int32)
        rows = row_ids.size
    acc = np.empty((rows, N), np.int32)
    if lib().u15o_gemm_i8_i32(pa, pw, pr, rows, K, N, acc.ctypes.data) != 0:
        raise OverflowError("int8 product does not fit in int32")
    return acc


def i8_product_sums(a, w):
    a, pa = _c(a, np.int8)
    w, pw = _c(w, np.int8)
    rows, K = a.shape
    N = w.shape[0]
    rs = np.empty(rows, np.int64)
    cs = np.empty(N, np.int64)
    lib().u15o_i8_product_sums(pa, pw, rows, K, N, rs.ctypes.data,
                               cs.ctypes.data)
    return rs, cs


def dequant_bf16(acc, sa, sw) -> np.ndarray:
    acc, pa = _c(acc, np.int32)
    sa, ps = _c(sa, np.float32)
    sw, pw = _c(sw, np.float32)
    rows, N = acc.shape
    y = np.empty((rows, N), np.uint16)
    lib().u15o_dequant_bf16(pa, ps, pw, rows, N, y.ctypes.data)
    return y


def dequant_f64(acc, sa, sw) -> np.ndarray:
    acc, pa = _c(acc, np.int32)
    sa, ps = _c(sa, np.float32)
    sw, pw = _c(sw, np.float32)
    rows, N = acc.shape
    y = np.empty((rows, N), np.float64)
    lib().u15o_dequant_f64(pa, ps, pw, rows, N, y.ctypes.data)
    return y


# ---- affine-quantized packs --------------------------------------------------
def pack_affine(w, bits, group):
    """(codes u32 [N][K*bits/32], scales bf16, biases bf16, deq f32)."""
    w, pw = _c(w, np.float32)
    N, K = w.shape
    codes = np.empty((N, K * bits // 32), np.uint32)
    scales = np.empty((N, K // group), np.uint16)
    biases = np.empty((N, K // group), np.uint16)
    deq = np.empty((N, K), np.float32)
    lib().u15o_pack_affine(pw, bits, group, N, K, codes.ctypes.data,
                           scales.ctypes.data, biases.ctypes.data,
                           deq.ctypes.data)
    return codes, scales, biases, deq


def dequant_affine(codes, scales, biases, bits, group, K):
    codes, pc = _c(codes, np.uint32)
    scales, ps = _c(scales, np.uint16)
    biases, pb = _c(biases, np.uint16)
    N = codes.shape[0]
    out = np.empty((N, K), np.uint16)
    lib().u15o_dequant_affine(pc, ps, pb, bits, group, N, K, out.ctypes.data)
    return out


def bias_add_bf16(y_bits, b_bits):
    y = np.array(y_bits, dtype=np.uint16, copy=True)
    b, pb = _c(b_bits, np.uint16)
    lib().u15o_bias_add_bf16(y.ctypes.data, pb, y.shape[0], y.shape[1])
    return y


# ---- split q/k norm + three-way RoPE ---------------------------------------------
def rms_norm(x, w, eps=1e-6):
    x, px = _c(x, np.float32)
    w, pw = _c(w, np.float32)
    rows, dim = x.shape
    out = np.empty_like(x)
    lib().u15o_rms_norm(px, pw, eps, rows, dim, out.ctypes.data)
    return out


def rope_inv_freq(dim, theta):
    out = np.empty(dim // 2, np.float32)
    lib().u15o_rope_inv_freq(dim, theta, out.ctypes.data)
    return out


def rope_half(x, inv, dim, pos):
    x = np.array(x, dtype=np.float32, copy=True)
    inv, pi = _c(inv, np.float32)
    lib().u15o_rope_half(x.ctypes.data, pi, dim, float(pos))
    return x


def rope_tables(pos_t, pos_h, pos_w, D, d_t, d_h, theta_t=5e6, theta_hw=1e4):
    pt, a = _c(pos_t, np.int32)
    ph, b = _c(pos_h, np.int32)
    pw, c = _c(pos_w, np.int32)
    T = pt.size
    cs = np.empty((T, D), np.float32)
    sn = np.empty((T, D), np.float32)
    lib().u15o_rope_tables(a, b, c, T, D, d_t, d_h, theta_t, theta_hw,
                           cs.ctypes.data, sn.ctypes.data)
    return cs, sn


def split_qk_norm_rope(x, w_t, w_hw, pos_t, pos_h, pos_w, H, D, d_t, d_h,
                       theta_t=5e6, theta_hw=1e4, eps=1e-6, norm=True,
                       rope=True):
    """x [T][H*D] f32 (returned as a new array)."""
    x = np.array(x, dtype=np.float32, copy=True)
    T = x.shape[0]
    wt, pwt = _c(w_t, np.float32)
    wh, pwh = _c(w_hw, np.float32)
    pt, a = _c(pos_t, np.int32)
    ph, b = _c(pos_h, np.int32)
    pw, c = _c(pos_w, np.int32)
    lib().u15o_split_qk_norm_rope(x.ctypes.data, pwt, pwh, a, b, c, T, H, D,
                                  d_t, d_h, theta_t, theta_hw, eps,
                                  int(norm), int(rope))
    return x


def ref_rms_norm(x, w, eps=1e-6):
    R = ref_lib()
    if R is None:
        return None
    x, px = _c(x, np.float32)
    w, pw = _c(w, np.float32)
    rows, dim = x.shape
    out = np.empty_like(x)
    R.u15ref_rms_norm(px, pw, eps, rows, dim, out.ctypes.data)
    return out


def ref_rope_inv_freq(dim, theta):
    R = ref_lib()
    if R is None:
        return None
    out = np.empty(dim // 2, np.float32)
    R.u15ref_rope_inv_freq(dim, theta, out.ctypes.data)
    return out


def ref_rope_half(x, inv, dim, pos):
    R = ref_lib()
    if R is None:
        return None
    x = np.array(x, dtype=np.float32, copy=True)
    inv, pi = _c(inv, np.float32)
    R.u15ref_rope_half(x.ctypes.data, pi, dim, float(pos))
    return x


def ref_split_rope_project(x, w_proj, w_norm, w_norm_hw, pos_t, pos_h, pos_w,
                           heads, head_dim, theta_t=5e6, theta_hw=1e4,
                           eps=1e-6):
    """The reference's projection + split norm + split RoPE; head-major
    [heads][tokens][head_dim] out."""
    R = ref_lib()
    if R is None:
        return None
    x, px = _c(x, np.float32)
    w_proj, pwp = _c(w_proj, np.float32)
    w_norm, pwn = _c(w_norm, np.float32)
    w_norm_hw, pwh = _c(w_norm_hw, np.float32)
    pt, a = _c(pos_t, np.int32)
    ph, b = _c(pos_h, np.int32)
    pw, c = _c(pos_w, np.int32)
    T, hidden = x.shape
    out = np.empty((heads, T, head_dim), np.float32)
    R.u15ref_split_rope_project(px, pwp, pwn, pwh, a, b, c, T, hidden, heads,
                                head_dim, theta_t, theta_hw, eps,
                                out.ctypes.data)
    return out


# ---- attention -------------------------------------------------------------------
MODES = {"bidirectional": 0, "causal": 1, "block_causal": 2}


def attention(q, k, v, hkv, tk, mode="bidirectional", t_index=None,
              q_offset=0):
    """q [hq][tq][d]; k, v caches [hkv][cap][d] (keys [0, tk) used);
    head-major f32 out [hq][tq][d]."""
    q, pq = _c(q, np.float32)
    k, pk = _c(k, np.float32)
    v, pv = _c(v, np.float32)
    hq, tq, d = q.shape
    cap = k.shape[1]
    pt = None
    if t_index is not None:
        t_index, pt = _c(t_index, np.int32)
    out = np.empty((hq, tq, d), np.float32)
    lib().u15o_attention(pq, pk, pv, MODES[mode], pt, hq, hkv, tq, tk, d, cap,
                         q_offset, out.ctypes.data)
    return out


def ref_attention(q, k, v, mask, hkv):
    """u15::ref::attention on packed k, v [hkv][tk][d]: TOKEN-major out
    [tq][hq*d] (the reference's own layout)."""
    R = ref_lib()
    if R is None:
        return None
    q, pq = _c(q, np.float32)
    k, pk = _c(k, np.float32)
    v, pv = _c(v, np.float32)
    hq, tq, d = q.shape
    tk = k.shape[1]
    pm = None
    if mask is not None:
        mask, pm = _c(mask, np.float32)
    out = np.empty((tq, hq * d), np.float32)
    R.u15ref_attention(pq, pk, pv, pm, hq, hkv, tq, tk, d, out.ctypes.data)
    return out


LAYER_WEIGHT_NAMES = ("input_layernorm", "post_attention_layernorm", "q_proj",
                      "k_proj", "v_proj", "o_proj", "q_norm", "k_norm",
                      "q_norm_hw", "k_norm_hw", "gate_proj", "up_proj", "down_proj")


def ref_decoder_layer(x, w, heads, kv_heads, head_dim, pos_t, pos_h, pos_w,
                      mask=None, eps=1e-6, theta_t=5000000.0, theta_hw=10000.0):
    """u15::ref::decoder_layer (src/u15-ref.cc:242-311): one expert's whole
    layer in f32, x [tokens][hidden] -> [tokens][hidden].  `w` maps
    LAYER_WEIGHT_NAMES to f32 arrays ([out][in] for the projections);
    `mask` [tokens][tokens] additive, or None (bidirectional)."""
    R = ref_lib()
    if R is None:
        return None
    x, px = _c(x, np.float32)
    tokens, hidden = x.shape
    arrs = [np.ascontiguousarray(w[n], np.float32) for n in LAYER_WEIGHT_NAMES]
    ptrs = (ctypes.c_void_p * 13)(*[a.ctypes.data for a in arrs])
    inter = arrs[10].shape[0]
    t, pt = _c(pos_t, np.int32)
    h, ph = _c(pos_h, np.int32)
    ww, pw = _c(pos_w, np.int32)
    pm = None
    if mask is not None:
        mask, pm = _c(mask, np.float32)
    out = np.empty((tokens, hidden), np.float32)
    R.u15ref_decoder_layer(px, ptrs, hidden, heads, kv_heads, head_dim, inter, eps,
                           theta_t, theta_hw, pt, ph, pw, pm, tokens,
                           out.ctypes.data)
    return out


def ref_block_causal_mask(t_index):
    R = ref_lib()
    if R is None:
        return None
    t, pt = _c(t_index, np.int32)
    out = np.empty((t.size, t.size), np.float32)
    R.u15ref_block_causal_mask(pt, t.size, out.ctypes.data)
    return out


# ---- metrics / generator ------------------------------------------------------
def rel_l2(a, b) -> float:
    a, pa = _c(a, np.float32)
    b, pb = _c(b, np.float32)
    return float(lib().u15o_rel_l2(pa, pb, a.size))


def max_rel(a, b) -> float:
    a, pa = _c(a, np.float32)
    b, pb = _c(b, np.float32)
    return float(lib().u15o_max_rel(pa, pb, a.size))


def randn_mt(seed: int, n: int, stddev: float = 1.0) -> np.ndarray:
    """The reference tests' generator (std::mt19937 + normal_distribution)."""
    out = np.empty(n, np.float32)
    lib().u15o_randn_mt(seed, stddev, n, out.ctypes.data)
    return out


# ---- the reference's own CPU path (oracle/_ref) ------------------------------
def ref_linear(x, w, b=None):
    R = ref_lib()
    if R is None:
        return None
    x, px = _c(x, np.float32)
    w, pw = _c(w, np.float32)
    rows, K = x.shape
    N = w.shape[0]
    pb = None
    if b is not None:
        b, pb = _c(b, np.float32)
    y = np.empty((rows, N), np.float32)
    R.u15ref_linear(px, pw, pb, rows, K, N, y.ctypes.data)
    return y


def ref_silu(x):
    R = ref_lib()
    if R is None:
        return None
    x = np.array(x, dtype=np.float32, copy=True)
    R.u15ref_silu(x.ctypes.data, x.size)
    return x
