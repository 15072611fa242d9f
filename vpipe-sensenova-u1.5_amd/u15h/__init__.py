"""Python host binding of the u15h C ABI (include/u15h.h).

`Ops` mirrors the GEMM half of the reference's op vocabulary,
`u15::MetalOps` (src/u15-metal-ops.h:59-531): `linear`, the int8 tier's
`enable_i8_gemm` / `release_i8_scratch`, `swiglu`, plus the two-group MoT
entry points that run both weight sets (base for understanding rows,
`_mot_gen` for generated-image rows) in one launch.

Every call goes through libu15h.so, built in-tree next to this package
(`make -C vpipe-sensenova-u1.5_amd`).  There is no CPU fallback: if the
library is missing, or there is no gfx950 device, construction raises.

Tensors are torch tensors on the GPU; torch is used for device memory and
streams only.  Shapes and dtypes are checked here, before the C ABI checks
them again.
"""
from __future__ import annotations

import ctypes
import os
import pathlib
import re

import torch

PKG_DIR = pathlib.Path(__file__).resolve().parent.parent
REPO_DIR = PKG_DIR.parent
LIB_PATH = PKG_DIR / "libu15h.so"
HEADER_PATH = REPO_DIR / "include" / "u15h.h"

OK, EINVAL, ENODEV, ELAUNCH, ENOMEM = 0, 1, 2, 3, 4
MAX_PROJ = 4

_lib = None


class U15hError(RuntimeError):
    def __init__(self, status: int, msg: str):
        super().__init__(msg)
        self.status = status


class _MotProj(ctypes.Structure):
    _fields_ = [("w_und", ctypes.c_void_p), ("w_gen", ctypes.c_void_p),
                ("bias_und", ctypes.c_void_p), ("bias_gen", ctypes.c_void_p),
                ("y", ctypes.c_void_p), ("N", ctypes.c_int)]


class _MotProjI8(ctypes.Structure):
    _fields_ = [("wq_und", ctypes.c_void_p), ("sw_und", ctypes.c_void_p),
                ("wq_gen", ctypes.c_void_p), ("sw_gen", ctypes.c_void_p),
                ("y", ctypes.c_void_p), ("N", ctypes.c_int)]


class _LayerIO(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in
                ("x", "q", "k", "v", "attn", "o", "x2", "gate", "up", "h",
                 "down", "xq", "sx")]


class _QkNorm(ctypes.Structure):
    _fields_ = [("q_t", ctypes.c_void_p), ("q_hw", ctypes.c_void_p),
                ("k_t", ctypes.c_void_p), ("k_hw", ctypes.c_void_p)]


class _LayerFullIO(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in
                ("x", "normed", "q", "k", "v", "attn", "proj", "h", "up", "xq",
                 "sx", "k_cache", "v_cache")] + \
               [(n, ctypes.c_int) for n in ("cap", "kv_off", "kv_len", "mode")] + \
               [("t_index", ctypes.c_void_p), ("cos_tab", ctypes.c_void_p),
                ("sin_tab", ctypes.c_void_p), ("d_t", ctypes.c_int),
                ("d_h", ctypes.c_int), ("eps", ctypes.c_float)]


class _QWeight(ctypes.Structure):
    _fields_ = [("codes", ctypes.c_void_p), ("scales", ctypes.c_void_p),
                ("biases", ctypes.c_void_p), ("bits", ctypes.c_int),
                ("group", ctypes.c_int)]


def declared_symbols() -> list[str]:
    """Every function include/u15h.h declares."""
    text = HEADER_PATH.read_text()
    return sorted(set(re.findall(r"\b(u15h_[a-z0-9_]+)\s*\(", text)))


def load_library() -> ctypes.CDLL:
    """Load libu15h.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise U15hError(ENODEV, f"{LIB_PATH} is not built; run "
                        f"`make -C {PKG_DIR}` (or __graft_entry__.build())")
    lib = ctypes.CDLL(str(LIB_PATH))
    vp, i, i64 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64
    sigs = {
        "u15h_create": (i, [i, ctypes.POINTER(vp)]),
        "u15h_destroy": (None, [vp]),
        "u15h_abi_version": (i, []),
        "u15h_status_str": (ctypes.c_char_p, [i]),
        "u15h_last_error": (ctypes.c_char_p, [vp]),
        "u15h_linear": (i, [vp, vp, vp, vp, vp, vp, i, i, i]),
        "u15h_mot_linear": (i, [vp, vp, vp, i, i, i,
                                ctypes.POINTER(_MotProj), i]),
        "u15h_mot_linear_noalloc": (i, [vp, vp, vp, i, i, i,
                                        ctypes.POINTER(_MotProj), i]),
        "u15h_swiglu": (i, [vp, vp, vp, vp, vp, i64]),
        "u15h_mot_gate_up_swiglu": (i, [vp, vp, vp, i, i, i, vp, vp, vp, vp,
                                        vp, i]),
        "u15h_enable_i8_gemm": (i, [vp, i]),
        "u15h_release_i8_scratch": (None, [vp]),
        "u15h_i8_min_m": (i, [vp]),
        "u15h_profile_next_gemm": (i, [vp, vp]),
        "u15h_profile_bracket_next_gemm": (i, [vp, vp, vp]),
        "u15h_profile_next_kernels": (i, [vp, vp, vp, vp, vp, vp, vp]),
        "u15h_quant_rows_i8": (i, [vp, vp, vp, i, i, vp, vp]),
        "u15h_mot_gemm_i8_i32": (i, [vp, vp, vp, i, i, i,
                                     ctypes.POINTER(_MotProjI8), i]),
        "u15h_mot_gemm_i8": (i, [vp, vp, vp, vp, i, i, i,
                                 ctypes.POINTER(_MotProjI8), i]),
        "u15h_route_rows": (i, [vp, i, vp, ctypes.POINTER(i),
                                ctypes.POINTER(i)]),
        "u15h_dequant_affine": (i, [vp, vp, ctypes.POINTER(_QWeight), i, i,
                                    vp]),
        "u15h_linear_q": (i, [vp, vp, vp, ctypes.POINTER(_QWeight), vp, vp,
                              i, i, i]),
        "u15h_swiglu_fused": (i, [vp, vp, vp, vp, vp, i, i, i]),
        "u15h_bias_add": (i, [vp, vp, vp, vp, i, i]),
        "u15h_f32_to_bf16": (i, [vp, vp, vp, i64, vp]),
        "u15h_f16_to_bf16": (i, [vp, vp, vp, i64, vp]),
        "u15h_qweight_geometry": (i, [i, i64, i64, ctypes.POINTER(i),
                                      ctypes.POINTER(i)]),
        "u15h_repack_affine_i8": (i, [vp, vp, ctypes.POINTER(_QWeight), i, i,
                                      vp, vp]),
        "u15h_split_qk_norm": (i, [vp, vp, vp, vp, vp, i, i, i,
                                   ctypes.c_float]),
        "u15h_split_rope": (i, [vp, vp, vp, vp, vp, i, i, i, i, i]),
        "u15h_split_qk_norm_rope": (i, [vp, vp, vp, vp, vp, vp, vp, i, i, i,
                                        i, i, ctypes.c_float]),
        "u15h_mot_attention_prologue": (i, [vp, vp, vp, vp, vp,
                                            ctypes.POINTER(_QkNorm),
                                            ctypes.POINTER(_QkNorm), vp, vp,
                                            i, i, i, i, i, i, i,
                                            ctypes.c_float, vp, vp, i, i]),
        "u15h_rms_norm": (i, [vp, vp, vp, vp, vp, i, i, ctypes.c_float]),
        "u15h_rms_norm_quant_i8": (i, [vp, vp, vp, vp, i, i, ctypes.c_float,
                                       vp, vp, vp]),
        "u15h_add": (i, [vp, vp, vp, vp, i64]),
        "u15h_swiglu_quant_i8": (i, [vp, vp, vp, vp, i, i, vp, vp, vp]),
        "u15h_mot_rms_norm": (i, [vp, vp, vp, vp, i, i, i, vp, vp, ctypes.c_float,
                                  vp, vp, vp]),
        "u15h_build_rope_tables": (i, [vp, vp, vp, i, i, i, i,
                                       ctypes.c_double, ctypes.c_double, vp,
                                       vp]),
        "u15h_sdpa": (i, [vp, vp, vp, vp, vp, vp, i, i, i, i, i, i, i, i]),
        "u15h_sdpa_block_causal": (i, [vp, vp, vp, vp, vp, vp, vp, i, i, i, i,
                                       i, i, i]),
        "u15h_attention_token_major": (i, [vp, vp, vp, vp, vp, vp, vp, i, i,
                                           i, i, i, i, i, i]),
        "u15h_transpose_thd": (i, [vp, vp, vp, vp, i, i, i]),
        "u15h_transpose_htd": (i, [vp, vp, vp, vp, i, i, i]),
        "u15h_transpose_into_cache": (i, [vp, vp, vp, vp, i, i, i, i, i]),
        "u15h_stack_create": (i, [i, i, i, i, i, i, ctypes.POINTER(vp)]),
        "u15h_stack_destroy": (None, [vp]),
        "u15h_weight_slot": (i, [ctypes.c_char_p, ctypes.POINTER(i),
                                 ctypes.POINTER(i), ctypes.POINTER(i)]),
        "u15h_stack_bind": (i, [vp, ctypes.c_char_p, vp]),
        "u15h_stack_bind_i8": (i, [vp, ctypes.c_char_p, vp, vp]),
        "u15h_stack_set": (i, [vp, i, i, i, vp, vp, vp]),
        "u15h_stack_check": (i, [vp, i, i, i, ctypes.c_char_p, ctypes.c_size_t]),
        "u15h_norm_slot": (i, [ctypes.c_char_p, ctypes.POINTER(i), ctypes.POINTER(i),
                               ctypes.POINTER(i)]),
        "u15h_stack_bind_norm": (i, [vp, ctypes.c_char_p, vp]),
        "u15h_stack_set_norm": (i, [vp, i, i, i, vp]),
        "u15h_stack_check_full": (i, [vp, i, i, i, ctypes.c_char_p, ctypes.c_size_t]),
        "u15h_stack_layer_full": (i, [vp, vp, vp, i, ctypes.POINTER(_LayerFullIO), i, i,
                                      i]),
        "u15h_stack_forward_full": (i, [vp, vp, vp, i, i, ctypes.POINTER(_LayerFullIO),
                                        ctypes.POINTER(vp), ctypes.POINTER(vp), i, i, i]),
        "u15h_stack_layer": (i, [vp, vp, vp, i, ctypes.POINTER(_LayerIO), i,
                                 i, i, i, i]),
        "u15h_stack_forward": (i, [vp, vp, vp, ctypes.POINTER(_LayerIO), i,
                                   i, i, i]),
        "u15h_gather_rows": (i, [vp, vp, vp, vp, i, i, vp]),
        "u15h_scatter_rows": (i, [vp, vp, vp, vp, i, i, vp]),
    }
    for name, (res, args) in sigs.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def route_rows(expert) -> tuple[list[int], int, int]:
    """Stable partition of token rows by expert (0 = und, 1 = gen).

    Host-side; returns (perm, M_und, M_gen) with perm[:M_und] the und rows.
    """
    lib = load_library()
    import numpy as np
    e = np.ascontiguousarray(np.asarray(expert, dtype=np.uint8))
    M = int(e.size)
    perm = np.zeros(max(M, 1), dtype=np.int32)
    mu, mg = ctypes.c_int(0), ctypes.c_int(0)
    st = lib.u15h_route_rows(e.ctypes.data if M else None, M,
                             perm.ctypes.data, ctypes.byref(mu),
                             ctypes.byref(mg))
    if st != OK:
        raise U15hError(st, "u15h_route_rows: invalid expert ids")
    return perm[:M], mu.value, mg.value


PROJ_NAMES = ("q", "k", "v", "o", "gate", "up", "down")
UND, GEN = 0, 1
STEP_QKV, STEP_O, STEP_GATE_UP, STEP_DOWN, STEP_ALL = 1, 2, 4, 8, 15
TIER_BF16, TIER_I8 = 0, 1
FUSED_SWIGLU = 1


def weight_slot(name: str) -> tuple[int, int, int]:
    """(layer, expert, projection index) of a reference tensor name, by the
    layer binder's rule (src/u15-weights.cc:539-578); U15hError otherwise."""
    lib = load_library()
    l, e, p = ctypes.c_int(0), ctypes.c_int(0), ctypes.c_int(0)
    st = lib.u15h_weight_slot(name.encode(), ctypes.byref(l), ctypes.byref(e),
                              ctypes.byref(p))
    if st != OK:
        raise U15hError(st, f"not a projection matrix name: {name!r}")
    return l.value, e.value, p.value


def slot_name(layer: int, expert: int, proj: int) -> str:
    """The reference's tensor name of a slot (the inverse of weight_slot)."""
    pre = f"language_model.model.layers.{layer}."
    sfx = "_mot_gen" if expert == GEN else ""
    n = PROJ_NAMES[proj]
    if proj <= 3:
        return f"{pre}self_attn.{n}_proj{sfx}.weight"
    return f"{pre}mlp{sfx}.{n}_proj.weight"


NORM_NAMES = ("input_layernorm", "post_attention_layernorm", "q_norm", "k_norm",
              "q_norm_hw", "k_norm_hw")


def norm_slot(name: str) -> tuple[int, int, int]:
    """(layer, expert, norm index) of a reference norm name, by the layer
    binder's rule (src/u15-weights.cc:549-566); U15hError otherwise."""
    lib = load_library()
    l, e, w = ctypes.c_int(0), ctypes.c_int(0), ctypes.c_int(0)
    st = lib.u15h_norm_slot(name.encode(), ctypes.byref(l), ctypes.byref(e),
                            ctypes.byref(w))
    if st != OK:
        raise U15hError(st, f"not a layer norm name: {name!r}")
    return l.value, e.value, w.value


def norm_slot_name(layer: int, expert: int, which: int) -> str:
    """The reference's tensor name of a norm slot (the inverse of norm_slot):
    the layernorms suffix the module, the head norms the tensor."""
    pre = f"language_model.model.layers.{layer}."
    sfx = "_mot_gen" if expert == GEN else ""
    n = NORM_NAMES[which]
    if which <= 1:
        return f"{pre}{n}{sfx}.weight"
    return f"{pre}self_attn.{n}{sfx}.weight"


class Stack:
    """u15h_stack: n_layers MotLayers of device-pointer bindings (the
    reference's MotLayer{und, gen}, src/u15-weights.h:97-117).  Holds a
    reference to every bound tensor so the memory stays alive."""

    def __init__(self, n_layers, hidden=4096, heads=32, kv_heads=8,
                 head_dim=128, inter=12288):
        self._lib = load_library()
        h = ctypes.c_void_p()
        st = self._lib.u15h_stack_create(n_layers, hidden, heads, kv_heads,
                                         head_dim, inter, ctypes.byref(h))
        if st != OK:
            raise U15hError(st, "u15h_stack_create: invalid shape")
        self._h = h
        self.n_layers = n_layers
        self.heads, self.kv_heads, self.head_dim = heads, kv_heads, head_dim
        self.hidden, self.qdim = hidden, heads * head_dim
        self.kvdim, self.inter = kv_heads * head_dim, inter
        self._keep = {}

    def shape(self, proj):
        """(N, K) of a projection."""
        return {0: (self.qdim, self.hidden), 1: (self.kvdim, self.hidden),
                2: (self.kvdim, self.hidden), 3: (self.hidden, self.qdim),
                4: (self.inter, self.hidden), 5: (self.inter, self.hidden),
                6: (self.hidden, self.inter)}[proj]

    def bind(self, name, w):
        l, e, p = weight_slot(name)
        _need(w, torch.bfloat16, self.shape(p), name)
        st = self._lib.u15h_stack_bind(self._h, name.encode(), _ptr(w))
        if st != OK:
            raise U15hError(st, f"u15h_stack_bind({name})")
        self._keep[(l, e, p, "w")] = w

    def bind_i8(self, name, wq, sw):
        l, e, p = weight_slot(name)
        N, K = self.shape(p)
        _need(wq, torch.int8, (N, K), name)
        _need(sw, torch.float32, (N,), name + " scales")
        st = self._lib.u15h_stack_bind_i8(self._h, name.encode(), _ptr(wq),
                                          _ptr(sw))
        if st != OK:
            raise U15hError(st, f"u15h_stack_bind_i8({name})")
        self._keep[(l, e, p, "q")] = (wq, sw)

    def bind_norm(self, name, w):
        l, e, k = norm_slot(name)
        _need(w, torch.bfloat16, (self.hidden if k <= 1 else self.head_dim // 2,), name)
        st = self._lib.u15h_stack_bind_norm(self._h, name.encode(), _ptr(w))
        if st != OK:
            raise U15hError(st, f"u15h_stack_bind_norm({name})")
        self._keep[(l, e, k, "n")] = w

    def check_full(self, need_und=True, need_gen=True, tier=TIER_BF16):
        """None if every matrix and norm of the pass is bound, else the first
        missing reference name."""
        buf = ctypes.create_string_buffer(256)
        st = self._lib.u15h_stack_check_full(self._h, int(need_und), int(need_gen),
                                             tier, buf, 256)
        return None if st == OK else buf.value.decode()

    def check(self, need_und=True, need_gen=True, tier=TIER_BF16):
        """None if the pass's matrices are bound, else the first missing
        reference name."""
        buf = ctypes.create_string_buffer(256)
        st = self._lib.u15h_stack_check(self._h, int(need_und), int(need_gen),
                                        tier, buf, 256)
        return None if st == OK else buf.value.decode()

    def close(self):
        if getattr(self, "_h", None):
            self._lib.u15h_stack_destroy(self._h)
            self._h = None
        self._keep = {}

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def layer_io(**bufs):
    """A u15h_layer_io from torch tensors (missing entries are NULL).  The
    tensors ride along (`io.tensors`) so that Ops.stack_layer and
    Ops.stack_forward can check them against the stack before the call."""
    unknown = set(bufs) - {n for n, _ in _LayerIO._fields_}
    if unknown:
        raise ValueError(f"layer_io: unknown buffers {sorted(unknown)}")
    io = _LayerIO()
    for name, _ in _LayerIO._fields_:
        t = bufs.get(name)
        setattr(io, name, None if t is None else t.data_ptr())
    io.tensors = dict(bufs)
    return io


# Which io buffers a step reads and writes, with their widths (a function
# of the stack): (name, width) pairs; the int8 tier adds xq and sx.
def _step_buffers(stack, step, fused):
    H, Q, KV, I = stack.hidden, stack.qdim, stack.kvdim, stack.inter
    if step == STEP_QKV:
        return [("x", H), ("q", Q), ("k", KV), ("v", KV)]
    if step == STEP_O:
        return [("attn", Q), ("o", H)]
    if step == STEP_GATE_UP:
        return [("x2", H), ("h", I)] if fused else \
            [("x2", H), ("gate", I), ("up", I)]
    return [("h", I), ("down", H)]


def _check_io(stack, io, M, steps, tier, flags):
    """Every io buffer the steps use: bf16 [M][width], contiguous, on the
    GPU; int8 tier: xq int8 [M][>= the widest K], sx f32 [M].  The C ABI
    cannot see sizes, so a short buffer would be written past its end."""
    tensors = getattr(io, "tensors", None)
    if tensors is None:
        raise ValueError("io must come from u15h.layer_io()")
    if M == 0:
        return
    # The io's pointers are fixed when it is made, so a passed check holds
    # for every later call with the same shapes (the bench's timed loop
    # calls the stack per step).
    key = (stack.hidden, stack.qdim, stack.kvdim, stack.inter, M, steps,
           tier, flags)
    done = io.__dict__.setdefault("checked", set())
    if key in done:
        return
    fused = bool(flags & FUSED_SWIGLU)
    want = []
    for b in range(4):
        step = 1 << b
        if steps & step:
            want += [(f"io.{n}", tensors.get(n), torch.bfloat16, (M, w))
                     for n, w in _step_buffers(stack, step, fused)]
    if tier == TIER_I8:
        xq = tensors.get("xq")
        kmax = max(stack.hidden, stack.qdim, stack.inter)
        if xq is None or xq.dtype != torch.int8 or xq.dim() != 2 or \
                xq.shape[0] != M or xq.shape[1] < kmax:
            raise ValueError(f"io.xq must be an int8 tensor [{M}][>= {kmax}]")
        want += [("io.xq", xq, torch.int8, tuple(xq.shape)),
                 ("io.sx", tensors.get("sx"), torch.float32, (M,))]
    # sizes of every buffer first (the usual mistake), then placement
    for name, t, dtype, shape in want:
        if t is None:
            raise ValueError(f"{name} is required")
        if t.dtype != dtype:
            raise TypeError(f"{name}: dtype {t.dtype}, expected {dtype}")
        if tuple(t.shape) != tuple(shape):
            raise ValueError(f"{name}: shape {tuple(t.shape)}, expected {tuple(shape)}")
    for name, t, dtype, shape in want:
        _need(t, dtype, shape, name)
    done.add(key)


def build_rope_tables(pos_t, pos_h, pos_w, head_dim, d_t, d_h,
                      theta_t=5000000.0, theta_hw=10000.0):
    """MetalOps::build_rope_tables on the host: (cos, sin) numpy f32
    [tokens][head_dim]."""
    import numpy as np
    lib = load_library()
    pt = np.ascontiguousarray(pos_t, dtype=np.int32)
    ph = np.ascontiguousarray(pos_h, dtype=np.int32)
    pw = np.ascontiguousarray(pos_w, dtype=np.int32)
    T = int(pt.size)
    if ph.size != T or pw.size != T:
        raise ValueError("pos_t, pos_h, pos_w must have one entry per token")
    cs = np.empty((max(T, 1), head_dim), np.float32)
    sn = np.empty((max(T, 1), head_dim), np.float32)
    st = lib.u15h_build_rope_tables(pt.ctypes.data, ph.ctypes.data,
                                    pw.ctypes.data, T, head_dim, d_t, d_h,
                                    theta_t, theta_hw, cs.ctypes.data,
                                    sn.ctypes.data)
    if st != OK:
        raise U15hError(st, "u15h_build_rope_tables: invalid arguments")
    return cs[:T], sn[:T]


def qweight_geometry(K, scales_cols, codes_cols):
    """(bits, group) of a quantized pack from its shapes, or U15hError if
    they do not close (bind_matrix_'s rule, src/u15-weights.cc:247-325)."""
    lib = load_library()
    b, g = ctypes.c_int(0), ctypes.c_int(0)
    st = lib.u15h_qweight_geometry(K, scales_cols, codes_cols, ctypes.byref(b),
                                   ctypes.byref(g))
    if st != OK:
        raise U15hError(st, f"pack shapes do not close: K={K}, scales cols="
                        f"{scales_cols}, codes cols={codes_cols}")
    return b.value, g.value


def load_bf16(ops, path, name):
    """A tensor of a safetensors file on the device as bf16, the way the
    reference's bind_bf16_ reads it (src/u15-weights.cc:96-151): the dtype
    is per tensor in the file's header; BF16 is bound as it sits, F32 and
    F16 are converted on the device with the loader's RNE."""
    from safetensors import safe_open
    with safe_open(str(path), framework="pt") as f:
        t = f.get_tensor(name)
    if t.dtype == torch.bfloat16:
        return t.cuda().contiguous()
    if t.dtype not in (torch.float32, torch.float16):
        raise U15hError(EINVAL, f"{name}: dtype {t.dtype} is not BF16/F32/F16")
    src = t.cuda().contiguous()
    n = src.numel()
    pad = (-n) % 4
    if pad:
        src = torch.cat([src.reshape(-1), src.new_zeros(pad)])
    dst = torch.empty(n + pad, dtype=torch.bfloat16, device="cuda")
    if t.dtype == torch.float32:
        ops.f32_to_bf16(src.reshape(-1), dst)
    else:
        ops.f16_to_bf16(src.reshape(-1), dst)
    return dst[:n].reshape(t.shape)


def load_matrix(ops, path, name, K):
    """A projection matrix `name` of a safetensors file, dense or quantized,
    by bind_matrix_'s rule (src/u15-weights.cc:247-325): a `.scales`
    sibling means `.weight` holds u32 codes, and (bits, group) follow from
    the shapes.  Returns ("dense", w bf16 [N][K]) or ("affine", (codes
    int32, scales bf16, biases bf16, bits, group))."""
    from safetensors import safe_open
    with safe_open(str(path), framework="pt") as f:
        keys = set(f.keys())
        if name + ".scales" in keys and name + ".weight" in keys:
            codes = f.get_tensor(name + ".weight")
            scols = f.get_slice(name + ".scales").get_shape()[1]
        else:
            codes = None
    if codes is None:
        return "dense", load_bf16(ops, path, name + ".weight")
    bits, group = qweight_geometry(K, scols, codes.shape[1])
    if codes.dtype not in (torch.int32, torch.uint32):
        raise U15hError(EINVAL, f"{name}.weight: codes must be 32-bit")
    codes = codes.view(torch.int32).cuda().contiguous()
    scales = load_bf16(ops, path, name + ".scales").contiguous()
    biases = load_bf16(ops, path, name + ".biases").contiguous()
    return "affine", (codes, scales, biases, bits, group)


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(stream):
    if stream is None:
        stream = torch.cuda.current_stream()
    return ctypes.c_void_p(stream.cuda_stream)


def _need(t, dtype, shape, name):
    if t is None:
        raise ValueError(f"{name} is required")
    if t.dtype != dtype:
        raise TypeError(f"{name}: dtype {t.dtype}, expected {dtype}")
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name}: shape {tuple(t.shape)}, expected {tuple(shape)}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be on the GPU")


def layer_scratch(stack, M, tier=TIER_BF16, device="cuda"):
    """The scratch buffers of u15h_stack_layer_full for M rows."""
    def bf(n):
        return torch.empty(M, n, dtype=torch.bfloat16, device=device)
    sc = dict(q=bf(stack.qdim), k=bf(stack.kvdim), v=bf(stack.kvdim),
              attn=bf(stack.qdim), proj=bf(stack.hidden), h=bf(stack.inter))
    if tier == TIER_I8:
        sc["up"] = bf(stack.inter)
        sc["xq"] = torch.empty(M, max(stack.hidden, stack.qdim, stack.inter),
                               dtype=torch.int8, device=device)
        sc["sx"] = torch.empty(M, dtype=torch.float32, device=device)
    else:
        sc["normed"] = bf(stack.hidden)
    return sc


class Ops:
    """The projection-GEMM operator surface on one gfx950 device."""

    def __init__(self, device: int = 0):
        self._lib = load_library()
        ctx = ctypes.c_void_p()
        st = self._lib.u15h_create(device, ctypes.byref(ctx))
        if st != OK:
            raise U15hError(st, f"u15h_create(device={device}): "
                            f"{self._lib.u15h_status_str(st).decode()}")
        self._ctx = ctx
        self.device = device

    def close(self):
        if getattr(self, "_ctx", None):
            self._lib.u15h_destroy(self._ctx)
            self._ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _check(self, st, what):
        if st != OK:
            msg = self._lib.u15h_last_error(self._ctx).decode()
            raise U15hError(st, f"{what}: "
                            f"{self._lib.u15h_status_str(st).decode()}: {msg}")

    # ---- dense -------------------------------------------------------
    def linear(self, x, w, bias, y, M, K, N, stream=None):
        """y[M][N] = x[M][K] . w[N][K]^T (+ bias) -- MetalOps::linear."""
        _need(x, torch.bfloat16, (M, K), "x")
        _need(w, torch.bfloat16, (N, K), "w")
        _need(y, torch.bfloat16, (M, N), "y")
        if bias is not None:
            _need(bias, torch.bfloat16, (N,), "bias")
        st = self._lib.u15h_linear(self._ctx, _stream(stream), _ptr(x),
                                   _ptr(w), _ptr(bias), _ptr(y), M, K, N)
        self._check(st, "u15h_linear")

    def mot_linear(self, x, M_und, M_gen, K, projs, stream=None,
                   noalloc=False):
        """Grouped MoT GEMM.  projs: list of dicts with keys
        w_und, w_gen, y and optionally bias_und, bias_gen.  noalloc=True
        calls u15h_mot_linear_noalloc (split-K sums in the library's static
        scratch; no device allocation)."""
        M = M_und + M_gen
        _need(x, torch.bfloat16, (M, K), "x")
        if not 1 <= len(projs) <= MAX_PROJ:
            raise ValueError(f"1..{MAX_PROJ} projections per launch")
        arr = (_MotProj * len(projs))()
        for i, p in enumerate(projs):
            N = p["y"].shape[1]
            _need(p["y"], torch.bfloat16, (M, N), f"projs[{i}].y")
            if M_und:
                _need(p["w_und"], torch.bfloat16, (N, K), f"projs[{i}].w_und")
            if M_gen:
                _need(p["w_gen"], torch.bfloat16, (N, K), f"projs[{i}].w_gen")
            for b in ("bias_und", "bias_gen"):
                if p.get(b) is not None:
                    _need(p[b], torch.bfloat16, (N,), f"projs[{i}].{b}")
            arr[i] = _MotProj(
                p["w_und"].data_ptr() if p.get("w_und") is not None else None,
                p["w_gen"].data_ptr() if p.get("w_gen") is not None else None,
                p["bias_und"].data_ptr() if p.get("bias_und") is not None else None,
                p["bias_gen"].data_ptr() if p.get("bias_gen") is not None else None,
                p["y"].data_ptr(), N)
        fn = self._lib.u15h_mot_linear_noalloc if noalloc else self._lib.u15h_mot_linear
        st = fn(self._ctx, _stream(stream), _ptr(x), M_und, M_gen, K, arr,
                len(projs))
        self._check(st, "u15h_mot_linear_noalloc" if noalloc else "u15h_mot_linear")

    # ---- affine-quantized weights ---------------------------------------
    @staticmethod
    def _qweight(qw, N, K):
        codes, scales, biases, bits, group = qw
        _need(codes, torch.int32, (N, K * bits // 32), "codes")
        _need(scales, torch.bfloat16, (N, K // group), "scales")
        _need(biases, torch.bfloat16, (N, K // group), "biases")
        return _QWeight(codes.data_ptr(), scales.data_ptr(),
                        biases.data_ptr(), bits, group)

    def dequant_affine(self, qw, N, K, w_out, stream=None):
        """Expand qw = (codes int32 [N][K*bits/32], scales bf16, biases bf16,
        bits, group) into w_out bf16 [N][K]."""
        _need(w_out, torch.bfloat16, (N, K), "w_out")
        q = self._qweight(qw, N, K)
        st = self._lib.u15h_dequant_affine(self._ctx, _stream(stream),
                                           ctypes.byref(q), N, K, _ptr(w_out))
        self._check(st, "u15h_dequant_affine")

    def linear_q(self, x, qw, bias, y, M, K, N, stream=None):
        """MetalOps::linear on a QWeight: dequant once, then the dense GEMM."""
        _need(x, torch.bfloat16, (M, K), "x")
        _need(y, torch.bfloat16, (M, N), "y")
        if bias is not None:
            _need(bias, torch.bfloat16, (N,), "bias")
        q = self._qweight(qw, N, K)
        st = self._lib.u15h_linear_q(self._ctx, _stream(stream), _ptr(x),
                                     ctypes.byref(q), _ptr(bias), _ptr(y),
                                     M, K, N)
        self._check(st, "u15h_linear_q")

    def bias_add(self, y, bias, stream=None):
        M, N = y.shape
        _need(y, torch.bfloat16, (M, N), "y")
        _need(bias, torch.bfloat16, (N,), "bias")
        st = self._lib.u15h_bias_add(self._ctx, _stream(stream), _ptr(y),
                                     _ptr(bias), M, N)
        self._check(st, "u15h_bias_add")

    def f32_to_bf16(self, src, dst, stream=None):
        _need(src, torch.float32, tuple(src.shape), "src")
        _need(dst, torch.bfloat16, tuple(src.shape), "dst")
        st = self._lib.u15h_f32_to_bf16(self._ctx, _stream(stream), _ptr(src),
                                        src.numel(), _ptr(dst))
        self._check(st, "u15h_f32_to_bf16")

    def f16_to_bf16(self, src, dst, stream=None):
        """src: f16 values (torch.float16) or their bit patterns (int16)."""
        if src.dtype not in (torch.float16, torch.int16):
            raise TypeError("src must be float16 (or its int16 bits)")
        _need(dst, torch.bfloat16, tuple(src.shape), "dst")
        if not src.is_contiguous():
            raise ValueError("src must be contiguous")
        st = self._lib.u15h_f16_to_bf16(self._ctx, _stream(stream), _ptr(src),
                                        src.numel(), _ptr(dst))
        self._check(st, "u15h_f16_to_bf16")

    def repack_affine_i8(self, qw, N, K, wq, sw, stream=None):
        """Affine pack -> per-channel int8 (wq int8 [N][K], sw f32 [N])."""
        _need(wq, torch.int8, (N, K), "wq")
        _need(sw, torch.float32, (N,), "sw")
        q = self._qweight(qw, N, K)
        st = self._lib.u15h_repack_affine_i8(self._ctx, _stream(stream),
                                             ctypes.byref(q), N, K, _ptr(wq),
                                             _ptr(sw))
        self._check(st, "u15h_repack_affine_i8")

    # ---- swiglu --------------------------------------------------------
    def swiglu_fused(self, x, w_fused, y, M, K, inter, stream=None):
        """MetalOps::swiglu_fused: w_fused [2*inter][K] row-interleaved
        (row 2i gate i, row 2i+1 up i)."""
        _need(x, torch.bfloat16, (M, K), "x")
        _need(w_fused, torch.bfloat16, (2 * inter, K), "w_fused")
        _need(y, torch.bfloat16, (M, inter), "y")
        st = self._lib.u15h_swiglu_fused(self._ctx, _stream(stream), _ptr(x),
                                         _ptr(w_fused), _ptr(y), M, K, inter)
        self._check(st, "u15h_swiglu_fused")

    def swiglu(self, gate, up, out, stream=None):
        n = gate.numel()
        for t, nm in ((gate, "gate"), (up, "up"), (out, "out")):
            _need(t, torch.bfloat16, tuple(gate.shape), nm)
        st = self._lib.u15h_swiglu(self._ctx, _stream(stream), _ptr(gate),
                                   _ptr(up), _ptr(out), n)
        self._check(st, "u15h_swiglu")

    def swiglu_quant_i8(self, gate, up, q, s, h=None, stream=None):
        """h = swiglu(gate, up) and its per-token int8 codes q, scales s in
        one pass (h written only when given)."""
        if gate.dim() != 2:
            raise ValueError("gate must be [rows][inter]")
        rows, inter = gate.shape
        _need(gate, torch.bfloat16, (rows, inter), "gate")
        _need(up, torch.bfloat16, (rows, inter), "up")
        _need(q, torch.int8, (rows, inter), "q")
        _need(s, torch.float32, (rows,), "s")
        if h is not None:
            _need(h, torch.bfloat16, (rows, inter), "h")
        st = self._lib.u15h_swiglu_quant_i8(self._ctx, _stream(stream), _ptr(gate),
                                            _ptr(up), rows, inter, _ptr(h), _ptr(q),
                                            _ptr(s))
        self._check(st, "u15h_swiglu_quant_i8")

    def mot_gate_up_swiglu(self, x, M_und, M_gen, K, wg_und, wu_und, wg_gen,
                           wu_gen, h, stream=None):
        M = M_und + M_gen
        I = h.shape[1]
        _need(x, torch.bfloat16, (M, K), "x")
        _need(h, torch.bfloat16, (M, I), "h")
        if M_und:
            _need(wg_und, torch.bfloat16, (I, K), "wg_und")
            _need(wu_und, torch.bfloat16, (I, K), "wu_und")
        if M_gen:
            _need(wg_gen, torch.bfloat16, (I, K), "wg_gen")
            _need(wu_gen, torch.bfloat16, (I, K), "wu_gen")
        st = self._lib.u15h_mot_gate_up_swiglu(
            self._ctx, _stream(stream), _ptr(x), M_und, M_gen, K,
            _ptr(wg_und), _ptr(wu_und), _ptr(wg_gen), _ptr(wu_gen), _ptr(h), I)
        self._check(st, "u15h_mot_gate_up_swiglu")

    # ---- int8 tier -----------------------------------------------------
    def enable_i8_gemm(self, want: bool) -> bool:
        """MetalOps::enable_i8_gemm: returns whether the tier is ON."""
        return bool(self._lib.u15h_enable_i8_gemm(self._ctx, 1 if want else 0))

    def release_i8_scratch(self):
        self._lib.u15h_release_i8_scratch(self._ctx)

    def i8_min_m(self) -> int:
        return int(self._lib.u15h_i8_min_m(self._ctx))

    def quant_rows_i8(self, x, q, s, stream=None):
        rows, K = x.shape
        _need(x, torch.bfloat16, (rows, K), "x")
        _need(q, torch.int8, (rows, K), "q")
        _need(s, torch.float32, (rows,), "s")
        st = self._lib.u15h_quant_rows_i8(self._ctx, _stream(stream), _ptr(x),
                                          rows, K, _ptr(q), _ptr(s))
        self._check(st, "u15h_quant_rows_i8")

    def _i8_projs(self, M, M_und, M_gen, K, projs, ydtype, need_scales):
        if not 1 <= len(projs) <= MAX_PROJ:
            raise ValueError(f"1..{MAX_PROJ} projections per launch")
        arr = (_MotProjI8 * len(projs))()
        for i, p in enumerate(projs):
            N = p["y"].shape[1]
            _need(p["y"], ydtype, (M, N), f"projs[{i}].y")
            for g, mg in (("und", M_und), ("gen", M_gen)):
                if mg:
                    _need(p["wq_" + g], torch.int8, (N, K), f"projs[{i}].wq_{g}")
                    if need_scales:
                        _need(p["sw_" + g], torch.float32, (N,), f"projs[{i}].sw_{g}")

            def g_(k):
                t = p.get(k)
                return t.data_ptr() if t is not None else None
            arr[i] = _MotProjI8(g_("wq_und"), g_("sw_und"), g_("wq_gen"),
                                g_("sw_gen"), p["y"].data_ptr(), N)
        return arr

    def mot_gemm_i8_i32(self, xq, M_und, M_gen, K, projs, stream=None):
        M = M_und + M_gen
        _need(xq, torch.int8, (M, K), "xq")
        arr = self._i8_projs(M, M_und, M_gen, K, projs, torch.int32, False)
        st = self._lib.u15h_mot_gemm_i8_i32(self._ctx, _stream(stream),
                                            _ptr(xq), M_und, M_gen, K, arr,
                                            len(projs))
        self._check(st, "u15h_mot_gemm_i8_i32")

    def mot_gemm_i8(self, xq, sx, M_und, M_gen, K, projs, stream=None):
        M = M_und + M_gen
        _need(xq, torch.int8, (M, K), "xq")
        _need(sx, torch.float32, (M,), "sx")
        arr = self._i8_projs(M, M_und, M_gen, K, projs, torch.bfloat16, True)
        st = self._lib.u15h_mot_gemm_i8(self._ctx, _stream(stream), _ptr(xq),
                                        _ptr(sx), M_und, M_gen, K, arr,
                                        len(projs))
        self._check(st, "u15h_mot_gemm_i8")

    # ---- profiling -------------------------------------------------------
    def profile_next_gemm(self, event):
        """Record the raw hipEvent_t `event` (a ctypes.c_void_p or int
        handle) right after the next GEMM kernel, before any split-K
        reduction kernel."""
        h = event if isinstance(event, ctypes.c_void_p) else ctypes.c_void_p(event)
        self._check(self._lib.u15h_profile_next_gemm(self._ctx, h),
                    "u15h_profile_next_gemm")

    def profile_bracket_next_gemm(self, before, after):
        """Record raw hipEvent_t handles right before and right after the
        next GEMM kernel (either may be None)."""
        def h(e):
            if e is None or isinstance(e, ctypes.c_void_p):
                return e
            return ctypes.c_void_p(e)
        self._check(self._lib.u15h_profile_bracket_next_gemm(self._ctx, h(before),
                                                             h(after)),
                    "u15h_profile_bracket_next_gemm")

    def profile_next_kernels(self, quant=(None, None), gemm=(None, None),
                             reduce=(None, None)):
        """Bind raw hipEvent_t pairs to the start and end timestamps of the
        next quantiser, GEMM kernel and reduction kernel launched through
        this context (u15h_profile_next_kernels)."""
        def h(e):
            if e is None or isinstance(e, ctypes.c_void_p):
                return e
            return ctypes.c_void_p(e)
        self._check(self._lib.u15h_profile_next_kernels(
            self._ctx, h(quant[0]), h(quant[1]), h(gemm[0]), h(gemm[1]),
            h(reduce[0]), h(reduce[1])), "u15h_profile_next_kernels")

    # ---- the step after the q/k projections -------------------------------
    def _head(self, x, heads, head_dim):
        tokens = x.shape[0]
        _need(x, torch.bfloat16, (tokens, heads * head_dim), "x")
        return tokens

    def split_qk_norm(self, x, w_t, w_hw, heads, head_dim, eps=1e-6,
                      stream=None):
        """MetalOps::split_qk_norm on x [tokens][heads*head_dim] in place."""
        T = self._head(x, heads, head_dim)
        _need(w_t, torch.bfloat16, (head_dim // 2,), "w_t")
        _need(w_hw, torch.bfloat16, (head_dim // 2,), "w_hw")
        st = self._lib.u15h_split_qk_norm(self._ctx, _stream(stream), _ptr(x),
                                          _ptr(w_t), _ptr(w_hw), heads, T,
                                          head_dim, eps)
        self._check(st, "u15h_split_qk_norm")

    def split_rope(self, x, cos, sin, heads, head_dim, d_t, d_h, stream=None):
        """MetalOps::split_rope with device f32 tables [tokens][head_dim]."""
        T = self._head(x, heads, head_dim)
        _need(cos, torch.float32, (T, head_dim), "cos")
        _need(sin, torch.float32, (T, head_dim), "sin")
        st = self._lib.u15h_split_rope(self._ctx, _stream(stream), _ptr(x),
                                       _ptr(cos), _ptr(sin), heads, T,
                                       head_dim, d_t, d_h)
        self._check(st, "u15h_split_rope")

    def split_qk_norm_rope(self, x, w_t, w_hw, cos, sin, heads, head_dim, d_t,
                           d_h, eps=1e-6, stream=None):
        T = self._head(x, heads, head_dim)
        _need(w_t, torch.bfloat16, (head_dim // 2,), "w_t")
        _need(w_hw, torch.bfloat16, (head_dim // 2,), "w_hw")
        _need(cos, torch.float32, (T, head_dim), "cos")
        _need(sin, torch.float32, (T, head_dim), "sin")
        st = self._lib.u15h_split_qk_norm_rope(
            self._ctx, _stream(stream), _ptr(x), _ptr(w_t), _ptr(w_hw),
            _ptr(cos), _ptr(sin), heads, T, head_dim, d_t, d_h, eps)
        self._check(st, "u15h_split_qk_norm_rope")

    def mot_attention_prologue(self, q, k, v, und, gen, cos, sin, M_und,
                               M_gen, hq, hkv, head_dim, d_t, d_h, k_cache,
                               v_cache, offset=0, eps=1e-6, stream=None):
        """u15h_mot_attention_prologue: q [T][hq*d] normed and rotated in
        place, k normed and rotated into k_cache [hkv][cap][d] at token
        offset `offset`, v copied into v_cache; rows [0, M_und) take `und`'s
        norm weights (a dict q_t, q_hw, k_t, k_hw of [d/2] bf16 tensors),
        the rest `gen`'s."""
        T = M_und + M_gen
        _need(q, torch.bfloat16, (T, hq * head_dim), "q")
        _need(k, torch.bfloat16, (T, hkv * head_dim), "k")
        _need(v, torch.bfloat16, (T, hkv * head_dim), "v")
        _need(cos, torch.float32, (T, head_dim), "cos")
        _need(sin, torch.float32, (T, head_dim), "sin")
        if k_cache.dim() != 3:
            raise ValueError("k_cache must be [hkv][cap][head_dim]")
        cap = k_cache.shape[1]
        _need(k_cache, torch.bfloat16, (hkv, cap, head_dim), "k_cache")
        _need(v_cache, torch.bfloat16, (hkv, cap, head_dim), "v_cache")
        norms = []
        for tag, n, rows in (("und", und, M_und), ("gen", gen, M_gen)):
            if rows == 0:
                norms.append(None)
                continue
            for f in ("q_t", "q_hw", "k_t", "k_hw"):
                _need(n.get(f) if n else None, torch.bfloat16,
                      (head_dim // 2,), f"{tag}.{f}")
            norms.append(_QkNorm(*[_ptr(n[f]) for f in ("q_t", "q_hw", "k_t", "k_hw")]))
        st = self._lib.u15h_mot_attention_prologue(
            self._ctx, _stream(stream), _ptr(q), _ptr(k), _ptr(v),
            None if norms[0] is None else ctypes.byref(norms[0]),
            None if norms[1] is None else ctypes.byref(norms[1]),
            _ptr(cos), _ptr(sin), M_und, M_gen, hq, hkv, head_dim, d_t, d_h,
            eps, _ptr(k_cache), _ptr(v_cache), cap, offset)
        self._check(st, "u15h_mot_attention_prologue")

    def stack_layer_full(self, stack, layer, M_und, M_gen, x, k_cache, v_cache,
                         cos, sin, kv_off=0, kv_len=None, mode=0, t_index=None,
                         d_t=None, d_h=None, eps=1e-6, tier=TIER_BF16, scratch=None,
                         stream=None):
        """u15h_stack_layer_full: one whole decoder layer of the stack on
        the residual stream x [M][hidden] (updated in place), attending this
        layer's caches [kv_heads][cap][head_dim] over keys [0, kv_len) with
        the pass at kv_off.  `scratch` (a dict from layer_scratch) is made
        when not given and returned."""
        M = M_und + M_gen
        hd = stack.head_dim
        d_t = hd // 2 if d_t is None else d_t
        d_h = hd // 4 if d_h is None else d_h
        kv_len = kv_off + M if kv_len is None else kv_len
        _need(x, torch.bfloat16, (M, stack.hidden), "x")
        cap = k_cache.shape[1]
        _need(k_cache, torch.bfloat16, (stack.kv_heads, cap, hd), "k_cache")
        _need(v_cache, torch.bfloat16, (stack.kv_heads, cap, hd), "v_cache")
        _need(cos, torch.float32, (M, hd), "cos")
        _need(sin, torch.float32, (M, hd), "sin")
        if mode == 2 and (t_index is None or t_index.dtype != torch.int32 or
                          t_index.numel() < max(kv_len, kv_off + M)):
            raise ValueError("t_index: int32 covering max(kv_len, kv_off + M)")
        if scratch is None:
            scratch = layer_scratch(stack, M, tier)
        sc = scratch
        io = _LayerFullIO(
            _ptr(x), _ptr(sc.get("normed")), _ptr(sc["q"]), _ptr(sc["k"]), _ptr(sc["v"]),
            _ptr(sc["attn"]), _ptr(sc["proj"]), _ptr(sc["h"]), _ptr(sc.get("up")),
            _ptr(sc.get("xq")), _ptr(sc.get("sx")), _ptr(k_cache), _ptr(v_cache),
            cap, kv_off, kv_len, mode, _ptr(t_index), _ptr(cos), _ptr(sin), d_t, d_h, eps)
        st = self._lib.u15h_stack_layer_full(self._ctx, _stream(stream), stack._h, layer,
                                             ctypes.byref(io), M_und, M_gen, tier)
        self._check(st, "u15h_stack_layer_full")
        return scratch

    def stack_forward_full(self, stack, first, count, M_und, M_gen, x, k_caches,
                           v_caches, cos, sin, kv_off=0, kv_len=None, mode=0,
                           t_index=None, d_t=None, d_h=None, eps=1e-6, tier=TIER_BF16,
                           scratch=None, stream=None):
        """u15h_stack_forward_full: whole layers [first, first + count) on
        the residual stream x [M][hidden] (updated in place), layer first + i
        attending k_caches[i] / v_caches[i] ([kv_heads][cap][head_dim], one
        capacity) over keys [0, kv_len) with the pass at kv_off.  Between
        layers the residual add and the next input norm run as one pass.
        `scratch` (a dict from layer_scratch) is made when not given and
        returned."""
        M = M_und + M_gen
        hd = stack.head_dim
        d_t = hd // 2 if d_t is None else d_t
        d_h = hd // 4 if d_h is None else d_h
        kv_len = kv_off + M if kv_len is None else kv_len
        if count < 1:
            raise ValueError("count must be at least 1")
        if len(k_caches) != count or len(v_caches) != count:
            raise ValueError(f"k_caches and v_caches must hold {count} caches")
        _need(x, torch.bfloat16, (M, stack.hidden), "x")
        cap = k_caches[0].shape[1]
        for n, c in enumerate(list(k_caches) + list(v_caches)):
            _need(c, torch.bfloat16, (stack.kv_heads, cap, hd), f"cache {n}")
        _need(cos, torch.float32, (M, hd), "cos")
        _need(sin, torch.float32, (M, hd), "sin")
        if mode == 2 and (t_index is None or t_index.dtype != torch.int32 or
                          t_index.numel() < max(kv_len, kv_off + M)):
            raise ValueError("t_index: int32 covering max(kv_len, kv_off + M)")
        if scratch is None:
            scratch = layer_scratch(stack, M, tier)
        sc = scratch
        io = _LayerFullIO(
            _ptr(x), _ptr(sc.get("normed")), _ptr(sc["q"]), _ptr(sc["k"]), _ptr(sc["v"]),
            _ptr(sc["attn"]), _ptr(sc["proj"]), _ptr(sc["h"]), _ptr(sc.get("up")),
            _ptr(sc.get("xq")), _ptr(sc.get("sx")), None, None,
            cap, kv_off, kv_len, mode, _ptr(t_index), _ptr(cos), _ptr(sin), d_t, d_h, eps)
        kc = (ctypes.c_void_p * count)(*[_ptr(c) for c in k_caches])
        vc = (ctypes.c_void_p * count)(*[_ptr(c) for c in v_caches])
        st = self._lib.u15h_stack_forward_full(self._ctx, _stream(stream), stack._h, first,
                                               count, ctypes.byref(io), kc, vc, M_und,
                                               M_gen, tier)
        self._check(st, "u15h_stack_forward_full")
        return scratch

    # ---- the layer norms and the residual add --------------------------
    def rms_norm(self, x, w, y, eps=1e-6, stream=None):
        """MetalOps::rms_norm: y [rows][dim] = bf16((x * inv) * w); y may
        be x."""
        if x.dim() != 2:
            raise ValueError("x must be [rows][dim]")
        rows, dim = x.shape
        _need(x, torch.bfloat16, (rows, dim), "x")
        _need(w, torch.bfloat16, (dim,), "w")
        _need(y, torch.bfloat16, (rows, dim), "y")
        st = self._lib.u15h_rms_norm(self._ctx, _stream(stream), _ptr(x), _ptr(w),
                                     _ptr(y), rows, dim, eps)
        self._check(st, "u15h_rms_norm")

    def rms_norm_quant_i8(self, x, w, q, s, y=None, eps=1e-6, stream=None):
        """The norm with the int8 tier's per-token quantisation of its bf16
        results: q [rows][dim] int8, s [rows] f32 (and y when given)."""
        if x.dim() != 2:
            raise ValueError("x must be [rows][dim]")
        rows, dim = x.shape
        _need(x, torch.bfloat16, (rows, dim), "x")
        _need(w, torch.bfloat16, (dim,), "w")
        _need(q, torch.int8, (rows, dim), "q")
        _need(s, torch.float32, (rows,), "s")
        if y is not None:
            _need(y, torch.bfloat16, (rows, dim), "y")
        st = self._lib.u15h_rms_norm_quant_i8(self._ctx, _stream(stream), _ptr(x),
                                              _ptr(w), rows, dim, eps, _ptr(y),
                                              _ptr(q), _ptr(s))
        self._check(st, "u15h_rms_norm_quant_i8")

    def mot_rms_norm(self, x, M_und, M_gen, w_und, w_gen, y=None, delta=None,
                     q=None, s=None, eps=1e-6, stream=None):
        """u15h_mot_rms_norm: with `delta`, x += delta first (in place);
        then y = the norm of x's rows (w_und for the first M_und, w_gen for
        the rest) and/or its per-token int8 codes q and scales s."""
        rows = M_und + M_gen
        if x.dim() != 2 or x.shape[0] != rows:
            raise ValueError(f"x must be [{rows}][dim]")
        dim = x.shape[1]
        _need(x, torch.bfloat16, (rows, dim), "x")
        if M_und:
            _need(w_und, torch.bfloat16, (dim,), "w_und")
        if M_gen:
            _need(w_gen, torch.bfloat16, (dim,), "w_gen")
        for name, t, dt, shape in (("y", y, torch.bfloat16, (rows, dim)),
                                   ("delta", delta, torch.bfloat16, (rows, dim)),
                                   ("q", q, torch.int8, (rows, dim)),
                                   ("s", s, torch.float32, (rows,))):
            if t is not None:
                _need(t, dt, shape, name)
        st = self._lib.u15h_mot_rms_norm(self._ctx, _stream(stream), _ptr(x), _ptr(delta),
                                         M_und, M_gen, dim, _ptr(w_und), _ptr(w_gen),
                                         eps, _ptr(y), _ptr(q), _ptr(s))
        self._check(st, "u15h_mot_rms_norm")

    def add(self, dst, src, stream=None):
        """MetalOps::add: dst += src elementwise (bf16, f32 add)."""
        if dst.numel() != src.numel():
            raise ValueError("dst and src must have the same length")
        for name, t in (("dst", dst), ("src", src)):
            if t.dtype != torch.bfloat16 or not t.is_contiguous() or t.device.type != "cuda":
                raise ValueError(f"{name} must be a contiguous bf16 GPU tensor")
        st = self._lib.u15h_add(self._ctx, _stream(stream), _ptr(dst), _ptr(src),
                                dst.numel())
        self._check(st, "u15h_add")

    # ---- attention -------------------------------------------------------
    def sdpa(self, q, k, v, out, hkv, tk, causal=False, q_offset=0,
             stream=None):
        """MetalOps::sdpa / sdpa_steel: q, out [hq][tq][d]; k, v caches
        [hkv][cap][d] with keys [0, tk) in use."""
        hq, tq, d = q.shape
        cap = k.shape[1]
        _need(q, torch.bfloat16, (hq, tq, d), "q")
        _need(out, torch.bfloat16, (hq, tq, d), "out")
        _need(k, torch.bfloat16, (hkv, cap, d), "k")
        _need(v, torch.bfloat16, (hkv, cap, d), "v")
        st = self._lib.u15h_sdpa(self._ctx, _stream(stream), _ptr(q), _ptr(k),
                                 _ptr(v), _ptr(out), hq, hkv, tq, tk, d, cap,
                                 1 if causal else 0, q_offset)
        self._check(st, "u15h_sdpa")

    def sdpa_block_causal(self, q, k, v, out, t_index, hkv, tk, q_offset=0,
                          stream=None):
        hq, tq, d = q.shape
        cap = k.shape[1]
        _need(q, torch.bfloat16, (hq, tq, d), "q")
        _need(out, torch.bfloat16, (hq, tq, d), "out")
        _need(k, torch.bfloat16, (hkv, cap, d), "k")
        _need(v, torch.bfloat16, (hkv, cap, d), "v")
        if t_index.dtype != torch.int32 or t_index.numel() < max(tk, q_offset + tq):
            raise ValueError("t_index: int32 covering max(tk, q_offset + tq)")
        st = self._lib.u15h_sdpa_block_causal(
            self._ctx, _stream(stream), _ptr(q), _ptr(k), _ptr(v), _ptr(out),
            _ptr(t_index), hq, hkv, tq, tk, d, cap, q_offset)
        self._check(st, "u15h_sdpa_block_causal")

    def attention_token_major(self, q, k, v, out, hq, hkv, tk, mode=0,
                              t_index=None, q_offset=0, stream=None):
        """q, out [tq][hq*d] token-major; mode 0/1/2 = bidirectional,
        causal, block-causal."""
        tq = q.shape[0]
        cap, d = k.shape[1], k.shape[2]
        _need(q, torch.bfloat16, (tq, hq * d), "q")
        _need(out, torch.bfloat16, (tq, hq * d), "out")
        _need(k, torch.bfloat16, (hkv, cap, d), "k")
        _need(v, torch.bfloat16, (hkv, cap, d), "v")
        st = self._lib.u15h_attention_token_major(
            self._ctx, _stream(stream), _ptr(q), _ptr(k), _ptr(v), _ptr(out),
            _ptr(t_index), hq, hkv, tq, tk, d, cap, q_offset, mode)
        self._check(st, "u15h_attention_token_major")

    def transpose_thd(self, x, out, T, H, D, stream=None):
        st = self._lib.u15h_transpose_thd(self._ctx, _stream(stream), _ptr(x),
                                          _ptr(out), T, H, D)
        self._check(st, "u15h_transpose_thd")

    def transpose_htd(self, x, out, T, H, D, stream=None):
        st = self._lib.u15h_transpose_htd(self._ctx, _stream(stream), _ptr(x),
                                          _ptr(out), T, H, D)
        self._check(st, "u15h_transpose_htd")

    def transpose_into_cache(self, x, cache, T, H, D, offset, stream=None):
        cap = cache.shape[1]
        st = self._lib.u15h_transpose_into_cache(self._ctx, _stream(stream),
                                                 _ptr(x), _ptr(cache), T, H, D,
                                                 cap, offset)
        self._check(st, "u15h_transpose_into_cache")

    # ---- routing -------------------------------------------------------
    def gather_rows(self, src, perm, dst, stream=None):
        M, cols = dst.shape
        _need(perm, torch.int32, (M,), "perm")
        st = self._lib.u15h_gather_rows(self._ctx, _stream(stream), _ptr(src),
                                        _ptr(perm), M, cols, _ptr(dst))
        self._check(st, "u15h_gather_rows")

    def scatter_rows(self, src, perm, dst, stream=None):
        M, cols = src.shape
        _need(perm, torch.int32, (M,), "perm")
        st = self._lib.u15h_scatter_rows(self._ctx, _stream(stream), _ptr(src),
                                         _ptr(perm), M, cols, _ptr(dst))
        self._check(st, "u15h_scatter_rows")

    # ---- the resident layer stack -----------------------------------------
    def stack_layer(self, stack, layer, io, M_und, M_gen, steps=STEP_ALL,
                    tier=TIER_BF16, flags=0, stream=None):
        """One layer's projection steps (u15h_stack_layer); `io` from
        layer_io()."""
        _check_io(stack, io, M_und + M_gen, steps, tier, flags)
        st = self._lib.u15h_stack_layer(self._ctx, _stream(stream), stack._h,
                                        layer, ctypes.byref(io), M_und, M_gen,
                                        steps, tier, flags)
        self._check(st, "u15h_stack_layer")

    def stack_forward(self, stack, io, M_und, M_gen, tier=TIER_BF16, flags=0,
                      stream=None):
        """Every layer's projection steps in order (u15h_stack_forward)."""
        _check_io(stack, io, M_und + M_gen, STEP_ALL, tier, flags)
        st = self._lib.u15h_stack_forward(self._ctx, _stream(stream), stack._h,
                                          ctypes.byref(io), M_und, M_gen, tier,
                                          flags)
        self._check(st, "u15h_stack_forward")

    # ---- raw access for tests of argument checking ----------------------
    @property
    def lib(self):
        return self._lib

    @property
    def ctx(self):
        return self._ctx
