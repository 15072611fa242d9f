"""CPU-side checks of the C ABI: the library loads, exports exactly what
include/u15h.h declares, and its host-only logic behaves (no GPU calls)."""
import ctypes

import numpy as np
import pytest

import u15h


def test_library_exports_every_declared_symbol():
    lib = u15h.load_library()
    declared = u15h.declared_symbols()
    assert len(declared) >= 18
    missing = [s for s in declared if not hasattr(lib, s)]
    assert missing == []


def test_abi_version_and_status_strings():
    lib = u15h.load_library()
    assert lib.u15h_abi_version() == 1
    for st in range(5):
        assert lib.u15h_status_str(st)
    assert lib.u15h_status_str(99) == b"unknown status"


def test_null_context_is_rejected_without_a_device():
    lib = u15h.load_library()
    assert lib.u15h_linear(None, None, None, None, None, None, 1, 8, 8) == u15h.EINVAL
    assert lib.u15h_enable_i8_gemm(None, 1) == 0
    assert lib.u15h_last_error(None) == b"null context"
    lib.u15h_destroy(None)                 # no-op
    assert lib.u15h_create(0, None) == u15h.EINVAL


def test_create_refuses_without_gfx950():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present; covered by the GPU tests")
    lib = u15h.load_library()
    ctx = ctypes.c_void_p()
    assert lib.u15h_create(0, ctypes.byref(ctx)) == u15h.ENODEV
    assert not ctx.value


def test_route_rows_is_a_stable_partition():
    rng = np.random.default_rng(0)
    e = rng.integers(0, 2, 1000).astype(np.uint8)
    perm, mu, mg = u15h.route_rows(e)
    assert mu == int((e == 0).sum()) and mg == 1000 - mu
    assert np.array_equal(perm[:mu], np.flatnonzero(e == 0))
    assert np.array_equal(perm[mu:], np.flatnonzero(e == 1))
    assert sorted(perm.tolist()) == list(range(1000))


def test_route_rows_edge_cases():
    perm, mu, mg = u15h.route_rows([])
    assert (len(perm), mu, mg) == (0, 0, 0)
    perm, mu, mg = u15h.route_rows([1, 1, 1])
    assert (list(perm), mu, mg) == ([0, 1, 2], 0, 3)
    with pytest.raises(u15h.U15hError):
        u15h.route_rows([0, 2])


def test_build_rope_tables_matches_oracle():
    """u15h_build_rope_tables is host code (no device): bit-equal to the
    oracle's restatement of build_rope_tables, including long positions."""
    import numpy as np
    import oracle
    rng = np.random.default_rng(4)
    T, D = 50, 128
    pt = rng.integers(0, 20000, T)
    ph = rng.integers(0, 64, T)
    pw = rng.integers(0, 64, T)
    c, s = u15h.build_rope_tables(pt, ph, pw, D, 64, 32)
    oc, osn = oracle.rope_tables(pt, ph, pw, D, 64, 32)
    assert np.array_equal(c, oc) and np.array_equal(s, osn)
    with pytest.raises(u15h.U15hError):
        u15h.build_rope_tables(pt, ph, pw, D, 64, 30)   # 64 + 60 != 128
    c0, s0 = u15h.build_rope_tables([], [], [], D, 64, 32)
    assert c0.shape == (0, D)


def test_qweight_geometry_rule():
    """bind_matrix_'s shape rule (src/u15-weights.cc:247-325)."""
    assert u15h.qweight_geometry(4096, 64, 1024) == (8, 64)
    assert u15h.qweight_geometry(4096, 128, 512) == (4, 32)
    assert u15h.qweight_geometry(12288, 192, 3072) == (8, 64)
    for K, sc, cc in ((4096, 100, 1024), (4096, 64, 1000), (4096, 16, 1024),
                      (4096, 64, 2048), (4096, 0, 1024), (0, 64, 1024),
                      (4096, 128, 768)):
        with pytest.raises(u15h.U15hError):
            u15h.qweight_geometry(K, sc, cc)


# ---- the resident layer stack: host logic ---------------------------------

def test_weight_slot_reference_names():
    """Literal names from the reference's own tests and docs: the attention
    suffixes the tensor, the MLP the module (src/u15-weights.cc:539-578;
    tests/u15-weights-test.cc:200, tests/u15-config-test.cc:98;
    ARCHITECTURE.md:77-78)."""
    ws = u15h.weight_slot
    assert ws("language_model.model.layers.0.self_attn.q_proj_mot_gen.weight") == (0, u15h.GEN, 0)
    assert ws("language_model.model.layers.0.mlp_mot_gen.gate_proj.weight") == (0, u15h.GEN, 4)
    assert ws("language_model.model.layers.41.mlp.down_proj.weight") == (41, u15h.UND, 6)
    assert ws("language_model.model.layers.7.self_attn.o_proj") == (7, u15h.UND, 3)
    assert ws("language_model.model.layers.12.self_attn.v_proj_mot_gen") == (12, u15h.GEN, 2)
    assert ws("language_model.model.layers.5.mlp.up_proj") == (5, u15h.UND, 5)


@pytest.mark.parametrize("bad", [
    "language_model.model.layers.03.self_attn.q_proj",          # leading zero
    "language_model.model.layers.-1.self_attn.q_proj",
    "language_model.model.layers..mlp.up_proj",
    "language_model.model.layers.3.self_attn.q_norm.weight",    # a norm
    "language_model.model.layers.3.self_attn.q_norm_hw_mot_gen.weight",
    "language_model.model.layers.3.input_layernorm.weight",
    "language_model.model.layers.3.mlp.gate_proj_mot_gen",      # wrong suffix place
    "language_model.model.layers.3.self_attn_mot_gen.q_proj",   # wrong suffix place
    "language_model.model.layers.3.self_attn.q_proj.weightx",
    "language_model.model.layers.3.self_attn.q_proj.bias",
    "language_model.model.norm_mot_gen.weight",
    "model.layers.3.mlp.up_proj.weight",
    "language_model.model.layers.1234567890.mlp.up_proj",
    "",
])
def test_weight_slot_refuses_other_names(bad):
    with pytest.raises(u15h.U15hError):
        u15h.weight_slot(bad)


def test_weight_slot_round_trip_over_the_stack():
    for layer in (0, 1, 9, 10, 41):
        for e in (u15h.UND, u15h.GEN):
            for p in range(7):
                assert u15h.weight_slot(u15h.slot_name(layer, e, p)) == (layer, e, p)


def test_norm_slot_reference_names():
    """The layer binder's norm names (src/u15-weights.cc:549-566): the
    layernorms suffix the module, the head norms the tensor, and the _hw
    norms are not read as their shorter prefixes."""
    ns = u15h.norm_slot
    assert ns("language_model.model.layers.0.input_layernorm.weight") == (0, u15h.UND, 0)
    assert ns("language_model.model.layers.3.input_layernorm_mot_gen.weight") == (3, u15h.GEN, 0)
    assert ns("language_model.model.layers.41.post_attention_layernorm_mot_gen") == \
        (41, u15h.GEN, 1)
    assert ns("language_model.model.layers.2.self_attn.q_norm.weight") == (2, u15h.UND, 2)
    assert ns("language_model.model.layers.2.self_attn.k_norm_mot_gen.weight") == (2, u15h.GEN, 3)
    assert ns("language_model.model.layers.9.self_attn.q_norm_hw.weight") == (9, u15h.UND, 4)
    assert ns("language_model.model.layers.9.self_attn.k_norm_hw_mot_gen") == (9, u15h.GEN, 5)


@pytest.mark.parametrize("bad", [
    "language_model.model.layers.3.self_attn.q_proj.weight",        # a matrix
    "language_model.model.layers.3.self_attn.q_norm.bias",
    "language_model.model.layers.3.self_attn.q_norm_mot_gen_hw.weight",   # suffix order
    "language_model.model.layers.3.self_attn_mot_gen.q_norm.weight",
    "language_model.model.layers.3.input_layernorm.weightx",
    "language_model.model.layers.03.input_layernorm.weight",
    "language_model.model.norm.weight",
    "language_model.model.layers.3.mlp.input_layernorm.weight",
    "",
])
def test_norm_slot_refuses_other_names(bad):
    with pytest.raises(u15h.U15hError):
        u15h.norm_slot(bad)


def test_norm_slot_round_trip_and_weight_slot_keeps_refusing_norms():
    for layer in (0, 7, 41):
        for e in (u15h.UND, u15h.GEN):
            for w in range(6):
                name = u15h.norm_slot_name(layer, e, w)
                assert u15h.norm_slot(name) == (layer, e, w)
                with pytest.raises(u15h.U15hError):
                    u15h.weight_slot(name)


def test_stack_check_full_names_the_first_missing_norm():
    """With every matrix bound (fake aligned device addresses: the check
    reads pointers only), check_full names the first unbound norm."""
    lib = u15h.load_library()
    st = u15h.Stack(2)
    for layer in range(2):
        for e in (u15h.UND, u15h.GEN):
            for p_ in range(7):
                assert lib.u15h_stack_set(st._h, layer, e, p_, ctypes.c_void_p(4096),
                                          None, None) == u15h.OK
    assert st.check() is None
    assert st.check_full() == "language_model.model.layers.0.input_layernorm.weight"
    assert st.check_full(need_und=False) == \
        "language_model.model.layers.0.input_layernorm_mot_gen.weight"
    for layer in range(2):
        for w in range(6):
            assert lib.u15h_stack_set_norm(st._h, layer, u15h.UND, w,
                                           ctypes.c_void_p(8192)) == u15h.OK
    assert st.check_full(need_gen=False) is None
    assert st.check_full() == "language_model.model.layers.0.input_layernorm_mot_gen.weight"
    assert lib.u15h_stack_set_norm(st._h, 0, u15h.GEN, 6, ctypes.c_void_p(8192)) == u15h.EINVAL
    assert lib.u15h_stack_set_norm(st._h, 2, u15h.GEN, 0, ctypes.c_void_p(8192)) == u15h.EINVAL
    assert lib.u15h_stack_set_norm(st._h, 0, u15h.GEN, 0, ctypes.c_void_p(8)) == u15h.EINVAL
    io = u15h._LayerFullIO()
    assert lib.u15h_stack_layer_full(None, None, st._h, 0, ctypes.byref(io), 0, 1,
                                     0) == u15h.EINVAL
    st.close()


def test_stack_check_names_the_first_missing_matrix():
    st = u15h.Stack(3)
    assert st.check() == "language_model.model.layers.0.self_attn.q_proj.weight"
    assert st.check(need_und=False) == \
        "language_model.model.layers.0.self_attn.q_proj_mot_gen.weight"
    assert st.check(tier=u15h.TIER_I8).endswith("(int8)")
    assert st.check(need_und=False, need_gen=False) is None   # nothing needed
    st.close()


def test_stack_refusals_without_a_device():
    lib = u15h.load_library()
    h = ctypes.c_void_p()
    # shapes: heads must be a multiple of kv_heads, widths multiples of 8
    assert lib.u15h_stack_create(2, 4096, 32, 5, 128, 12288, ctypes.byref(h)) == u15h.EINVAL
    assert lib.u15h_stack_create(2, 4100, 32, 8, 128, 12288, ctypes.byref(h)) == u15h.EINVAL
    assert lib.u15h_stack_create(0, 4096, 32, 8, 128, 12288, ctypes.byref(h)) == u15h.EINVAL
    assert lib.u15h_stack_create(2, 4096, 32, 8, 128, 12288, ctypes.byref(h)) == u15h.OK
    # by index: layer, expert and projection ranges; a half-given int8 pair
    assert lib.u15h_stack_set(h, 2, 0, 0, None, None, None) == u15h.EINVAL
    assert lib.u15h_stack_set(h, 0, 2, 0, None, None, None) == u15h.EINVAL
    assert lib.u15h_stack_set(h, 0, 0, 7, None, None, None) == u15h.EINVAL
    assert lib.u15h_stack_set(h, 0, 0, 0, None, ctypes.c_void_p(256), None) == u15h.EINVAL
    assert lib.u15h_stack_set(h, 0, 0, 0, ctypes.c_void_p(8), None, None) == u15h.EINVAL
    # a name whose layer lies outside the stack
    assert lib.u15h_stack_bind(h, b"language_model.model.layers.2.mlp.up_proj",
                               ctypes.c_void_p(256)) == u15h.EINVAL
    # calls need a context
    io = u15h.layer_io()
    assert lib.u15h_stack_layer(None, None, h, 0, ctypes.byref(io), 0, 1, 15, 0, 0) == u15h.EINVAL
    assert lib.u15h_stack_forward(None, None, h, ctypes.byref(io), 0, 1, 0, 0) == u15h.EINVAL
    fio = u15h._LayerFullIO()
    caches = (ctypes.c_void_p * 2)()
    assert lib.u15h_stack_layer_full(None, None, h, 0, ctypes.byref(fio), 0, 1, 0) == u15h.EINVAL
    assert lib.u15h_stack_forward_full(None, None, h, 0, 2, ctypes.byref(fio), caches, caches,
                                       0, 1, 0) == u15h.EINVAL
    lib.u15h_stack_destroy(h)


def test_stack_check_refuses_int8_widths_past_the_gemm_limit():
    """An int8-tier pass over a stack whose widths exceed u15h_mot_gemm_i8's
    K limits is refused by the stack's own check, which the pass runs before
    its first launch (so no step's quantiser runs before a later step
    would refuse)."""
    big = u15h.Stack(1, hidden=4096, heads=32, kv_heads=8, head_dim=128,
                     inter=131072 + 128)
    assert "at most 131072" in big.check(tier=u15h.TIER_I8)
    # the bf16 tier has no such limit: it reports the first unbound matrix
    assert big.check().endswith("q_proj.weight")
    big.close()
    odd = u15h.Stack(1, hidden=4096 + 64, heads=32, kv_heads=8, head_dim=128,
                     inter=12288)
    assert "multiple of 128" in odd.check(tier=u15h.TIER_I8)
    odd.close()


def test_stack_io_is_checked_against_the_stack_before_the_call():
    """Ops.stack_layer / stack_forward check every io buffer the requested
    steps and tier use (the C ABI cannot see sizes): short, mistyped or
    missing buffers raise before anything is launched.  Host tensors of
    the right shapes pass the shape checks and stop at the device check."""
    import torch
    st = u15h.Stack(1, hidden=64, heads=2, kv_heads=1, head_dim=32, inter=128)
    M = 5

    def bufs(**over):
        b = dict(x=torch.zeros(M, 64, dtype=torch.bfloat16),
                 q=torch.zeros(M, 64, dtype=torch.bfloat16),
                 k=torch.zeros(M, 32, dtype=torch.bfloat16),
                 v=torch.zeros(M, 32, dtype=torch.bfloat16),
                 xq=torch.zeros(M, 128, dtype=torch.int8),
                 sx=torch.zeros(M, dtype=torch.float32))
        b.update(over)
        return {k: v for k, v in b.items() if v is not None}

    def check(steps=u15h.STEP_QKV, tier=u15h.TIER_BF16, **over):
        u15h._check_io(st, u15h.layer_io(**bufs(**over)), M, steps, tier, 0)

    with pytest.raises(ValueError, match="shape"):       # q one column short
        check(q=torch.zeros(M, 63, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="shape"):       # one row short
        check(k=torch.zeros(M - 1, 32, dtype=torch.bfloat16))
    with pytest.raises(TypeError):                       # f32 output
        check(v=torch.zeros(M, 32, dtype=torch.float32))
    with pytest.raises(ValueError, match="required"):    # missing output
        check(v=None)
    with pytest.raises(ValueError, match="required"):    # o step: no attn
        check(steps=u15h.STEP_O)
    with pytest.raises(ValueError, match="xq"):          # int8: xq too narrow
        check(tier=u15h.TIER_I8, xq=torch.zeros(M, 64, dtype=torch.int8))
    with pytest.raises(ValueError, match="GPU"):         # shapes right, host memory
        check()
    with pytest.raises(ValueError, match="unknown"):
        u15h.layer_io(xx=torch.zeros(1))
    # an io not made by layer_io carries no tensors to check
    with pytest.raises(ValueError, match="layer_io"):
        u15h._check_io(st, u15h._LayerIO(), M, u15h.STEP_QKV, u15h.TIER_BF16, 0)
    st.close()
