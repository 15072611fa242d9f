"""GPU parity of the flash attention over the K/V cache.

Bar: the reference's bf16 bar, rel-L2 < 4e-3 (tests/u15-kernels-test.cc:55,
used by test_sdpa, test_block_causal and test_steel_attn), against the oracle
on the same bf16 inputs; the oracle is pinned bit-equal to the reference's
u15::ref::attention.  Outputs are compared head-major, as the reference
compares its SDPA kernels.
"""
import numpy as np
import pytest
import torch

import oracle
import u15h
from helpers import dev_bf16, host_f32, max_rel, rel_l2

pytestmark = pytest.mark.gpu

BAR = 4e-3


def widen(b):
    return oracle.bf16_to_f32(b)


def bf16_cache(kk, cap, fill=0.0):
    """A [hkv][cap][d] bf16 cache holding kk's keys; the slots past them
    hold `fill` (NaN exercises the rule that keys past tk are never read)."""
    hkv, tk, d = kk.shape
    c = np.full((hkv, cap, d), fill, np.float32)
    c[:, :tk] = kk
    return oracle.f32_to_bf16(c)


def run_sdpa(ops, qb, kb, vb, hkv, tk, causal=False, q_offset=0):
    q = dev_bf16(qb)
    out = torch.empty_like(q)
    ops.sdpa(q, dev_bf16(kb), dev_bf16(vb), out, hkv, tk, causal, q_offset)
    torch.cuda.synchronize()
    return host_f32(out)


@pytest.mark.parametrize("causal", [False, True])
def test_reference_sdpa_case(ops, causal):
    """test_sdpa (tests/u15-kernels-test.cc:510-600): hq=4, hkv=2, tq=tk=6,
    d=32, a cache of 10."""
    hq, hkv, tq, tk, d, cap = 4, 2, 6, 6, 32, 10
    qb = oracle.f32_to_bf16(oracle.randn_mt(61, hq * tq * d).reshape(hq, tq, d))
    kb = bf16_cache(oracle.randn_mt(62, hkv * tk * d).reshape(hkv, tk, d), cap)
    vb = bf16_cache(oracle.randn_mt(63, hkv * tk * d).reshape(hkv, tk, d), cap)
    got = run_sdpa(ops, qb, kb, vb, hkv, tk, causal)
    ref = oracle.attention(widen(qb), widen(kb), widen(vb), hkv, tk,
                           "causal" if causal else "bidirectional")
    assert rel_l2(got, ref) < BAR


def test_reference_block_causal_case(ops):
    """test_block_causal (tests/u15-kernels-test.cc:604-666): an
    edit-shaped prefix, 3 text tokens, a 6-token image block sharing one t,
    2 more text tokens; the plain causal answer must differ."""
    hq, hkv, d = 4, 2, 32
    t_idx = np.array([0, 1, 2, 3, 3, 3, 3, 3, 3, 4, 5], np.int32)
    T = t_idx.size
    cap = T + 4
    qb = oracle.f32_to_bf16(oracle.randn_mt(71, hq * T * d).reshape(hq, T, d))
    kb = bf16_cache(oracle.randn_mt(72, hkv * T * d).reshape(hkv, T, d), cap)
    vb = bf16_cache(oracle.randn_mt(73, hkv * T * d).reshape(hkv, T, d), cap)
    q = dev_bf16(qb)
    out = torch.empty_like(q)
    ops.sdpa_block_causal(q, dev_bf16(kb), dev_bf16(vb), out,
                          torch.from_numpy(t_idx).cuda(), hkv, T)
    torch.cuda.synchronize()
    got = host_f32(out)
    ref = oracle.attention(widen(qb), widen(kb), widen(vb), hkv, T,
                           "block_causal", t_idx)
    assert rel_l2(got, ref) < BAR
    causal = oracle.attention(widen(qb), widen(kb), widen(vb), hkv, T, "causal")
    assert rel_l2(got, causal) > 1e-2


def test_reference_steel_case_and_gqa_control(ops):
    """test_steel_attn (tests/u15-kernels-test.cc:738-826): head_dim 128,
    GQA 8/2, tq=48, tk=67, a cache of tk + 21.  The GQA group is load-
    bearing: the same queries against a cache whose heads are mapped one to
    one (a cache allocated with hq heads, so nothing is read out of range)
    give a different answer."""
    hq, hkv, tq, tk, d = 8, 2, 48, 67, 128
    cap = tk + 21
    qb = oracle.f32_to_bf16(oracle.randn_mt(81, hq * tq * d).reshape(hq, tq, d))
    kk = oracle.randn_mt(82, hkv * tk * d).reshape(hkv, tk, d)
    vv = oracle.randn_mt(83, hkv * tk * d).reshape(hkv, tk, d)
    kb, vb = bf16_cache(kk, cap), bf16_cache(vv, cap)
    got = run_sdpa(ops, qb, kb, vb, hkv, tk)
    ref = oracle.attention(widen(qb), widen(kb), widen(vb), hkv, tk)
    assert rel_l2(got, ref) < BAR
    assert max_rel(got, ref) <= 1e-2
    k8 = np.concatenate([kk, oracle.randn_mt(84, 6 * tk * d).reshape(6, tk, d)])
    v8 = np.concatenate([vv, oracle.randn_mt(85, 6 * tk * d).reshape(6, tk, d)])
    bad = run_sdpa(ops, qb, bf16_cache(k8, cap), bf16_cache(v8, cap), hq, tk)
    assert rel_l2(bad, ref) > 1e-2


def test_keys_past_tk_are_never_read(ops):
    """Cache slots past tk hold NaN; they must not reach the output."""
    hq, hkv, tq, tk, d = 8, 2, 100, 130, 128
    cap = 200
    rng = np.random.default_rng(0)
    qb = oracle.f32_to_bf16(rng.standard_normal((hq, tq, d)).astype(np.float32))
    kk = rng.standard_normal((hkv, tk, d)).astype(np.float32)
    vv = rng.standard_normal((hkv, tk, d)).astype(np.float32)
    kb, vb = bf16_cache(kk, cap, np.nan), bf16_cache(vv, cap, np.nan)
    got = run_sdpa(ops, qb, kb, vb, hkv, tk)
    assert np.all(np.isfinite(got))
    ref = oracle.attention(widen(qb), widen(bf16_cache(kk, cap)),
                           widen(bf16_cache(vv, cap)), hkv, tk)
    assert rel_l2(got, ref) < BAR


@pytest.mark.parametrize("mode", ["causal", "block_causal"])
def test_masked_with_query_offset(ops, mode):
    """Queries sitting at q_offset within the keys (a generation block after
    a frozen prefix), unaligned tq and tk."""
    hq, hkv, d = 8, 2, 128
    pre, tq = 70, 90
    tk = pre + tq
    cap = tk + 5
    rng = np.random.default_rng(7)
    qb = oracle.f32_to_bf16(rng.standard_normal((hq, tq, d)).astype(np.float32))
    kb = bf16_cache(rng.standard_normal((hkv, tk, d)).astype(np.float32), cap)
    vb = bf16_cache(rng.standard_normal((hkv, tk, d)).astype(np.float32), cap)
    t_idx = np.concatenate([np.arange(pre), np.full(tq, pre)]).astype(np.int32)
    q = dev_bf16(qb)
    out = torch.empty_like(q)
    if mode == "causal":
        ops.sdpa(q, dev_bf16(kb), dev_bf16(vb), out, hkv, tk, True, pre)
    else:
        ops.sdpa_block_causal(q, dev_bf16(kb), dev_bf16(vb), out,
                              torch.from_numpy(t_idx).cuda(), hkv, tk, pre)
    torch.cuda.synchronize()
    ref = oracle.attention(widen(qb), widen(kb), widen(vb), hkv, tk, mode,
                           t_idx, q_offset=pre)
    assert rel_l2(host_f32(out), ref) < BAR


@pytest.mark.parametrize("pre", [64, 70])
def test_block_causal_image_blocks(ops, pre):
    """Image blocks of 256 tokens after a text prefix, as in the generation
    pass: each 128-query workgroup lies in one block, so the tiles of its
    block past the causal frontier are wholly visible and skip the mask
    when all 64 of their keys carry the block's t (prefix 64: tiles align
    with the blocks); with prefix 70 the tiles straddle the prefix and the
    block boundaries and keep the mask.  Two blocks, so the second block's
    keys stay hidden from the first block's queries."""
    hq, hkv, d = 4, 2, 128
    tq = 512
    tk = pre + tq
    cap = tk + 3
    rng = np.random.default_rng(pre)
    qb = oracle.f32_to_bf16(rng.standard_normal((hq, tq, d)).astype(np.float32))
    kb = bf16_cache(rng.standard_normal((hkv, tk, d)).astype(np.float32), cap)
    vb = bf16_cache(rng.standard_normal((hkv, tk, d)).astype(np.float32), cap)
    t_idx = np.concatenate([np.arange(pre), pre + np.arange(tq) // 256]).astype(np.int32)
    q = dev_bf16(qb)
    out = torch.empty_like(q)
    ops.sdpa_block_causal(q, dev_bf16(kb), dev_bf16(vb), out,
                          torch.from_numpy(t_idx).cuda(), hkv, tk, pre)
    torch.cuda.synchronize()
    ref = oracle.attention(widen(qb), widen(kb), widen(vb), hkv, tk, "block_causal",
                           t_idx, q_offset=pre)
    causal = oracle.attention(widen(qb), widen(kb), widen(vb), hkv, tk, "causal",
                              t_idx, q_offset=pre)
    got = host_f32(out)
    assert rel_l2(got, ref) < BAR
    assert rel_l2(got, causal) > 1e-2          # the blocks are load-bearing


def test_model_shape_generation_pass(ops):
    """Config 2's generation pass: 32 query heads over 8 kv heads, 4096 gen
    queries against the 128-token frozen prefix plus themselves
    (tk = 4224), head_dim 128, cache capacity 4352; sampled queries
    against the oracle; the token-major entry point is bit-identical."""
    hq, hkv, d = 32, 8, 128
    tq, tk, cap = 4096, 4224, 4352
    g = torch.Generator(device="cuda").manual_seed(9)
    q = torch.randn(hq, tq, d, generator=g, device="cuda").to(torch.bfloat16)
    k = torch.randn(hkv, cap, d, generator=g, device="cuda").to(torch.bfloat16)
    v = torch.randn(hkv, cap, d, generator=g, device="cuda").to(torch.bfloat16)
    out = torch.empty_like(q)
    ops.sdpa(q, k, v, out, hkv, tk)
    qt = q.transpose(0, 1).contiguous().view(tq, hq * d)
    ot = torch.empty_like(qt)
    ops.attention_token_major(qt, k, v, ot, hq, hkv, tk)
    torch.cuda.synchronize()
    assert torch.equal(ot.view(tq, hq, d).transpose(0, 1).contiguous().view(torch.int16),
                       out.view(torch.int16))
    rows = np.array([0, 1, 31, 32, 127, 128, 2047, 4095])
    qs = host_f32(q)[:, rows]
    ref = oracle.attention(qs, host_f32(k), host_f32(v), hkv, tk)
    got = host_f32(out)[:, rows]
    assert rel_l2(got, ref) < BAR
    assert max_rel(got, ref) <= 1e-2


def test_transposes(ops):
    T, H, D, cap, off = 37, 8, 128, 64, 11
    rng = np.random.default_rng(1)
    xb = oracle.f32_to_bf16(rng.standard_normal((T, H * D)).astype(np.float32))
    x = dev_bf16(xb)
    hm = torch.empty(H, T, D, dtype=torch.bfloat16, device="cuda")
    ops.transpose_thd(x, hm, T, H, D)
    back = torch.empty_like(x)
    ops.transpose_htd(hm, back, T, H, D)
    cache = torch.zeros(H, cap, D, dtype=torch.bfloat16, device="cuda")
    ops.transpose_into_cache(x, cache, T, H, D, off)
    torch.cuda.synchronize()
    x3 = torch.from_numpy(xb.view(np.int16)).view(T, H, D)
    assert torch.equal(hm.cpu().view(torch.int16), x3.transpose(0, 1))
    assert torch.equal(back.view(torch.int16), x.view(torch.int16))
    c = cache.cpu().view(torch.int16)
    assert torch.equal(c[:, off:off + T], x3.transpose(0, 1))
    assert torch.all(c[:, :off] == 0) and torch.all(c[:, off + T:] == 0)
    with pytest.raises(u15h.U15hError):
        ops.transpose_into_cache(x, cache, T, H, D, cap - T + 1)


def test_attention_rejects_bad_shapes(ops):
    q = torch.zeros(4, 8, 128, dtype=torch.bfloat16, device="cuda")
    k = torch.zeros(2, 16, 128, dtype=torch.bfloat16, device="cuda")
    o = torch.empty_like(q)
    import ctypes
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    L, c = ops.lib, ops.ctx
    p = lambda t: ctypes.c_void_p(t.data_ptr())
    # tk > cap, hq % hkv, d = 96, block-causal without t_index
    assert L.u15h_sdpa(c, s, p(q), p(k), p(k), p(o), 4, 2, 8, 17, 128, 16, 0, 0) == u15h.EINVAL
    assert L.u15h_sdpa(c, s, p(q), p(k), p(k), p(o), 4, 3, 8, 8, 128, 16, 0, 0) == u15h.EINVAL
    assert L.u15h_sdpa(c, s, p(q), p(k), p(k), p(o), 4, 2, 8, 8, 96, 16, 0, 0) == u15h.EINVAL
    assert L.u15h_sdpa_block_causal(c, s, p(q), p(k), p(k), p(o), None, 4, 2,
                                    8, 8, 128, 16, 0) == u15h.EINVAL


@pytest.mark.parametrize("d", [32, 64, 128])
@pytest.mark.parametrize("mode", ["bidirectional", "causal", "block_causal"])
@pytest.mark.parametrize("tk", [1, 63, 64, 65, 128, 192, 257])
def test_tile_counts_head_dims_and_masks(ops, d, mode, tk):
    """Every head_dim the entry points accept, every mask, and key counts
    giving 1, 2, 3, 4 and 5 key tiles, partial and whole: the pipelined
    loop runs tiles in pairs and prefetches two ahead.  Queries are the
    last tq keys (q_offset = tk - tq), as in a generation block."""
    hq, hkv = 8, 2
    tq = min(tk, 70)
    pre = tk - tq
    cap = tk + 9
    rng = np.random.default_rng(d * 1000 + tk)
    qb = oracle.f32_to_bf16(rng.standard_normal((hq, tq, d)).astype(np.float32))
    kb = bf16_cache(rng.standard_normal((hkv, tk, d)).astype(np.float32), cap)
    vb = bf16_cache(rng.standard_normal((hkv, tk, d)).astype(np.float32), cap)
    # image-like blocks of 5 keys sharing a t, after a text prefix
    t_idx = np.concatenate([np.arange(pre), pre + np.arange(tq) // 5]).astype(np.int32)
    q = dev_bf16(qb)
    out = torch.empty_like(q)
    if mode == "block_causal":
        ops.sdpa_block_causal(q, dev_bf16(kb), dev_bf16(vb), out,
                              torch.from_numpy(t_idx).cuda(), hkv, tk, pre)
    else:
        ops.sdpa(q, dev_bf16(kb), dev_bf16(vb), out, hkv, tk, mode == "causal", pre)
    torch.cuda.synchronize()
    ref = oracle.attention(widen(qb), widen(kb), widen(vb), hkv, tk, mode,
                           t_idx, q_offset=pre)
    got = host_f32(out)
    assert np.all(np.isfinite(got))
    assert rel_l2(got, ref) < BAR
    assert max_rel(got, ref) <= 1e-2


@pytest.mark.parametrize("mode", [1, 2])
def test_token_major_masked_matches_head_major(ops, mode):
    """The token-major entry point runs the same kernel on other strides:
    bit-identical to the head-major result for the masked modes too."""
    hq, hkv, d, tq, tk = 16, 4, 128, 200, 330
    pre = tk - tq
    cap = tk + 3
    g = torch.Generator(device="cuda").manual_seed(mode)
    q = torch.randn(hq, tq, d, generator=g, device="cuda").to(torch.bfloat16)
    k = torch.randn(hkv, cap, d, generator=g, device="cuda").to(torch.bfloat16)
    v = torch.randn(hkv, cap, d, generator=g, device="cuda").to(torch.bfloat16)
    t_idx = torch.from_numpy(np.concatenate(
        [np.arange(pre), pre + np.arange(tq) // 16]).astype(np.int32)).cuda()
    out = torch.empty_like(q)
    if mode == 1:
        ops.sdpa(q, k, v, out, hkv, tk, True, pre)
    else:
        ops.sdpa_block_causal(q, k, v, out, t_idx, hkv, tk, pre)
    qt = q.transpose(0, 1).contiguous().view(tq, hq * d)
    ot = torch.empty_like(qt)
    ops.attention_token_major(qt, k, v, ot, hq, hkv, tk, t_index=t_idx,
                              q_offset=pre, mode=mode)
    torch.cuda.synchronize()
    assert torch.equal(ot.view(tq, hq, d).transpose(0, 1).contiguous().view(torch.int16),
                       out.view(torch.int16))
