"""GPU checks of the on-disk formats that feed the kernels: the loader's
f16 -> bf16, safetensors tensors bound by dtype, quantized packs bound by
shape, and the affine-pack -> per-channel int8 repack.  All bit-exact
against the oracle."""
import numpy as np
import pytest
import torch

import oracle
import u15h
from helpers import dev_bf16, host_bits, host_f32, max_rel

pytestmark = pytest.mark.gpu


def test_f16_to_bf16_every_pattern(ops):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    src = torch.from_numpy(h.view(np.int16)).cuda()
    dst = torch.empty(65536, dtype=torch.bfloat16, device="cuda")
    ops.f16_to_bf16(src, dst)
    torch.cuda.synchronize()
    assert np.array_equal(host_bits(dst), oracle.f16_to_bf16(h))


@pytest.mark.parametrize("bits,group", [(8, 64), (4, 32)])
def test_repack_affine_i8_bit_exact(ops, bits, group):
    N, K = 520, 4096
    w = oracle.randn_mt(13 + bits, N * K, 0.05).reshape(N, K)
    codes, sc, bi, _ = oracle.pack_affine(w, bits, group)
    wd = oracle.dequant_affine(codes, sc, bi, bits, group, K)
    q_ref, s_ref = oracle.quant_rows_i8(wd)
    qw = (torch.from_numpy(codes.view(np.int32)).cuda(), dev_bf16(sc),
          dev_bf16(bi), bits, group)
    wq = torch.empty(N, K, dtype=torch.int8, device="cuda")
    sw = torch.empty(N, dtype=torch.float32, device="cuda")
    ops.repack_affine_i8(qw, N, K, wq, sw)
    torch.cuda.synchronize()
    assert np.array_equal(wq.cpu().numpy(), q_ref)
    assert np.array_equal(sw.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))


def test_repacked_int8_gemm_tracks_the_pack(ops):
    """The repacked weights drive the int8 GEMM; its result stays within the
    int8 tier's bar of the bf16 product on the pack's own meaning."""
    M, N, K = 256, 512, 4096
    w = oracle.randn_mt(21, N * K, 0.05).reshape(N, K)
    codes, sc, bi, _ = oracle.pack_affine(w, 8, 64)
    wd = oracle.dequant_affine(codes, sc, bi, 8, 64, K)
    qw = (torch.from_numpy(codes.view(np.int32)).cuda(), dev_bf16(sc),
          dev_bf16(bi), 8, 64)
    wq = torch.empty(N, K, dtype=torch.int8, device="cuda")
    sw = torch.empty(N, dtype=torch.float32, device="cuda")
    ops.repack_affine_i8(qw, N, K, wq, sw)
    xb = oracle.f32_to_bf16(oracle.randn_mt(22, M * K).reshape(M, K))
    x = dev_bf16(xb)
    xq = torch.empty(M, K, dtype=torch.int8, device="cuda")
    sx = torch.empty(M, dtype=torch.float32, device="cuda")
    ops.quant_rows_i8(x, xq, sx)
    y = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    ops.mot_gemm_i8(xq, sx, M, 0, K, [dict(wq_und=wq, sw_und=sw, y=y)])
    torch.cuda.synchronize()
    ref = oracle.linear_bf16(xb, wd)
    assert max_rel(host_f32(y), ref) <= 5e-2


def test_safetensors_bound_by_dtype(ops, tmp_path):
    """bind_bf16_ (src/u15-weights.cc:96-151): BF16 as it sits, F32 and F16
    converted with the loader's RNE."""
    from safetensors.torch import save_file
    rng = np.random.default_rng(0)
    a32 = rng.standard_normal((64, 96)).astype(np.float32)
    a16 = (rng.standard_normal((40, 24)) * 100).astype(np.float16)
    ab = torch.from_numpy(rng.standard_normal((8, 16)).astype(np.float32)).to(torch.bfloat16)
    path = tmp_path / "w.safetensors"
    save_file({"a.f32": torch.from_numpy(a32), "a.f16": torch.from_numpy(a16),
               "a.bf16": ab}, str(path))
    t = u15h.load_bf16(ops, path, "a.f32")
    assert np.array_equal(host_bits(t), oracle.f32_to_bf16(a32))
    t = u15h.load_bf16(ops, path, "a.f16")
    assert np.array_equal(host_bits(t), oracle.f16_to_bf16(a16.view(np.uint16)))
    t = u15h.load_bf16(ops, path, "a.bf16")
    assert torch.equal(t.cpu().view(torch.int16), ab.view(torch.int16))


def test_safetensors_matrix_dense_or_quantized(ops, tmp_path):
    """bind_matrix_ (src/u15-weights.cc:247-325): a `.scales` sibling makes
    `.weight` u32 codes; bits and group follow from the shapes; F16 scales
    and biases become bf16; the pack then runs through linear_q."""
    from safetensors.torch import save_file
    N, K = 256, 1024
    w = oracle.randn_mt(31, N * K, 0.05).reshape(N, K)
    codes, sc, bi, _ = oracle.pack_affine(w, 8, 64)
    sc16 = oracle.bf16_to_f32(sc).astype(np.float16)
    bi16 = oracle.bf16_to_f32(bi).astype(np.float16)
    dense = oracle.randn_mt(32, N * K, 0.05).reshape(N, K)
    path = tmp_path / "m.safetensors"
    save_file({"q_proj.weight": torch.from_numpy(codes.view(np.int32)),
               "q_proj.scales": torch.from_numpy(sc16),
               "q_proj.biases": torch.from_numpy(bi16),
               "o_proj.weight": torch.from_numpy(dense)}, str(path))
    kind, m = u15h.load_matrix(ops, path, "o_proj", K)
    assert kind == "dense"
    assert np.array_equal(host_bits(m), oracle.f32_to_bf16(dense))
    kind, qw = u15h.load_matrix(ops, path, "q_proj", K)
    assert kind == "affine" and qw[3:] == (8, 64)
    assert np.array_equal(host_bits(qw[1]), oracle.f16_to_bf16(sc16.view(np.uint16)))
    wd = torch.empty(N, K, dtype=torch.bfloat16, device="cuda")
    ops.dequant_affine(qw, N, K, wd)
    torch.cuda.synchronize()
    want = oracle.dequant_affine(codes, oracle.f16_to_bf16(sc16.view(np.uint16)),
                                 oracle.f16_to_bf16(bi16.view(np.uint16)), 8, 64, K)
    assert np.array_equal(host_bits(wd), want)
    with pytest.raises(u15h.U15hError):
        u15h.load_matrix(ops, path, "q_proj", K + 64)   # shapes do not close
