"""GGUF tensors to packed HBM weights on the GPU (mvlm_weight_from_gguf).

The GGUF dims are ne0 = K (contiguous) and ne1 = N; the packed weight must
hold exactly the tensor's values (bit for bit against the oracle's GGUF
dequantization for Q8_0/Q4_0, and the stored values for F32/F16/BF16), and a
GEMV through it must equal one through the same bytes packed directly.  The
reference's upload (moondream2.cpp:62-84) swapped rows and columns for F16
and could not consume quantized tensors at all."""
from __future__ import annotations

import numpy as np
import pytest

import mvlm_amd as m
from mvlm_amd import native
from gguf_writer import STRING, GGUFWriter

pytestmark = pytest.mark.gpu

GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q8_0, GGML_Q2_K, GGML_BF16 = 0, 1, 2, 8, 10, 30


@pytest.fixture(scope="module")
def gguf_file(tmp_path_factory, orc):
    N, K = 96, 256
    rng = np.random.default_rng(3)
    q8 = orc.q8_0_blocks(N * K // 32, 0x51)
    q4 = orc.q4_0_blocks(N * K // 32, 0x52)
    f16 = orc.normal_f16(N * K, 0x53, 0.02)
    f32 = rng.standard_normal(N * K).astype(np.float32)
    bf16 = (f32.view(np.uint32) >> 16).astype(np.uint16)          # any bf16 bit patterns
    w = GGUFWriter(alignment=64).add_kv("general.architecture", STRING, "phi2")
    w.add_tensor("blk.0.attn_qkv.weight", [K, N], GGML_Q8_0, q8.tobytes())
    w.add_tensor("blk.0.ffn_up.weight", [K, N], GGML_Q4_0, q4.tobytes())
    w.add_tensor("token_embd.weight", [K, N], GGML_F16, f16.tobytes())
    w.add_tensor("output.weight", [K, N], GGML_F32, f32.tobytes())
    w.add_tensor("vision.weight", [K, N], GGML_BF16, bf16.tobytes())
    w.add_tensor("output_norm.weight", [K], GGML_F32, f32[:K].tobytes())
    w.add_tensor("blk.0.ffn_down.weight", [256, 2], GGML_Q2_K, bytes(2 * 84))
    path = tmp_path_factory.mktemp("gguf") / "w.gguf"
    w.write(path)
    return str(path), N, K, {"q8": q8, "q4": q4, "f16": f16, "f32": f32, "bf16": bf16}


def test_quant_tensors_bit_exact(dev, orc, gguf_file):
    path, N, K, src = gguf_file
    with m.Gguf(path) as g:
        for name, qt, blocks, deq in (("blk.0.attn_qkv.weight", m.Q8_0, src["q8"], orc.dequant_q8_0),
                                      ("blk.0.ffn_up.weight", m.Q4_0, src["q4"], orc.dequant_q4_0)):
            W = dev.weight_from_gguf(g, g.find(name))
            assert W.shape == (N, K) and W.dtype == qt
            assert np.array_equal(W.dequant(), deq(blocks).reshape(N, K)), name
            # same GEMV result as the same bytes packed directly
            x = orc.normal_f32(K, 0x60)
            dx, y1, y2 = dev.upload(x), dev.alloc(N * 4), dev.alloc(N * 4)
            dev.gemv(dx, m.F32, W, y1, m.F32, N, K)
            dev.gemv(dx, m.F32, dev.pack(blocks, qt, N, K), y2, m.F32, N, K)
            assert np.array_equal(y1.download(np.float32), y2.download(np.float32))


def test_dense_tensors_exact(dev, orc, gguf_file):
    path, N, K, src = gguf_file
    with m.Gguf(path) as g:
        f16 = dev.weight_from_gguf(g, g.find("token_embd.weight")).dequant()
        assert np.array_equal(f16, src["f16"].view(np.float16).astype(np.float32).reshape(N, K))
        f32 = dev.weight_from_gguf(g, g.find("output.weight")).dequant()
        assert np.array_equal(f32, src["f32"].reshape(N, K))
        bf = dev.weight_from_gguf(g, g.find("vision.weight")).dequant()
        assert np.array_equal(bf.view(np.uint32), (src["bf16"].astype(np.uint32) << 16).reshape(N, K))


def test_unpackable_tensors(dev, gguf_file):
    path, _, _, _ = gguf_file
    with m.Gguf(path) as g:
        with pytest.raises(m.MvlmError) as e:
            dev.weight_from_gguf(g, g.find("output_norm.weight"))        # 1-D
        assert e.value.code == native.ERR_INVALID_ARG
        with pytest.raises(m.MvlmError) as e:
            dev.weight_from_gguf(g, g.find("blk.0.ffn_down.weight"))     # Q2_K
        assert e.value.code == native.ERR_UNSUPPORTED
