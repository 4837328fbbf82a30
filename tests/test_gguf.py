"""GGUF reader of the C library (include/mvlm_gguf.h), on the CPU.

Mirrors the reference's loader tests (tests/test_gguf.cpp:16-100: type and
block sizes, a missing file, the minimal file of tests/test_utils.h:100-113,
a bad magic) and adds what they leave open: metadata of every value type,
tensor infos and data at aligned offsets, general.alignment, and malformed
files (every truncation of a small file must be rejected, never crash)."""
from __future__ import annotations

import struct

import numpy as np
import pytest

import mvlm_amd as m
from mvlm_amd import native
from gguf_writer import (ARRAY, BOOL, FLOAT32, FLOAT64, INT32, INT64, STRING, UINT8, UINT16, UINT32, UINT64,
                         GGUFWriter)

GGML_F32, GGML_F16, GGML_Q4_0, GGML_Q8_0, GGML_Q2_K, GGML_BF16 = 0, 1, 2, 8, 10, 30


def status_of(fn, *a):
    with pytest.raises(m.MvlmError) as e:
        fn(*a)
    return e.value.code


def test_type_sizes_match_reference_tests():
    # test_gguf.cpp:16-34
    for t, size in ((0, 4), (1, 2), (2, 18), (8, 34), (24, 1), (25, 2), (26, 4)):
        assert m.ggml_type_size(t)[0] == size
    for t, block in ((0, 1), (1, 1), (2, 32), (8, 32), (10, 256), (24, 1)):
        assert m.ggml_type_size(t)[1] == block
    assert m.ggml_type_size(GGML_BF16) == (2, 1)
    assert status_of(m.ggml_type_size, 99) == native.ERR_NOT_FOUND


def test_missing_file(tmp_path):
    assert status_of(m.Gguf, str(tmp_path / "nonexistent.gguf")) == native.ERR_NOT_FOUND


def test_minimal_file(tmp_path):
    # the reference's create_test_gguf_file: v3, no tensors, no metadata, padding, 32 bytes
    p = tmp_path / "min.gguf"
    GGUFWriter().write(p, trailing=b"\0" * 32)
    with m.Gguf(str(p)) as g:
        info = g.info()
        assert (info.version, info.tensor_count, info.metadata_kv_count) == (3, 0, 0)
        assert info.alignment == 32 and info.data_offset == 32


def test_bad_magic(tmp_path):
    p = tmp_path / "bad.gguf"
    GGUFWriter().write(p, magic=b"GGUG", trailing=b"\0" * 32)
    assert status_of(m.Gguf, str(p)) == native.ERR_FORMAT


def test_unsupported_version(tmp_path):
    p = tmp_path / "v1.gguf"
    GGUFWriter(version=1).write(p, trailing=b"\0" * 32)
    assert status_of(m.Gguf, str(p)) == native.ERR_FORMAT


def test_metadata_values(tmp_path):
    p = tmp_path / "meta.gguf"
    w = GGUFWriter()
    tokens = ["a", "b", "ab", "c", "▁"]
    scores = [5.0, 4.0, 3.0, 2.0, 1.0]
    w.add_kv("tokenizer.ggml.tokens", ARRAY, (STRING, tokens))
    w.add_kv("tokenizer.ggml.scores", ARRAY, (FLOAT32, scores))
    w.add_kv("tokenizer.ggml.bos_token_id", UINT32, 1)
    w.add_kv("tokenizer.ggml.eos_token_id", INT32, 2)
    w.add_kv("general.name", STRING, "phi-1.5 test")
    w.add_kv("u8", UINT8, 7).add_kv("u16", UINT16, 65535).add_kv("u64", UINT64, 2 ** 40)
    w.add_kv("i64", INT64, -3).add_kv("f64", FLOAT64, 0.25).add_kv("flag", BOOL, True)
    w.add_kv("nested", ARRAY, (ARRAY, [(UINT32, [1, 2]), (UINT32, [3])]))
    w.add_kv("ids", ARRAY, (INT32, [-1, 0, 5]))
    w.write(p, trailing=b"\0" * 8)
    with m.Gguf(str(p)) as g:
        assert g.info().metadata_kv_count == 13
        assert g.get_array("tokenizer.ggml.tokens") == tokens
        assert g.get_array("tokenizer.ggml.scores").tolist() == scores
        assert g.get_u32("tokenizer.ggml.bos_token_id") == 1
        assert g.get_u32("tokenizer.ggml.eos_token_id") == 2      # INT32 accepted, like the reference
        assert g.get_string("general.name") == "phi-1.5 test"
        assert g.get_array("ids").tolist() == [-1, 0, 5]
        assert status_of(g.get_u32, "general.name") == native.ERR_INVALID_ARG
        assert status_of(g.get_u32, "no.such.key") == native.ERR_NOT_FOUND
        assert status_of(g.get_string, "u8") == native.ERR_INVALID_ARG


def _tensor_file(tmp_path, alignment=None, name="t.gguf"):
    rng = np.random.default_rng(7)
    K, N = 64, 3
    w = GGUFWriter(alignment=alignment)
    w.add_kv("general.architecture", STRING, "phi2")
    specs = [
        ("blk.0.attn_qkv.weight", [K, N], GGML_Q8_0, rng.integers(0, 256, N * K // 32 * 34, dtype=np.uint8).tobytes()),
        ("blk.0.ffn_up.weight", [K, N], GGML_Q4_0, rng.integers(0, 256, N * K // 32 * 18, dtype=np.uint8).tobytes()),
        ("token_embd.weight", [K, N], GGML_F16, rng.standard_normal(N * K).astype(np.float16).tobytes()),
        ("output_norm.weight", [K], GGML_F32, rng.standard_normal(K).astype(np.float32).tobytes()),
        ("blk.0.ffn_down.weight", [256, 2], GGML_Q2_K, rng.integers(0, 256, 2 * 84, dtype=np.uint8).tobytes()),
    ]
    for s in specs:
        w.add_tensor(*s)
    path = tmp_path / name
    blob = w.write(path)
    return path, specs, w, blob


@pytest.mark.parametrize("alignment", [None, 64, 256])
def test_tensor_infos_and_data(tmp_path, alignment):
    path, specs, w, _ = _tensor_file(tmp_path, alignment)
    align = alignment or 32
    with m.Gguf(str(path)) as g:
        info = g.info()
        assert info.tensor_count == len(specs) and info.alignment == align
        assert info.data_offset == w.data_offset and info.data_offset % align == 0
        for i, (name, dims, t, data) in enumerate(specs):
            ti = g.tensor(i)
            assert ti["name"] == name and ti["type"] == t and ti["n_dims"] == len(dims)
            assert ti["dims"][:len(dims)] == dims and all(d == 1 for d in ti["dims"][len(dims):])
            assert ti["offset"] % align == 0 and ti["bytes"] == len(data)
            assert g.data(i) == data
            assert g.find(name) == i
        assert status_of(g.find, "missing.weight") == native.ERR_NOT_FOUND


def test_every_truncation_is_rejected(tmp_path):
    path, _, _, blob = _tensor_file(tmp_path)
    cut = tmp_path / "cut.gguf"
    for n in range(0, len(blob), 7):
        cut.write_bytes(blob[:n])
        assert status_of(m.Gguf, str(cut)) == native.ERR_FORMAT, n


def test_malformed_tensor_infos(tmp_path):
    def one(dims, offset_shift=0, t=GGML_F32, data=b"\0" * 16, extra=b""):
        w = GGUFWriter().add_tensor("x", dims, t, data)
        b = bytearray(w.build())
        if offset_shift:   # rewrite the offset field: header, name "x", n_dims, dims, type, then offset
            pos = 24 + (8 + 1) + 4 + 8 * len(dims) + 4
            b[pos:pos + 8] = struct.pack("<Q", offset_shift)
        p = tmp_path / "x.gguf"
        p.write_bytes(bytes(b) + extra)
        return p
    assert status_of(m.Gguf, str(one([2, 2, 1, 1, 1]))) == native.ERR_FORMAT          # 5 dims
    assert status_of(m.Gguf, str(one([64], data=b"\0" * 16))) == native.ERR_FORMAT    # data past the end
    assert status_of(m.Gguf, str(one([4], offset_shift=8))) == native.ERR_FORMAT     # offset not aligned
    ok = one([4])
    with m.Gguf(str(ok)) as g:
        assert g.tensor(0)["bytes"] == 16


def test_implausible_counts(tmp_path):
    p = tmp_path / "count.gguf"
    GGUFWriter().write(p, tensor_count=2 ** 40, trailing=b"\0" * 32)
    assert status_of(m.Gguf, str(p)) == native.ERR_FORMAT


def test_bad_alignment(tmp_path):
    p = tmp_path / "align.gguf"
    GGUFWriter(alignment=48).write(p, trailing=b"\0" * 64)
    assert status_of(m.Gguf, str(p)) == native.ERR_FORMAT
