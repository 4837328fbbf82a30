"""The C ABI library, without a GPU: it loads, exports every symbol the header
declares, and its host-side argument checks fail with the documented codes."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
INCLUDE = os.path.join(ROOT, "include")


def declared_functions():
    names = set()
    for h in sorted(os.listdir(INCLUDE)):
        if h.endswith(".h"):
            text = re.sub(r"/\*.*?\*/", "", open(os.path.join(INCLUDE, h)).read(), flags=re.S)
            names.update(re.findall(r"\b(mvlm_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def test_header_declares_the_boundary():
    names = declared_functions()
    for must in ["mvlm_gemm_naive", "mvlm_gemm_tiled", "mvlm_gemm_packed", "mvlm_gemv", "mvlm_gemv_exact",
                 "mvlm_gemv_q8_0", "mvlm_gemv_q4_0", "mvlm_gemm_q8_0", "mvlm_gemm_q4_0",
                 "mvlm_gemm_batched", "mvlm_weight_pack", "mvlm_pool_init", "mvlm_device_create",
                 "mvlm_gguf_open", "mvlm_gguf_find_tensor", "mvlm_weight_from_gguf"]:
        assert must in names


def test_library_exports_every_declared_symbol():
    from mvlm_amd import native
    from mvlm_amd.build import exported_symbols
    lib = native.lib()
    exported = set(exported_symbols(native.LIB_PATH))
    for name in declared_functions():
        assert name in exported, name
        assert getattr(lib, name) is not None
        assert name in native._SIGNATURES, f"{name} has no ctypes signature"


def test_abi_version():
    from mvlm_amd import native
    assert native.lib().mvlm_abi_version() == 3


def test_device_count_without_gpu_is_not_an_error():
    from mvlm_amd import native
    assert native.device_count() >= 0


def test_device_create_reports_no_device():
    from mvlm_amd import native
    if native.device_count() > 0:
        pytest.skip("a GPU is visible; the no-device path is not reachable")
    with pytest.raises(native.MvlmError) as e:
        native.Device(0)
    assert e.value.code == native.ERR_NO_DEVICE
    assert "no HIP device" in native.last_error()


def test_null_arguments_are_rejected_on_the_host():
    from mvlm_amd import native
    L = native.lib()
    out = ctypes.c_void_p()
    assert L.mvlm_device_create(0, None) == native.ERR_INVALID_ARG
    assert L.mvlm_buffer_alloc(None, 16, ctypes.byref(out)) == native.ERR_INVALID_ARG
    assert L.mvlm_gemm_naive(None, None, None, None, 4, 4, 4, None) == native.ERR_INVALID_ARG
    assert L.mvlm_gemm_tiled(None, None, None, None, 4, 4, 4, None) == native.ERR_INVALID_ARG
    assert L.mvlm_gemv_exact(None, None, None, None, 4, 4, None) == native.ERR_INVALID_ARG
    assert L.mvlm_gemm_packed(None, None, 1, None, None, 0, 4, 4, 4, None) == native.ERR_INVALID_ARG
    assert L.mvlm_gemv(None, None, 0, None, None, 0, 4, 4, None) == native.ERR_INVALID_ARG
    assert L.mvlm_gemv_q8_0(None, None, None, None, 4, 32, None) == native.ERR_INVALID_ARG
    assert L.mvlm_gemm_q4_0(None, None, None, None, 2, 4, 32, None) == native.ERR_INVALID_ARG
    assert L.mvlm_gemm_batched(None, None, None, None, 1, 1, 1, 8, 8, 8, 1, 0, 0, 0, None) == native.ERR_INVALID_ARG
    assert L.mvlm_weight_pack(None, None, 8, 0, 4, 32, ctypes.byref(out)) == native.ERR_INVALID_ARG
    assert L.mvlm_pool_swap(None) == native.ERR_INVALID_ARG
    assert L.mvlm_event_release(None) == native.ERR_INVALID_ARG
    assert L.mvlm_pool_current(None) is None
    assert L.mvlm_buffer_size(None) == 0
    assert "null" in native.last_error()


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    """The binding raises when the HIP library is absent; nothing falls back."""
    from mvlm_amd import native
    monkeypatch.setattr(native, "_lib", None)
    monkeypatch.setattr(native, "LIB_PATH", str(tmp_path / "absent.so"))
    with pytest.raises(ImportError):
        native.lib()
