"""CPU checks of the amuda / BitNet C ABI library (libamuda_hip.so, include/amuda_hip.h): it loads and exports every
function the header declares, its structs have the reference's layout (as ctypes sees it), ac_gguf_get_tensor_scale
reads the reference's own I2_S fixtures' scale trailers, and invalid arguments are refused before any GPU call."""
import ctypes
import glob
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLD = os.path.join(ROOT, "tests", "golden")
LIB = os.path.join(ROOT, "ameva_compute_amd", "libamuda_hip.so")


class AcContext(ctypes.Structure):
    _fields_ = [("driver_handle", ctypes.c_void_p), ("platform_id", ctypes.c_void_p), ("device_id", ctypes.c_void_p),
                ("context", ctypes.c_void_p), ("command_queue", ctypes.c_void_p),
                ("device_name", ctypes.c_char * 128), ("vendor_name", ctypes.c_char * 64),
                ("vendor_id", ctypes.c_uint32), ("max_compute_units", ctypes.c_uint32),
                ("max_work_group_size", ctypes.c_uint64), ("max_work_item_sizes", ctypes.c_uint64 * 3),
                ("global_mem_size", ctypes.c_uint64), ("local_mem_size", ctypes.c_uint64),
                ("active_quirks", ctypes.c_uint32), ("is_uma_supported", ctypes.c_bool)]


class AcBuffer(ctypes.Structure):
    _fields_ = [("host_ptr", ctypes.c_void_p), ("native_mem", ctypes.c_void_p), ("size_bytes", ctypes.c_size_t),
                ("flags", ctypes.c_uint32), ("is_mapped", ctypes.c_bool), ("is_user_allocated", ctypes.c_bool)]


class AcEvent(ctypes.Structure):
    _fields_ = [("native_event", ctypes.c_void_p), ("submit_time_ns", ctypes.c_uint64),
                ("start_time_ns", ctypes.c_uint64), ("end_time_ns", ctypes.c_uint64), ("duration_us", ctypes.c_uint64)]


class GgufTensor(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 64), ("n_dims", ctypes.c_uint32), ("ne", ctypes.c_uint64 * 4),
                ("type", ctypes.c_uint32), ("offset", ctypes.c_uint64), ("data_ptr", ctypes.c_void_p),
                ("size_bytes", ctypes.c_size_t), ("ac_buf", ctypes.c_void_p)]


def load():
    if not os.path.exists(LIB):
        pytest.skip("libamuda_hip.so not built")
    lib = ctypes.CDLL(LIB)
    lib.ac_gguf_get_tensor_scale.argtypes = [ctypes.POINTER(GgufTensor), ctypes.POINTER(ctypes.c_float)]
    lib.ac_gguf_get_tensor_scale.restype = ctypes.c_int
    lib.ac_ops_bitnet_gemv_i2_s_exact.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                                  ctypes.c_void_p, ctypes.c_float, ctypes.c_void_p,
                                                  ctypes.POINTER(ctypes.c_void_p)]
    lib.ac_ops_bitnet_gemv_i2_s_exact.restype = ctypes.c_int
    lib.bitnet_raw_vec_dot_i2_s.argtypes = [ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                            ctypes.c_int32, ctypes.c_int32]
    lib.bitnet_raw_vec_dot_i2_s.restype = None
    return lib


def test_exports_every_declared_function():
    lib = load()
    text = re.sub(r"/\*.*?\*/", "", open(os.path.join(ROOT, "include", "amuda_hip.h")).read(), flags=re.S)
    names = re.findall(r"^\s*(?:AcResult|void|uint64_t)\s+([a-z_0-9]+)\s*\(", text, re.M)
    assert len(names) == 13, names
    assert all(hasattr(lib, n) for n in names)


def test_struct_layouts():
    # the reference's legacy structs (include/ac_types.h:38-91, amuda_gguf.h:58-68) on LP64; the library pins the same
    # numbers with static_assert
    assert ctypes.sizeof(AcContext) == 296 and AcContext.vendor_id.offset == 232
    assert AcContext.is_uma_supported.offset == 292
    assert ctypes.sizeof(AcBuffer) == 32 and AcBuffer.is_user_allocated.offset == 29
    assert ctypes.sizeof(AcEvent) == 40
    assert ctypes.sizeof(GgufTensor) == 144 and GgufTensor.type.offset == 104 and GgufTensor.data_ptr.offset == 120


def tensor(data: np.ndarray, ne0: int, ne1: int, t: int = 36):
    g = GgufTensor()
    g.name = b"blk.0.attn_v.weight"
    g.n_dims = 2
    g.ne[0], g.ne[1] = ne0, ne1
    g.type = t
    g.data_ptr = data.ctypes.data
    g.size_bytes = data.nbytes
    return g


def test_tensor_scale_on_reference_fixtures():
    lib = load()
    out = ctypes.c_float()
    fx = np.fromfile(os.path.join(GOLD, "fixture_i2s_upstream.bin"), np.uint8)  # 256 weights + 32-byte trailer
    assert lib.ac_gguf_get_tensor_scale(ctypes.byref(tensor(fx, 128, 2)), ctypes.byref(out)) == 0
    assert out.value == 1.625
    sl = np.fromfile(os.path.join(GOLD, "gguf_slice_blk0_v.bin"), np.uint8)      # one 128-weight row + trailer
    assert lib.ac_gguf_get_tensor_scale(ctypes.byref(tensor(sl, 128, 1)), ctypes.byref(out)) == 0
    assert abs(out.value - 2.2931101322) < 1e-6
    # a trailer past the tensor's bytes is corrupt; F32 / F16 tensors have scale 1; other types are refused
    assert lib.ac_gguf_get_tensor_scale(ctypes.byref(tensor(fx[:66], 128, 2)), ctypes.byref(out)) == -304
    assert lib.ac_gguf_get_tensor_scale(ctypes.byref(tensor(fx, 16, 1, t=0)), ctypes.byref(out)) == 0
    assert out.value == 1.0
    assert lib.ac_gguf_get_tensor_scale(ctypes.byref(tensor(fx, 16, 1, t=2)), ctypes.byref(out)) == -104
    assert lib.ac_gguf_get_tensor_scale(None, ctypes.byref(out)) == -205


def test_argument_errors_before_any_gpu_call():
    lib = load()
    ev = ctypes.c_void_p(123)
    # null context / buffers: AC_ERR_NULL_POINTER, out_event cleared first (amuda_ops.c:308-311)
    assert lib.ac_ops_bitnet_gemv_i2_s_exact(None, 4, 128, None, None, 1.0, None, ctypes.byref(ev)) == -205
    assert ev.value is None
    dummy = AcBuffer()
    p = ctypes.cast(ctypes.pointer(dummy), ctypes.c_void_p)
    assert lib.ac_ops_bitnet_gemv_i2_s_exact(p, 4, 100, p, p, 1.0, p, None) == -303      # K % 128
    assert lib.ac_ops_bitnet_gemv_i2_s_exact(p, 0, 128, p, p, 1.0, p, None) == -303      # M <= 0
    assert lib.ac_ops_bitnet_gemv_i2_s_exact(p, 4, 128, p, p, 1.0, p, None) == -206      # buffers of 0 bytes
    # the raw dot returns without writing on invalid arguments (c_api.cpp:27)
    s = np.full(4, 7.0, np.float32)
    lib.bitnet_raw_vec_dot_i2_s(100, s.ctypes.data, s.ctypes.data, s.ctypes.data, 2, 0)
    lib.bitnet_raw_vec_dot_i2_s(128, s.ctypes.data, None, s.ctypes.data, 2, 0)
    lib.bitnet_raw_vec_dot_i2_s(128, s.ctypes.data, s.ctypes.data, s.ctypes.data, 0, 0)
    assert (s == 7.0).all()
