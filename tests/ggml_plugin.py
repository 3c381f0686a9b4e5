"""Test-side ggml host for libggml-ameva.so: ctypes mirrors of the ggml structs the plugin reads, the plugin's vtables,
and a small graph builder that lays out tensors in AMEVA buffers the way ggml-alloc does (contiguous, 256-aligned).

The host symbol the plugin needs (ggml_backend_buffer_init) comes from tests/ggml_host/libggml_testhost.so, loaded
with RTLD_GLOBAL first. Test infrastructure only (the reference drives its plugin through real ggml graphs in
tests/ameva_qmm_check.cpp; ggml itself is not in this image).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from ctypes import (CFUNCTYPE, POINTER, Structure, c_bool, c_char, c_char_p, c_float, c_int, c_int32, c_int64,
                    c_size_t, c_uint8, c_uint64, c_void_p)

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HOST_SRC = os.path.join(ROOT, "tests", "ggml_host", "ggml_testhost.c")
HOST_LIB = os.path.join(ROOT, "tests", "ggml_host", "libggml_testhost.so")
PLUGIN_LIB = os.path.join(ROOT, "ameva_compute_amd", "libggml-ameva.so")

# ggml enums (the plugin's ggml_abi.h)
F32, F16, Q4_0, Q8_0, Q4_K, Q6_K, I32, I64 = 0, 1, 2, 8, 12, 14, 26, 27
OP_NONE, OP_ADD, OP_MUL, OP_RMS_NORM, OP_MUL_MAT, OP_CPY = 0, 2, 7, 25, 29, 34
OP_RESHAPE, OP_VIEW, OP_PERMUTE, OP_GET_ROWS, OP_SET_ROWS = 36, 37, 38, 40, 42
OP_SOFT_MAX, OP_ROPE, OP_FLASH_ATTN_EXT, OP_GLU = 46, 48, 74, 96
GLU_SWIGLU = 2
USAGE_ANY, USAGE_WEIGHTS, USAGE_COMPUTE = 0, 1, 2
STATUS_SUCCESS, STATUS_FAILED = 0, -1
BLOCK = {F32: (1, 4), F16: (1, 2), Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210), I32: (1, 4),
         I64: (1, 8)}


class Tensor(Structure):
    _fields_ = [("type", c_int), ("buffer", c_void_p), ("ne", c_int64 * 4), ("nb", c_size_t * 4), ("op", c_int),
                ("op_params", c_int32 * 16), ("flags", c_int32), ("src", c_void_p * 10), ("view_src", c_void_p),
                ("view_offs", c_size_t), ("data", c_void_p), ("name", c_char * 64), ("extra", c_void_p),
                ("padding", c_char * 8)]


class HashSet(Structure):
    _fields_ = [("size", c_size_t), ("used", c_void_p), ("keys", c_void_p)]


class Cgraph(Structure):
    _fields_ = [("size", c_int), ("n_nodes", c_int), ("n_leafs", c_int), ("nodes", POINTER(c_void_p)),
                ("grads", c_void_p), ("grad_accs", c_void_p), ("leafs", c_void_p), ("use_counts", c_void_p),
                ("visited_hash_set", HashSet), ("order", c_int), ("uid", c_uint64)]


P = c_void_p


class BufferTypeI(Structure):
    _fields_ = [("get_name", CFUNCTYPE(c_char_p, P)), ("alloc_buffer", CFUNCTYPE(P, P, c_size_t)),
                ("get_alignment", CFUNCTYPE(c_size_t, P)), ("get_max_size", CFUNCTYPE(c_size_t, P)),
                ("get_alloc_size", CFUNCTYPE(c_size_t, P, P)), ("is_host", CFUNCTYPE(c_bool, P))]


class BufferType(Structure):
    _fields_ = [("iface", BufferTypeI), ("device", P), ("context", P)]


class BufferI(Structure):
    _fields_ = [("free_buffer", CFUNCTYPE(None, P)), ("get_base", CFUNCTYPE(P, P)),
                ("init_tensor", CFUNCTYPE(c_int, P, P)),
                ("memset_tensor", CFUNCTYPE(None, P, P, c_uint8, c_size_t, c_size_t)),
                ("set_tensor", CFUNCTYPE(None, P, P, P, c_size_t, c_size_t)),
                ("get_tensor", CFUNCTYPE(None, P, P, P, c_size_t, c_size_t)),
                ("set_tensor_2d", P), ("get_tensor_2d", P),
                ("cpy_tensor", CFUNCTYPE(c_bool, P, P, P)), ("clear", CFUNCTYPE(None, P, c_uint8)), ("reset", P)]


class Buffer(Structure):
    _fields_ = [("iface", BufferI), ("buft", P), ("context", P), ("size", c_size_t), ("usage", c_int)]


class BackendI(Structure):
    _fields_ = [("get_name", CFUNCTYPE(c_char_p, P)), ("free", CFUNCTYPE(None, P))] + \
               [(f"p{i}", P) for i in range(10)] + \
               [("graph_compute", CFUNCTYPE(c_int, P, P)), ("event_record", P), ("event_wait", P),
                ("graph_optimize", P)]


class Backend(Structure):
    _fields_ = [("guid", P), ("iface", BackendI), ("device", P), ("context", P)]


class DevCaps(Structure):
    _fields_ = [("async_", c_bool), ("host_buffer", c_bool), ("buffer_from_host_ptr", c_bool), ("events", c_bool)]


class DevProps(Structure):
    _fields_ = [("name", c_char_p), ("description", c_char_p), ("memory_free", c_size_t), ("memory_total", c_size_t),
                ("type", c_int), ("device_id", c_char_p), ("caps", DevCaps)]


class DeviceI(Structure):
    _fields_ = [("get_name", CFUNCTYPE(c_char_p, P)), ("get_description", CFUNCTYPE(c_char_p, P)),
                ("get_memory", CFUNCTYPE(None, P, POINTER(c_size_t), POINTER(c_size_t))),
                ("get_type", CFUNCTYPE(c_int, P)), ("get_props", CFUNCTYPE(None, P, POINTER(DevProps))),
                ("init_backend", CFUNCTYPE(P, P, c_char_p)), ("get_buffer_type", CFUNCTYPE(P, P)),
                ("get_host_buffer_type", P), ("buffer_from_host_ptr", P),
                ("supports_op", CFUNCTYPE(c_bool, P, P)), ("supports_buft", CFUNCTYPE(c_bool, P, P)),
                ("offload_op", CFUNCTYPE(c_bool, P, P)), ("event_new", P), ("event_free", P),
                ("event_synchronize", P)]


class Device(Structure):
    _fields_ = [("iface", DeviceI), ("reg", P), ("context", P)]


class RegI(Structure):
    _fields_ = [("get_name", CFUNCTYPE(c_char_p, P)), ("get_device_count", CFUNCTYPE(c_size_t, P)),
                ("get_device", CFUNCTYPE(P, P, c_size_t)), ("get_proc_address", CFUNCTYPE(P, P, c_char_p))]


class Reg(Structure):
    _fields_ = [("api_version", c_int), ("iface", RegI), ("context", P)]


def build_host() -> None:
    if not os.path.exists(HOST_LIB) or os.path.getmtime(HOST_LIB) < os.path.getmtime(HOST_SRC):
        subprocess.run(["gcc", "-O2", "-fPIC", "-shared", "-o", HOST_LIB, HOST_SRC], check=True)


_loaded = None


def load():
    """(host, plugin) CDLLs; the plugin's ggml_backend_buffer_init binds to the test host."""
    global _loaded
    if _loaded is None:
        build_host()
        host = ctypes.CDLL(HOST_LIB, mode=ctypes.RTLD_GLOBAL)
        host.ggml_backend_buffer_init.restype = P
        host.ggml_testhost_buffer_set_usage.argtypes = [P, c_int]
        host.ggml_testhost_buffer_free.argtypes = [P]
        host.ggml_testhost_tensor_size.restype = c_size_t
        host.ggml_testhost_cgraph_size.restype = c_size_t
        plugin = ctypes.CDLL(PLUGIN_LIB)
        plugin.ggml_backend_init.restype = P
        plugin.ggml_backend_ameva_reg.restype = P
        plugin.ggml_backend_ameva_init.restype = P
        plugin.ggml_backend_ameva_init.argtypes = [c_size_t]
        plugin.ggml_backend_ameva_buffer_type.restype = P
        plugin.ggml_backend_ameva_buffer_type.argtypes = [c_size_t]
        plugin.ggml_backend_is_ameva.argtypes = [P]
        plugin.ggml_backend_is_ameva.restype = c_bool
        plugin.ggml_backend_ameva_op_unsupported_reason.restype = c_char_p
        plugin.ggml_backend_ameva_op_unsupported_reason.argtypes = [P]
        plugin.ggml_backend_ameva_set_failure_injection.argtypes = [c_int]
        plugin.ggml_backend_ameva_get_failure_injection.restype = c_int
        plugin.ggml_backend_ameva_get_build_commit.restype = c_char_p
        for name in dir(plugin):
            pass
        _loaded = (host, plugin)
    return _loaded


def counter(plugin, name: str) -> int:
    fn = getattr(plugin, f"ggml_backend_ameva_get_{name}")
    fn.restype = c_int64
    return int(fn())


def row_bytes(t: int, n: int) -> int:
    be, bb = BLOCK[t]
    return n // be * bb


class Graph:
    """Tensors in two AMEVA buffers (a WEIGHTS buffer and a COMPUTE buffer) and the nodes of one graph."""

    def __init__(self, weight_bytes: int, compute_bytes: int):
        self.host, self.plugin = load()
        buft = self.plugin.ggml_backend_ameva_buffer_type(0)
        self.buft = ctypes.cast(buft, POINTER(BufferType)).contents
        self.bufs = {}
        self.cursor = {}
        for kind, size, usage in (("w", weight_bytes, USAGE_WEIGHTS), ("c", compute_bytes, USAGE_COMPUTE)):
            b = self.buft.iface.alloc_buffer(buft, max(size, 256))
            assert b, "alloc_buffer failed"
            self.host.ggml_testhost_buffer_set_usage(b, usage)
            self.bufs[kind] = b
            self.cursor[kind] = 0
        self.tensors = []  # keep the ctypes objects alive
        self.nodes = []
        be = self.plugin.ggml_backend_ameva_init(0)
        assert be
        self.backend = ctypes.cast(be, POINTER(Backend)).contents
        self.backend_ptr = be

    def buf(self, kind):
        return ctypes.cast(self.bufs[kind], POINTER(Buffer)).contents

    def base(self, kind) -> int:
        b = self.buf(kind)
        return b.iface.get_base(self.bufs[kind])

    def free(self):
        for b in self.bufs.values():
            self.host.ggml_testhost_buffer_free(b)
        self.bufs = {}
        if self.backend_ptr:
            self.backend.iface.free(self.backend_ptr)
            self.backend_ptr = None

    # ------------------------------------------------------------------------------------------ tensors
    def _new(self, t: int, ne, kind: str, name: str, data=None, nb=None) -> Tensor:
        ne = list(ne) + [1] * (4 - len(ne))
        x = Tensor()
        x.type = t
        x.ne[:] = ne
        be, bb = BLOCK[t]
        if nb is None:
            nb = [bb, bb * (ne[0] // be)]
            nb += [nb[1] * ne[1], nb[1] * ne[1] * ne[2]]
        x.nb[:] = nb
        x.name = name.encode()[:63]
        if data is None:
            size = nb[3] * ne[3]
            off = (self.cursor[kind] + 255) // 256 * 256
            assert off + size <= self.buf(kind).size, f"buffer {kind} too small"
            self.cursor[kind] = off + size
            x.data = self.base(kind) + off
            x.buffer = self.bufs[kind]
        else:
            x.data, x.buffer = data
        self.tensors.append(x)
        return x

    def tensor(self, t: int, ne, kind: str = "c", name: str = "t") -> Tensor:
        return self._new(t, ne, kind, name)

    def view(self, src: Tensor, t: int, ne, nb, offset: int, name: str = "view") -> Tensor:
        v = self._new(t, ne, "c", name, data=(src.data + offset, src.buffer), nb=list(nb))
        v.op = OP_VIEW
        v.view_src = ctypes.addressof(src)
        v.view_offs = offset
        v.src[0] = ctypes.addressof(src)
        return v

    def set(self, x: Tensor, arr: np.ndarray) -> None:
        a = np.ascontiguousarray(arr)
        buf = ctypes.cast(x.buffer, POINTER(Buffer)).contents
        buf.iface.set_tensor(x.buffer, ctypes.addressof(x), a.ctypes.data, 0, a.nbytes)

    def get(self, x: Tensor, dtype, shape=None) -> np.ndarray:
        n = x.nb[3] * x.ne[3]
        out = np.empty(n, np.uint8)
        buf = ctypes.cast(x.buffer, POINTER(Buffer)).contents
        buf.iface.get_tensor(x.buffer, ctypes.addressof(x), out.ctypes.data, 0, n)
        out = out.view(dtype)
        return out.reshape(shape) if shape is not None else out

    # ------------------------------------------------------------------------------------------ ops
    def _node(self, op: int, t: int, ne, srcs, name: str, params=()) -> Tensor:
        x = self.tensor(t, ne, "c", name)
        x.op = op
        for i, s in enumerate(srcs):
            x.src[i] = ctypes.addressof(s) if s is not None else None
        for i, p in enumerate(params):
            if isinstance(p, float):
                x.op_params[i] = np.array([p], np.float32).view(np.int32)[0]
            else:
                x.op_params[i] = p
        self.nodes.append(x)
        return x

    def mul_mat(self, w: Tensor, x: Tensor, name="mul_mat") -> Tensor:
        return self._node(OP_MUL_MAT, F32, [w.ne[1], x.ne[1], x.ne[2], x.ne[3]], [w, x], name)

    def rms_norm(self, x: Tensor, eps: float, name="norm") -> Tensor:
        return self._node(OP_RMS_NORM, F32, list(x.ne), [x], name, [eps])

    def mul(self, a: Tensor, b: Tensor, name="mul") -> Tensor:
        return self._node(OP_MUL, F32, list(a.ne), [a, b], name)

    def add(self, a: Tensor, b: Tensor, name="add") -> Tensor:
        return self._node(OP_ADD, F32, list(a.ne), [a, b], name)

    def reshape_3d(self, x: Tensor, ne0, ne1, ne2, name="reshape") -> Tensor:
        r = self._new(x.type, [ne0, ne1, ne2], "c", name, data=(x.data, x.buffer))
        r.op = OP_RESHAPE
        r.src[0] = ctypes.addressof(x)
        r.view_src = ctypes.addressof(x)
        self.nodes.append(r)
        return r

    def view_nd(self, x: Tensor, op: int, ne, nb, offset: int = 0, name="view") -> Tensor:
        """A VIEW / PERMUTE / RESHAPE node over x's memory with the given shape and strides."""
        v = self._new(x.type, list(ne), "c", name, data=(x.data + offset, x.buffer), nb=list(nb))
        v.op = op
        v.src[0] = ctypes.addressof(x)
        v.view_src = ctypes.addressof(x)
        v.view_offs = offset
        self.nodes.append(v)
        return v

    def rope(self, x: Tensor, pos: Tensor, n_dims: int, mode: int, base: float, name="rope") -> Tensor:
        # op_params: n_past, n_dims, mode, n_ctx, n_ctx_orig, freq_base, freq_scale, ext_factor, attn_factor,
        # beta_fast, beta_slow
        return self._node(OP_ROPE, F32, list(x.ne), [x, pos], name,
                          [0, n_dims, mode, 0, 0, base, 1.0, 0.0, 1.0, 32.0, 1.0])

    def flash_attn_ext(self, q: Tensor, k: Tensor, v: Tensor, mask: Tensor | None, scale: float,
                       name="fa") -> Tensor:
        # res [D, n_head, n_batch]
        return self._node(OP_FLASH_ATTN_EXT, F32, [v.ne[0], q.ne[2], q.ne[1], 1], [q, k, v, mask], name,
                          [scale, 0.0, 0.0])

    def swiglu(self, g: Tensor, u: Tensor, name="swiglu", swapped: bool = False) -> Tensor:
        """ggml_swiglu_split: silu(src0) * src1; swapped (op_params[1] = 1): silu(src1) * src0."""
        return self._node(OP_GLU, F32, list(g.ne), [g, u], name, [GLU_SWIGLU, 1 if swapped else 0])

    def set_rows(self, dst: Tensor, src: Tensor, idx: Tensor, name="set_rows") -> Tensor:
        x = self._new(dst.type, list(dst.ne), "c", name, data=(dst.data, dst.buffer), nb=list(dst.nb))
        x.op = OP_SET_ROWS
        x.src[0] = ctypes.addressof(src)
        x.src[1] = ctypes.addressof(idx)
        x.view_src = ctypes.addressof(dst)
        self.nodes.append(x)
        return x

    def get_rows(self, src: Tensor, idx: Tensor, name="get_rows") -> Tensor:
        return self._node(OP_GET_ROWS, F32, [src.ne[0], idx.ne[0]], [src, idx], name)

    # ------------------------------------------------------------------------------------------ compute
    def compute(self, nodes=None) -> int:
        nodes = self.nodes if nodes is None else nodes
        arr = (c_void_p * len(nodes))(*[ctypes.addressof(n) for n in nodes])
        g = Cgraph()
        g.size = len(nodes)
        g.n_nodes = len(nodes)
        g.nodes = ctypes.cast(arr, POINTER(c_void_p))
        self._keep = (arr, g)
        return self.backend.iface.graph_compute(self.backend_ptr, ctypes.addressof(g))

    def reason(self, node: Tensor):
        r = self.plugin.ggml_backend_ameva_op_unsupported_reason(ctypes.addressof(node))
        return None if r is None else r.decode()
