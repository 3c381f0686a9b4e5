"""The ggml backend plugin boundary on the CPU (no GPU call): libggml-ameva.so loads into a ggml host, exports the
dynamic-loader entry points and the reference's ggml_backend_ameva_* API, fills the vtables in ggml 0.9.8's layout,
and its supports_op contract accepts exactly the nodes graph_compute can run (checked on hand-built tensors whose
buffers are plain host structs: the contract never touches device memory)."""
import ctypes
import re

import pytest

import ggml_plugin as gp  # noqa: E402


@pytest.fixture(scope="module")
def libs():
    return gp.load()


def test_struct_layouts_match_the_host(libs):
    host, _ = libs
    assert ctypes.sizeof(gp.Tensor) == 336 == host.ggml_testhost_tensor_size()
    assert ctypes.sizeof(gp.Cgraph) == host.ggml_testhost_cgraph_size()
    assert ctypes.sizeof(gp.BufferI) == 11 * 8 and ctypes.sizeof(gp.BackendI) == 16 * 8
    assert ctypes.sizeof(gp.DeviceI) == 15 * 8


def test_dl_entry_points_and_registry(libs):
    _, plugin = libs
    plugin.ggml_backend_score.restype = ctypes.c_int
    assert plugin.ggml_backend_score() == 100
    reg = ctypes.cast(plugin.ggml_backend_init(), ctypes.POINTER(gp.Reg)).contents
    assert reg.api_version == 2
    regp = plugin.ggml_backend_ameva_reg()
    assert reg.iface.get_name(regp) == b"AMEVA"
    assert reg.iface.get_device_count(regp) == 1
    assert not reg.iface.get_device(regp, 1)
    devp = reg.iface.get_device(regp, 0)
    dev = ctypes.cast(devp, ctypes.POINTER(gp.Device)).contents
    assert dev.iface.get_name(devp) == b"AMEVA0"
    assert b"MI355X" in dev.iface.get_description(devp)
    assert dev.iface.get_type(devp) == 1  # GPU
    buftp = dev.iface.get_buffer_type(devp)
    assert buftp == plugin.ggml_backend_ameva_buffer_type(0)
    assert not plugin.ggml_backend_ameva_buffer_type(1)
    assert dev.iface.supports_buft(devp, buftp)
    assert not dev.iface.supports_buft(devp, None)
    buft = ctypes.cast(buftp, ctypes.POINTER(gp.BufferType)).contents
    assert buft.iface.get_name(buftp) == b"AMEVA0"
    assert buft.iface.get_alignment(buftp) == 256
    assert not buft.iface.is_host(buftp)
    assert reg.iface.get_proc_address(regp, b"ggml_backend_ameva_profile_report")
    assert not plugin.ggml_backend_is_ameva(None)


def test_public_header_symbols_exported(libs):
    import os
    _, plugin = libs
    text = open(os.path.join(gp.ROOT, "include", "ggml-ameva.h")).read()
    names = re.findall(r"^\s*(?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\s*\**\s*(ggml_backend_[a-z0-9_]+)\s*\(", text, re.M)
    assert len(names) >= 30
    for n in names:
        assert hasattr(plugin, n), n


def test_conv_and_window_counters(libs):
    """The reference's convolution / group-norm / window counters (ggml-ameva.h:70-78) link and read as nothing run:
    its tests/ameva_window_check.cpp binds them."""
    _, plugin = libs
    for n in ("conv_count", "conv_bias_count", "group_norm_count", "window_node_count"):
        f = getattr(plugin, "ggml_backend_ameva_get_" + n)
        f.restype = ctypes.c_int64
        assert f() == 0, n
    plugin.ggml_backend_ameva_get_conv_f16_decoder.restype = ctypes.c_int
    assert plugin.ggml_backend_ameva_get_conv_f16_decoder() == -1


class FakeHost:
    """Tensors whose buffer struct names the AMEVA buffer type, with made-up aligned device addresses."""

    def __init__(self, plugin):
        self.plugin = plugin
        self.buf = gp.Buffer()
        self.buf.buft = plugin.ggml_backend_ameva_buffer_type(0)
        self.buf.usage = gp.USAGE_WEIGHTS
        self.foreign = gp.Buffer()
        self.keep = []
        self.addr = 1 << 32

    def t(self, typ, ne, foreign=False, nb=None):
        x = gp.Tensor()
        x.type = typ
        ne = list(ne) + [1] * (4 - len(ne))
        x.ne[:] = ne
        be, bb = gp.BLOCK[typ]
        if nb is None:
            nb = [bb, bb * (ne[0] // be)]
            nb += [nb[1] * ne[1], nb[1] * ne[1] * ne[2]]
        x.nb[:] = nb
        x.buffer = ctypes.addressof(self.foreign if foreign else self.buf)
        x.data = self.addr
        self.addr += 1 << 28
        self.keep.append(x)
        return x

    def node(self, op, typ, ne, srcs, params=()):
        x = self.t(typ, ne)
        x.op = op
        for i, s in enumerate(srcs):
            x.src[i] = ctypes.addressof(s) if s is not None else None
        for i, p in enumerate(params):
            x.op_params[i] = p if isinstance(p, int) else int(
                __import__("numpy").array([p], "float32").view("int32")[0])
        return x

    def reason(self, n):
        r = self.plugin.ggml_backend_ameva_op_unsupported_reason(ctypes.addressof(n))
        return None if r is None else r.decode()


def test_contract_accepts_the_hot_path_and_declines_the_rest(libs):
    _, plugin = libs
    h = FakeHost(plugin)
    x = h.t(gp.F32, [4096, 1])
    for wt in (gp.Q4_0, gp.Q8_0, gp.Q4_K, gp.Q6_K):
        w = h.t(wt, [4096, 14336])
        assert h.reason(h.node(gp.OP_MUL_MAT, gp.F32, [14336, 1], [w, x])) is None
    w16 = h.t(gp.F16, [4096, 64])
    assert "src0 type" in h.reason(h.node(gp.OP_MUL_MAT, gp.F32, [64, 1], [w16, x]))
    w3 = h.t(gp.Q4_0, [4096, 64, 2])
    assert "2-D" in h.reason(h.node(gp.OP_MUL_MAT, gp.F32, [64, 1, 2], [w3, x]))
    wf = h.t(gp.Q4_0, [4096, 64], foreign=True)
    assert "AMEVA buffer" in h.reason(h.node(gp.OP_MUL_MAT, gp.F32, [64, 1], [wf, x]))
    # RMS_NORM, ROPE, GLU, SET_ROWS, FA
    assert h.reason(h.node(gp.OP_RMS_NORM, gp.F32, [4096, 3], [h.t(gp.F32, [4096, 3])], [1e-5])) is None
    q = h.t(gp.F32, [128, 32, 1])
    pos = h.t(gp.I32, [1])
    assert h.reason(h.node(gp.OP_ROPE, gp.F32, [128, 32, 1], [q, pos], [0, 128, 0, 0, 0, 5e5, 1.0, 0.0, 1.0])) is None
    assert "YaRN" in h.reason(h.node(gp.OP_ROPE, gp.F32, [128, 32, 1], [q, pos], [0, 128, 0, 0, 0, 5e5, 1.0, 0.5, 1.0]))
    assert "mode" in h.reason(h.node(gp.OP_ROPE, gp.F32, [128, 32, 1], [q, pos], [0, 128, 8, 0, 0, 5e5, 1.0, 0.0]))
    g = h.t(gp.F32, [14336, 1])
    u = h.t(gp.F32, [14336, 1])
    assert h.reason(h.node(gp.OP_GLU, gp.F32, [14336, 1], [g, u], [gp.GLU_SWIGLU, 0])) is None
    assert "SWIGLU" in h.reason(h.node(gp.OP_GLU, gp.F32, [14336, 1], [g, u], [1, 0]))
    cache = h.t(gp.F16, [1024, 4096])
    kc = h.t(gp.F32, [1024, 1])
    idx = h.t(gp.I64, [1])
    assert h.reason(h.node(gp.OP_SET_ROWS, gp.F16, [1024, 4096], [kc, idx])) is None
    qf = h.t(gp.F32, [128, 1, 32], nb=[4, 128 * 32 * 4, 128 * 4, 128 * 32 * 4])
    k = h.t(gp.F16, [128, 4096, 8], nb=[2, 8 * 128 * 2, 128 * 2, 8 * 128 * 2 * 4096])
    v = h.t(gp.F16, [128, 4096, 8], nb=[2, 8 * 128 * 2, 128 * 2, 8 * 128 * 2 * 4096])
    mask = h.t(gp.F16, [4096, 1])
    fa = h.node(gp.OP_FLASH_ATTN_EXT, gp.F32, [128, 32, 1], [qf, k, v, mask], [0.088, 0.0, 0.0])
    assert h.reason(fa) is None
    k64 = h.t(gp.F16, [64, 4096, 8])
    assert "head size" in h.reason(h.node(gp.OP_FLASH_ATTN_EXT, gp.F32, [64, 32, 1], [h.t(gp.F32, [64, 1, 32]), k64, k64, None], [0.1, 0.0, 0.0]))
    assert "softcap" in h.reason(h.node(gp.OP_FLASH_ATTN_EXT, gp.F32, [128, 32, 1], [qf, k, v, mask], [0.088, 0.0, 30.0]))
    assert "not implemented" in h.reason(h.node(gp.OP_SOFT_MAX, gp.F32, [4096, 1], [x]))
    # views and reshapes are free
    assert h.reason(h.node(gp.OP_VIEW, gp.F32, [4096, 1], [x])) is None


def test_supports_op_is_the_contract_and_counts(libs):
    _, plugin = libs
    h = FakeHost(plugin)
    regp = plugin.ggml_backend_ameva_reg()
    reg = ctypes.cast(regp, ctypes.POINTER(gp.Reg)).contents
    devp = reg.iface.get_device(regp, 0)
    dev = ctypes.cast(devp, ctypes.POINTER(gp.Device)).contents
    plugin.ggml_backend_ameva_reset_counters()
    x = h.t(gp.F32, [4096, 1])
    ok = h.node(gp.OP_MUL_MAT, gp.F32, [64, 1], [h.t(gp.Q4_0, [4096, 64]), x])
    bad = h.node(gp.OP_MUL_MAT, gp.F32, [64, 1], [h.t(gp.F16, [4096, 64]), x])
    assert dev.iface.supports_op(devp, ctypes.addressof(ok))
    assert not dev.iface.supports_op(devp, ctypes.addressof(bad))
    assert gp.counter(plugin, "supports_query_count") == 2
    assert gp.counter(plugin, "supported_op_count") == 1
    assert dev.iface.offload_op(devp, ctypes.addressof(h.node(gp.OP_MUL_MAT, gp.F32, [64, 512], [h.t(gp.Q4_0, [4096, 64]), h.t(gp.F32, [4096, 512])])))
    assert not dev.iface.offload_op(devp, ctypes.addressof(ok))


def test_failure_injection_rejects_from_the_host(libs):
    _, plugin = libs
    h = FakeHost(plugin)
    n = h.node(gp.OP_RMS_NORM, gp.F32, [4096, 1], [h.t(gp.F32, [4096, 1])], [1e-5])
    assert h.reason(n) is None
    plugin.ggml_backend_ameva_set_failure_injection(10)  # AMEVA_FAIL_TENSOR_RANGE_OOB
    try:
        assert plugin.ggml_backend_ameva_get_failure_injection() == 10
        assert "failure injection" in h.reason(n)
    finally:
        plugin.ggml_backend_ameva_set_failure_injection(0)
    assert h.reason(n) is None


def test_host_abi_check_passes_on_a_matching_host(libs):
    """ggml_backend_init, ggml_backend_ameva_register and ggml_backend_ameva_init check the host's ggml ABI first
    (ameva_abi_check, ggml-ameva-device.cpp:415-495): on a host whose accessors read the plugin's structs as it lays
    them out, the check passes and the registry is returned."""
    _, plugin = libs
    plugin.ggml_backend_ameva_abi_check.restype = ctypes.c_char_p
    assert plugin.ggml_backend_ameva_abi_check() is None
    assert plugin.ggml_backend_init()


_SKEWED_LOAD = r"""
import ctypes, sys
host = ctypes.CDLL(sys.argv[1], mode=ctypes.RTLD_GLOBAL)
plugin = ctypes.CDLL(sys.argv[2])
plugin.ggml_backend_init.restype = ctypes.c_void_p
plugin.ggml_backend_ameva_abi_check.restype = ctypes.c_char_p
plugin.ggml_backend_ameva_reg.restype = ctypes.c_void_p
print("init", plugin.ggml_backend_init() or 0)
print("why", plugin.ggml_backend_ameva_abi_check().decode())
"""


@pytest.mark.parametrize("skew,what", [(1, "struct ggml_backend"), (2, "GGML_MAX_NAME")])
def test_host_abi_check_refuses_a_skewed_host(tmp_path, skew, what):
    """A host built from other ggml headers: one whose ggml_backend_i has one member fewer (it reads the device one
    slot early), and one built with GGML_MAX_NAME 128. ggml_backend_init returns NULL (llama.cpp's loader then reports
    the backend as failed) and the reason names the struct. Each host is loaded in a process of its own."""
    import subprocess
    import sys
    so = tmp_path / f"libggml_testhost_skew{skew}.so"
    subprocess.run(["gcc", "-O2", "-fPIC", "-shared", f"-DGGML_TESTHOST_SKEW={skew}", "-o", str(so), gp.HOST_SRC],
                   check=True)
    r = subprocess.run([sys.executable, "-c", _SKEWED_LOAD, str(so), gp.PLUGIN_LIB], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode == 0, r.stderr[-2000:]
    out = dict(line.split(" ", 1) for line in r.stdout.splitlines())
    assert out["init"] == "0"
    assert "ABI mismatch" in out["why"] and what in out["why"], out["why"]
    assert "refusing to load" in r.stderr
