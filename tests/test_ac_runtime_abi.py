"""The ac_runtime C ABI of libac_runtime_hip.so without a GPU: the exported names against the reference's symbol list
(docs/abi/ac_runtime_symbols.txt, copied as tests/golden/ac_runtime_symbols.txt), the descriptor layouts of
include/ac_runtime_hip.h against the reference's layout record (docs/abi/ac_runtime_layout.txt, copied as
tests/golden/ac_runtime_layout.txt) as a C compiler sees them, the abi_version gate of the reference's
tests/ac_abi_check.c:80-101, out-pointer clearing and handle checks that fail before any device call, and the
generation-based error state (src/runtime/ac_error.cpp)."""
import ctypes
import os
import subprocess

import pytest

import ac_rt

HERE = os.path.dirname(os.path.abspath(__file__))
GOLDEN = os.path.join(HERE, "golden")

LAYOUT_C = r"""
#include <stddef.h>
#include <stdio.h>
#include "ac_runtime_hip.h"
#define SZ(T) printf("ABI_LAYOUT %s size %zu\n", #T, sizeof(T))
#define AT(T, f) printf("ABI_LAYOUT %s %s %zu\n", #T, #f, offsetof(T, f))
int main(void) {
    SZ(AcDim3); AT(AcDim3, x); AT(AcDim3, y); AT(AcDim3, z);
    SZ(AcSpecConstant); SZ(AcSpecConstantSchemaEntry); SZ(AcRuntimeBindingDesc); SZ(AcKernelRuntimeMetadata);
    SZ(AcContextDesc); AT(AcContextDesc, abi_version); AT(AcContextDesc, struct_size);
    AT(AcContextDesc, backend_kind); AT(AcContextDesc, flags);
    SZ(AcBufferDesc); AT(AcBufferDesc, abi_version); AT(AcBufferDesc, struct_size);
    SZ(AcKernelDesc); AT(AcKernelDesc, abi_version); AT(AcKernelDesc, struct_size);
    SZ(AcLaunchDesc); AT(AcLaunchDesc, abi_version); AT(AcLaunchDesc, struct_size);
    SZ(AcBatchDesc); AT(AcBatchDesc, abi_version); AT(AcBatchDesc, struct_size);
    SZ(AcBufferBinding);
    SZ(AcBatchStats); AT(AcBatchStats, abi_version); AT(AcBatchStats, struct_size);
    SZ(AcDeviceLimits); AT(AcDeviceLimits, abi_version); AT(AcDeviceLimits, struct_size);
    SZ(AcKernelSourceDesc); AT(AcKernelSourceDesc, abi_version); AT(AcKernelSourceDesc, struct_size);
    AT(AcKernelSourceDesc, source); AT(AcKernelSourceDesc, source_size); AT(AcKernelSourceDesc, build_options);
    AT(AcKernelSourceDesc, metadata); AT(AcKernelSourceDesc, flags);
    unsigned v[] = {0x00020100u, 0x00020200u, 0x00020300u, 0x00020400u, 0x00020000u, 0x00030000u, 0x00010100u,
                    0x00020301u, 0x99999999u};
    for (unsigned i = 0; i < sizeof(v) / sizeof(v[0]); ++i) printf("COMPAT %08X %d\n", v[i], AC_ABI_COMPATIBLE(v[i]) ? 1 : 0);
    return 0;
}
"""


@pytest.fixture(scope="module")
def rt():
    if not os.path.exists(ac_rt.LIB):
        pytest.fail("libac_runtime_hip.so is not built (run __graft_entry__.build())")
    return ac_rt.load()


@pytest.fixture(scope="module")
def layout(tmp_path_factory):
    d = tmp_path_factory.mktemp("layout")
    src = d / "layout.c"
    src.write_text(LAYOUT_C)
    exe = d / "layout"
    subprocess.run(["gcc", "-std=c11", "-Wall", "-I", os.path.join(ac_rt.ROOT, "include"), str(src), "-o", str(exe)],
                   check=True)
    return subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.splitlines()


def test_exports_the_reference_symbol_list(rt):
    want = sorted(open(os.path.join(GOLDEN, "ac_runtime_symbols.txt")).read().split())
    assert len(want) == 53
    assert ac_rt.names() == want
    out = subprocess.run(["nm", "-D", "--defined-only", ac_rt.LIB], check=True, capture_output=True, text=True).stdout
    got = sorted(line.split()[-1] for line in out.splitlines() if line.split()[-1].startswith("ac_runtime_"))
    assert got == want


def test_descriptor_layouts_match_the_reference(layout):
    want = open(os.path.join(GOLDEN, "ac_runtime_layout.txt")).read().splitlines()
    assert [l for l in layout if l.startswith("ABI_LAYOUT")] == want


def test_ctypes_mirror_matches_the_header(layout):
    size = {l.split()[1]: int(l.split()[3]) for l in layout if l.startswith("ABI_LAYOUT") and l.split()[2] == "size"}
    for name, cls in [("AcDim3", ac_rt.Dim3), ("AcKernelRuntimeMetadata", ac_rt.Metadata),
                      ("AcContextDesc", ac_rt.ContextDesc), ("AcBufferDesc", ac_rt.BufferDesc),
                      ("AcKernelDesc", ac_rt.KernelDesc), ("AcLaunchDesc", ac_rt.LaunchDesc),
                      ("AcBatchDesc", ac_rt.BatchDesc), ("AcBufferBinding", ac_rt.BufferBinding),
                      ("AcBatchStats", ac_rt.BatchStats), ("AcDeviceLimits", ac_rt.DeviceLimits),
                      ("AcKernelSourceDesc", ac_rt.KernelSourceDesc)]:
        assert ctypes.sizeof(cls) == size[name], name


def test_abi_version_gate(rt, layout):
    assert rt.ac_runtime_abi_version() == ac_rt.ABI
    compat = {l.split()[1]: l.split()[2] for l in layout if l.startswith("COMPAT")}
    assert compat == {"00020100": "1", "00020200": "1", "00020300": "1", "00020400": "0", "00020000": "0",
                      "00030000": "0", "00010100": "0", "00020301": "0", "99999999": "0"}
    # refused before any device call, with a cleared context (ac_abi_check.c:45-57)
    for v in (0x00020400, 0x00020000, 0x00030000, 0x00020301):
        ctx = ctypes.c_void_p(1)
        d = ac_rt.desc(ac_rt.ContextDesc, abi_version=v, backend_kind=ac_rt.BACKEND_VULKAN)
        assert rt.ac_runtime_context_create(ctypes.byref(d), ctypes.byref(ctx)) == ac_rt.E["INVALID_ARGUMENT"]
        assert ctx.value is None
    ctx = ctypes.c_void_p(1)
    d = ac_rt.desc(ac_rt.ContextDesc, backend_kind=ac_rt.BACKEND_HIP)
    d.struct_size = 12
    assert rt.ac_runtime_context_create(ctypes.byref(d), ctypes.byref(ctx)) == ac_rt.E["INVALID_ARGUMENT"]
    assert ctx.value is None
    d = ac_rt.desc(ac_rt.ContextDesc, backend_kind=ac_rt.BACKEND_HIP, flags=1)
    assert rt.ac_runtime_context_create(ctypes.byref(d), ctypes.byref(ctx)) == ac_rt.E["INVALID_ARGUMENT"]
    d = ac_rt.desc(ac_rt.ContextDesc, backend_kind=ac_rt.BACKEND_OPENCL)
    assert rt.ac_runtime_context_create(ctypes.byref(d), ctypes.byref(ctx)) == ac_rt.E["DRIVER_NOT_FOUND"]
    d = ac_rt.desc(ac_rt.ContextDesc, backend_kind=7)
    assert rt.ac_runtime_context_create(ctypes.byref(d), ctypes.byref(ctx)) == ac_rt.E["DEVICE_NOT_SUPPORTED"]
    assert ctx.value is None
    assert rt.ac_runtime_context_create(None, ctypes.byref(ctx)) == ac_rt.E["NULL_POINTER"]
    assert rt.ac_runtime_context_create(ctypes.byref(d), None) == ac_rt.E["NULL_POINTER"]


def test_null_handles(rt):
    E = ac_rt.E
    size = ctypes.c_size_t(5)
    assert rt.ac_runtime_buffer_get_size(None, ctypes.byref(size)) == E["INVALID_ARGUMENT"] and size.value == 0
    ptr = ctypes.c_void_p(1)
    assert rt.ac_runtime_buffer_get_mapped_ptr(None, ctypes.byref(ptr)) == E["INVALID_ARGUMENT"] and ptr.value is None
    assert rt.ac_runtime_buffer_destroy(None) == E["INVALID_ARGUMENT"]
    assert rt.ac_runtime_kernel_destroy(None) == E["INVALID_ARGUMENT"]
    assert rt.ac_runtime_kernel_get_push_constant_size(None, None) == E["NULL_POINTER"]
    assert rt.ac_runtime_kernel_get_push_constant_size(None, ctypes.byref(size)) == E["INVALID_ARGUMENT"]
    local = ac_rt.Dim3(1, 1, 1)
    assert rt.ac_runtime_kernel_get_effective_local_size(None, ctypes.byref(local)) == E["INVALID_ARGUMENT"]
    assert (local.x, local.y, local.z) == (0, 0, 0)
    buf = ctypes.create_string_buffer(65)
    buf.value = b"x"
    assert rt.ac_runtime_kernel_get_pipeline_identity(None, buf, 65) == E["INVALID_ARGUMENT"] and buf.value == b""
    assert rt.ac_runtime_event_wait(None, 0) == E["INVALID_ARGUMENT"]
    assert rt.ac_runtime_event_destroy(None) == E["INVALID_ARGUMENT"]
    assert rt.ac_runtime_context_destroy(None) == E["INVALID_CONTEXT"]
    kind = ctypes.c_uint32(9)
    assert rt.ac_runtime_context_get_backend_kind(None, ctypes.byref(kind)) == E["INVALID_CONTEXT"] and kind.value == 0
    b = ctypes.c_void_p(1)
    assert rt.ac_runtime_batch_begin(None, ctypes.byref(b)) == E["NULL_POINTER"] and b.value is None
    assert rt.ac_runtime_batch_submit(None, None) == E["INVALID_ARGUMENT"]
    assert rt.ac_runtime_batch_abort(None) == E["INVALID_ARGUMENT"]
    rt.ac_runtime_batch_destroy(None)
    n = ctypes.c_uint32(3)
    assert rt.ac_runtime_batch_get_dispatch_times(None, None, 0, ctypes.byref(n)) == E["INVALID_ARGUMENT"]
    assert n.value == 0


def test_error_state_generations(rt):
    rt.ac_runtime_reset_error_state()
    g0 = rt.ac_runtime_get_generation()
    assert g0 >= 1
    rt.ac_runtime_set_error(-206, 5, 64, 128, 96)  # AMEVA_BACKEND_OP_COPY_HTOD
    rt.ac_runtime_set_error(-202, 1, 0, 0, 0)      # a later error in the same generation does not replace it
    s = rt.ac_runtime_get_error_state()
    assert (s.generation, s.first_error, s.operation, s.offset, s.requested_bytes, s.capacity_bytes) == \
        (g0, -206, 5, 64, 128, 96)
    rt.ac_runtime_set_error(0, 1, 1, 1, 1)          # 0 is not an error
    assert rt.ac_runtime_consume_error() == -206
    assert rt.ac_runtime_consume_error() == 0
    rt.ac_runtime_set_error(-101, 7, 0, 0, 0)
    assert rt.ac_runtime_advance_generation() == g0 + 1
    s = rt.ac_runtime_get_error_state()
    assert s.generation == g0 + 1 and s.first_error == 0 and s.operation == 0
    # per-context states are independent, start at generation 1
    cid = 0xC0FFEE
    assert rt.ac_runtime_get_generation_ctx(cid) == 1
    rt.ac_runtime_set_error_ctx(cid, -407, 8, 1, 2, 3)
    assert rt.ac_runtime_get_error_state().first_error == 0
    assert rt.ac_runtime_get_error_state_ctx(cid).first_error == -407
    rt.ac_runtime_reset_error_state_ctx(cid)
    s = rt.ac_runtime_get_error_state_ctx(cid)
    assert s.first_error == 0 and s.generation == 1 and s.requested_bytes == 0
    assert rt.ac_runtime_advance_generation_ctx(cid) == 2
    assert rt.ac_runtime_consume_error_ctx(cid) == 0
