"""libac_runtime_hip.so on the GPU, the flows of the reference's runtime tests (tests/test_phase4_runtime_abi.cpp:
buffer contract, kernel creation, dispatch with and without an event, context isolation, destruction rules;
tests/test_batch_api_kat.cpp and test_batch_graph_kat.cpp: batches, hazard statistics, flush, dispatch times), with
AMDGPU code-object kernels (tests/ac_kernels/ac_test_kernels.hip) in place of SPIR-V: every result is checked against
numpy on the host, the pipeline identity against an independent hashlib computation of the reference's canonical
byte layout (src/runtime/ac_runtime.cpp:787-838)."""
import ctypes
import hashlib
import struct

import numpy as np
import pytest

import ac_rt

pytestmark = pytest.mark.gpu
E = ac_rt.E
OK = ac_rt.SUCCESS


@pytest.fixture(scope="module")
def rt():
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return ac_rt.load()


@pytest.fixture(scope="module")
def image():
    return open(ac_rt.KERNELS, "rb").read()


def new_ctx(rt, kind=ac_rt.BACKEND_HIP):
    ctx = ctypes.c_void_p()
    d = ac_rt.desc(ac_rt.ContextDesc, backend_kind=kind)
    assert rt.ac_runtime_context_create(ctypes.byref(d), ctypes.byref(ctx)) == OK
    return ctx


def new_buf(rt, ctx, nbytes, data=None):
    b = ctypes.c_void_p()
    d = ac_rt.desc(ac_rt.BufferDesc, size_bytes=nbytes, usage=ac_rt.USAGE_STORAGE | ac_rt.USAGE_DST)
    assert rt.ac_runtime_buffer_create(ctx, ctypes.byref(d), ctypes.byref(b)) == OK
    if data is not None:
        assert rt.ac_runtime_buffer_write(b, 0, data.ctypes.data, data.nbytes) == OK
    return b


def read(rt, b, n, dtype=np.float32, offset=0):
    out = np.empty(n, dtype)
    assert rt.ac_runtime_buffer_read(b, offset, out.ctypes.data, out.nbytes) == OK
    return out


class Kernel:
    """A kernel description kept alive with its metadata arrays."""

    def __init__(self, image, entry, nbind, push, local=(256, 1, 1), schemas=(), specs=(), sha=None):
        self.image = ctypes.create_string_buffer(image, len(image))
        self.binds = (ac_rt.BindingDesc * max(nbind, 1))(
            *[ac_rt.BindingDesc(i, 0, ac_rt.STAGE_COMPUTE) for i in range(nbind)])
        self.schemas = (ac_rt.SpecSchema * max(len(schemas), 1))(*schemas)
        self.specs = (ac_rt.SpecConstant * max(len(specs), 1))(*specs)
        self.sha = (sha or hashlib.sha256(image).hexdigest()).encode()
        self.meta = ac_rt.Metadata(kernel_name=entry.encode(), entry_point=entry.encode(), binding_count=nbind,
                                   bindings=self.binds, push_constant_size=push, local_size=ac_rt.Dim3(*local),
                                   expected_spirv_sha256=self.sha, specialization_schema_count=len(schemas),
                                   specialization_schemas=self.schemas)
        self.desc = ac_rt.desc(ac_rt.KernelDesc, spirv_code=ctypes.addressof(self.image), code_size_bytes=len(image),
                               metadata=ctypes.pointer(self.meta), specialization_count=len(specs),
                               specializations=self.specs)

    def create(self, rt, ctx):
        k = ctypes.c_void_p(1)
        r = rt.ac_runtime_kernel_create(ctx, ctypes.byref(self.desc), ctypes.byref(k))
        return r, k


def make(rt, ctx, image, *a, **kw):
    kd = Kernel(image, *a, **kw)
    r, k = kd.create(rt, ctx)
    assert r == OK, r
    return k


def launch(kernel, bufs, push, grid):
    arr = (ctypes.c_void_p * max(len(bufs), 1))(*[b.value for b in bufs])
    pc = ctypes.create_string_buffer(push, len(push)) if push else None
    d = ac_rt.desc(ac_rt.LaunchDesc, kernel=kernel.value, buffers=ctypes.cast(arr, ac_rt.PP), buffer_count=len(bufs),
                   push_constants=ctypes.addressof(pc) if pc else None, push_constants_size=len(push),
                   grid_dim=ac_rt.Dim3(*grid))
    d._keep = (arr, pc)
    return d


def test_context_limits_and_isolation(rt):
    ctx = new_ctx(rt, ac_rt.BACKEND_VULKAN)  # the reference's default request is served by the HIP backend
    kind = ctypes.c_uint32()
    assert rt.ac_runtime_context_get_backend_kind(ctx, ctypes.byref(kind)) == OK and kind.value == ac_rt.BACKEND_HIP
    name = ctypes.create_string_buffer(256)
    assert rt.ac_runtime_context_get_device_name(ctx, name, 256) == OK and b"gfx950" in name.value
    lim = ac_rt.desc(ac_rt.DeviceLimits)
    assert rt.ac_runtime_context_get_limits(ctx, ctypes.byref(lim)) == OK
    assert lim.subgroup_size == 64 and lim.max_compute_workgroup_invocations == 1024
    assert lim.max_push_constants_size == 128 and lim.timestamps_supported == 1
    assert lim.integer_dot_product == 1 and lim.max_memory_allocation_size > (200 << 30)
    old = ac_rt.desc(ac_rt.DeviceLimits, integer_dot_product=77, integer_dot_product_accelerated=77)
    old.struct_size = ac_rt.DeviceLimits.integer_dot_product.offset  # a caller of the first struct version
    assert rt.ac_runtime_context_get_limits(ctx, ctypes.byref(old)) == OK
    assert old.integer_dot_product == 77 and old.subgroup_size == 64
    bad = ac_rt.desc(ac_rt.DeviceLimits)
    bad.struct_size = 8
    assert rt.ac_runtime_context_get_limits(ctx, ctypes.byref(bad)) == E["INVALID_ARGUMENT"]
    # destruction refused while a child lives
    b = new_buf(rt, ctx, 64)
    assert rt.ac_runtime_context_destroy(ctx) == E["RESOURCE_IN_USE"]
    assert rt.ac_runtime_buffer_destroy(b) == OK
    assert rt.ac_runtime_context_destroy(ctx) == OK


def test_buffer_contract(rt):
    ctx = new_ctx(rt)
    b = ctypes.c_void_p(1)
    for kw, want in [(dict(size_bytes=0, usage=1), E["INVALID_BUFFER_SIZE"]),
                     (dict(size_bytes=64, usage=0), E["INVALID_ARGUMENT"]),
                     (dict(size_bytes=64, usage=16), E["INVALID_ARGUMENT"]),
                     (dict(size_bytes=64, usage=1, force_non_coherent=2), E["INVALID_ARGUMENT"])]:
        d = ac_rt.desc(ac_rt.BufferDesc, **kw)
        assert rt.ac_runtime_buffer_create(ctx, ctypes.byref(d), ctypes.byref(b)) == want and b.value is None
    n = 1000
    x = np.arange(n, dtype=np.float32)
    buf = new_buf(rt, ctx, x.nbytes, x)
    size, alloc = ctypes.c_size_t(), ctypes.c_size_t()
    assert rt.ac_runtime_buffer_get_size(buf, ctypes.byref(size)) == OK and size.value == 4000
    assert rt.ac_runtime_buffer_get_allocation_size(buf, ctypes.byref(alloc)) == OK and alloc.value == 4096
    assert np.array_equal(read(rt, buf, n), x)
    assert rt.ac_runtime_buffer_fill(buf, 8, 16, 0xFF) == OK
    got = read(rt, buf, n)
    assert np.all(np.isnan(got[2:6])) and np.array_equal(got[6:], x[6:]) and np.array_equal(got[:2], x[:2])
    tail = np.array([7.0, 8.0], np.float32)
    assert rt.ac_runtime_buffer_write(buf, 3992, tail.ctypes.data, 8) == OK
    assert np.array_equal(read(rt, buf, 2, offset=3992), tail)
    assert rt.ac_runtime_buffer_write(buf, 3996, tail.ctypes.data, 8) == E["INVALID_BUFFER_SIZE"]
    assert rt.ac_runtime_buffer_read(buf, 4001, tail.ctypes.data, 0) == E["INVALID_BUFFER_SIZE"]
    assert rt.ac_runtime_buffer_write(buf, 0, None, 4) == E["NULL_POINTER"]
    assert rt.ac_runtime_buffer_fill(buf, 4000, 1, 0) == E["INVALID_BUFFER_SIZE"]
    p = ctypes.c_void_p(1)
    assert rt.ac_runtime_buffer_get_mapped_ptr(buf, ctypes.byref(p)) == E["BUFFER_NOT_MAPPED"] and p.value is None
    coh = ctypes.c_uint32(5)
    assert rt.ac_runtime_buffer_is_coherent(buf, ctypes.byref(coh)) == E["BUFFER_NOT_MAPPED"] and coh.value == 0
    assert rt.ac_runtime_buffer_flush(buf, 0, 4) == E["BUFFER_NOT_MAPPED"]
    assert rt.ac_runtime_buffer_invalidate(buf, 0, 4) == E["BUFFER_NOT_MAPPED"]
    assert rt.ac_runtime_buffer_get_address(buf, ctypes.byref(p)) == OK and p.value
    assert rt.ac_runtime_buffer_destroy(buf) == OK
    assert rt.ac_runtime_buffer_destroy(buf) == E["INVALID_ARGUMENT"]  # the handle is gone
    assert rt.ac_runtime_context_destroy(ctx) == OK


def identity(image, entry, specs):
    h = hashlib.sha256()
    h.update(b"AMEVA-PIPELINE-ID\0")
    h.update(struct.pack("<I", 1))
    h.update(hashlib.sha256(image).digest())
    h.update(struct.pack("<I", len(entry)) + entry.encode())
    h.update(struct.pack("<I", len(specs)))
    for cid, typ, bits in sorted(specs):
        h.update(struct.pack("<III", cid, typ, bits))
    return h.hexdigest()


def f32bits(v):
    return struct.unpack("<I", struct.pack("<f", v))[0]


def test_kernel_creation_rules_and_identity(rt, image):
    ctx = new_ctx(rt)
    r, k = Kernel(image, "ac_axpy", 3, 8, sha="0" * 64).create(rt, ctx)
    assert r == E["BINARY_CORRUPTED"] and k.value is None
    spirv = struct.pack("<I", 0x07230203) + b"\0" * 60
    assert Kernel(spirv, "main", 0, 0).create(rt, ctx)[0] == E["FEATURE_NOT_SUPPORTED"]
    assert Kernel(b"\1\2\3\4" * 16, "main", 0, 0).create(rt, ctx)[0] == E["BINARY_CORRUPTED"]
    assert Kernel(image, "no_such_kernel", 0, 0).create(rt, ctx)[0] == E["KERNEL_NOT_FOUND"]
    assert Kernel(image, "ac_axpy", 3, 8, local=(0, 1, 1)).create(rt, ctx)[0] == E["INVALID_WORK_GROUP_SIZE"]
    assert Kernel(image, "ac_axpy", 3, 8, local=(2048, 1, 1)).create(rt, ctx)[0] == E["INVALID_WORK_GROUP_SIZE"]
    assert Kernel(image, "ac_axpy", 3, 200).create(rt, ctx)[0] == E["INVALID_ARGUMENT"]
    # an override of an undeclared constant, a schema default that disagrees with the local size
    und = Kernel(image, "ac_axpy", 3, 8, specs=[ac_rt.SpecConstant(9, ac_rt.SPEC_U32, 1)])
    assert und.create(rt, ctx)[0] == E["KERNEL_ARG_INVALID"]
    mis = Kernel(image, "ac_scale_spec", 2, 4, local=(128, 1, 1),
                 schemas=[ac_rt.SpecSchema(7, ac_rt.SPEC_U32, 64, 1, 1024, 1)])
    assert mis.create(rt, ctx)[0] == E["INVALID_ARGUMENT"]
    src = ac_rt.desc(ac_rt.KernelSourceDesc, source=b"__kernel void f() {}", metadata=ctypes.pointer(mis.meta))
    kk = ctypes.c_void_p(1)
    assert rt.ac_runtime_kernel_create_from_source(ctx, ctypes.byref(src), ctypes.byref(kk)) == \
        E["FEATURE_NOT_SUPPORTED"] and kk.value is None

    schemas = [ac_rt.SpecSchema(7, ac_rt.SPEC_U32, 256, 64, 1024, 1),
               ac_rt.SpecSchema(3, ac_rt.SPEC_F32, f32bits(1.0), f32bits(-8.0), f32bits(8.0), 0)]
    base = make(rt, ctx, image, "ac_scale_spec", 2, 4, schemas=schemas)
    over = make(rt, ctx, image, "ac_scale_spec", 2, 4, schemas=schemas,
                specs=[ac_rt.SpecConstant(3, ac_rt.SPEC_F32, f32bits(2.5)), ac_rt.SpecConstant(7, ac_rt.SPEC_U32, 128)])
    bad = Kernel(image, "ac_scale_spec", 2, 4, schemas=schemas,
                 specs=[ac_rt.SpecConstant(3, ac_rt.SPEC_F32, f32bits(9.0))])
    assert bad.create(rt, ctx)[0] == E["INVALID_ARGUMENT"]  # outside [min, max]
    hx = ctypes.create_string_buffer(65)
    assert rt.ac_runtime_kernel_get_pipeline_identity(base, hx, 64) == E["INVALID_ARGUMENT"]
    assert rt.ac_runtime_kernel_get_pipeline_identity(base, hx, 65) == OK
    assert hx.value.decode() == identity(image, "ac_scale_spec", [(3, 2, f32bits(1.0)), (7, 0, 256)])
    assert rt.ac_runtime_kernel_get_pipeline_identity(over, hx, 65) == OK
    assert hx.value.decode() == identity(image, "ac_scale_spec", [(3, 2, f32bits(2.5)), (7, 0, 128)])
    loc = ac_rt.Dim3()
    assert rt.ac_runtime_kernel_get_effective_local_size(over, ctypes.byref(loc)) == OK and loc.x == 128
    ps = ctypes.c_size_t()
    assert rt.ac_runtime_kernel_get_push_constant_size(over, ctypes.byref(ps)) == OK and ps.value == 4

    # the specialization values and the overridden local size reach the kernel
    n = 1000
    x = np.linspace(-3, 3, n).astype(np.float32)
    bx, by = new_buf(rt, ctx, x.nbytes, x), new_buf(rt, ctx, x.nbytes)
    for k, scale, lx in ((base, 1.0, 256), (over, 2.5, 128)):
        d = launch(k, [bx, by], struct.pack("<I", n), ((n + lx - 1) // lx, 1, 1))
        assert rt.ac_runtime_dispatch(ctx, ctypes.byref(d), None) == OK
        assert np.array_equal(read(rt, by, n), x * np.float32(scale) + np.float32(lx))
    for h in (bx, by):
        assert rt.ac_runtime_buffer_destroy(h) == OK
    assert rt.ac_runtime_context_destroy(ctx) == E["RESOURCE_IN_USE"]
    for k in (base, over):
        assert rt.ac_runtime_kernel_destroy(k) == OK
    assert rt.ac_runtime_context_destroy(ctx) == OK


def test_dispatch_events_and_errors(rt, image):
    ctx, other = new_ctx(rt), new_ctx(rt)
    k = make(rt, ctx, image, "ac_axpy", 3, 8)
    n = 100000
    rng = np.random.default_rng(1)
    x, y = rng.standard_normal(n).astype(np.float32), rng.standard_normal(n).astype(np.float32)
    bx, by, bo = new_buf(rt, ctx, x.nbytes, x), new_buf(rt, ctx, y.nbytes, y), new_buf(rt, ctx, x.nbytes)
    push = struct.pack("<If", n, 0.5)
    grid = ((n + 255) // 256, 1, 1)
    d = launch(k, [bx, by, bo], push, grid)
    ev = ctypes.c_void_p()
    assert rt.ac_runtime_dispatch(ctx, ctypes.byref(d), ctypes.byref(ev)) == OK and ev.value
    assert rt.ac_runtime_event_wait(ev, 5_000_000_000) == OK
    assert rt.ac_runtime_event_wait(ev, 0) == OK  # idempotent
    wall, gpu = ctypes.c_uint64(), ctypes.c_uint64()
    assert rt.ac_runtime_event_get_timing(ev, ctypes.byref(wall), ctypes.byref(gpu)) == OK
    assert 0 < gpu.value < 1_000_000_000 and wall.value > 0
    assert np.array_equal(read(rt, bo, n), np.float32(0.5) * x + y)
    assert rt.ac_runtime_context_destroy(ctx) == E["RESOURCE_IN_USE"]  # the event is a child
    assert rt.ac_runtime_event_destroy(ev) == OK
    # errors of the launch descriptor
    for bufs, p, g, want in [([bx, by], push, grid, E["KERNEL_ARG_INVALID"]),
                             ([bx, by, bo], push + b"\0" * 4, grid, E["KERNEL_ARG_INVALID"]),
                             ([bx, by, bo], push, (0, 1, 1), E["INVALID_WORK_GROUP_SIZE"]),
                             ([bx, by, bo], push, (1 << 21, 1, 1), E["INVALID_WORK_GROUP_SIZE"]),
                             ([bx, by, bo], push, (4096, 4096, 2), E["INVALID_WORK_GROUP_SIZE"])]:
        dd = launch(k, bufs, p, g)
        ev = ctypes.c_void_p(1)
        assert rt.ac_runtime_dispatch(ctx, ctypes.byref(dd), ctypes.byref(ev)) == want and ev.value is None
    ob = new_buf(rt, other, x.nbytes)
    assert rt.ac_runtime_dispatch(other, ctypes.byref(d), None) == E["CONTEXT_MISMATCH"]
    dd = launch(k, [bx, by, ob], push, grid)
    assert rt.ac_runtime_dispatch(ctx, ctypes.byref(dd), None) == E["CONTEXT_MISMATCH"]
    d.abi_version = 0x00030000
    assert rt.ac_runtime_dispatch(ctx, ctypes.byref(d), None) == E["INVALID_ARGUMENT"]
    for h in (bx, by, bo):
        assert rt.ac_runtime_buffer_destroy(h) == OK
    assert rt.ac_runtime_buffer_destroy(ob) == OK
    assert rt.ac_runtime_kernel_destroy(k) == OK
    assert rt.ac_runtime_context_destroy(ctx) == OK
    assert rt.ac_runtime_context_destroy(other) == OK


def test_batch_hazards_flush_and_dispatch_times(rt, image):
    ctx = new_ctx(rt)
    k = make(rt, ctx, image, "ac_add_one", 2, 4)
    n = 4096
    a = np.arange(n, dtype=np.float32)
    A, B, C, D = new_buf(rt, ctx, a.nbytes, a), new_buf(rt, ctx, a.nbytes), new_buf(rt, ctx, a.nbytes), \
        new_buf(rt, ctx, a.nbytes)
    bd = ac_rt.desc(ac_rt.BatchDesc, max_dispatches=3, flags=ac_rt.FLAG_TIMESTAMPS | ac_rt.FLAG_DISPATCH_TIMESTAMPS)
    bt = ctypes.c_void_p()
    assert rt.ac_runtime_batch_begin_ex(ctx, ctypes.byref(bd), ctypes.byref(bt)) == OK
    push, grid = struct.pack("<I", n), (n // 256, 1, 1)
    d1, d2, d3 = launch(k, [A, B], push, grid), launch(k, [B, C], push, grid), launch(k, [A, D], push, grid)
    ev1 = ctypes.c_void_p()
    assert rt.ac_runtime_batch_dispatch(bt, k, ctypes.byref(d1), ctypes.byref(ev1)) == OK
    assert rt.ac_runtime_event_wait(ev1, 0) == E["INVALID_ARGUMENT"]  # not issued yet
    assert rt.ac_runtime_batch_flush(bt) == OK
    assert rt.ac_runtime_batch_flush(bt) == OK  # nothing new: a no-op
    assert rt.ac_runtime_batch_dispatch(bt, k, ctypes.byref(d2), None) == OK
    assert rt.ac_runtime_batch_dispatch(bt, k, ctypes.byref(d3), None) == OK
    assert rt.ac_runtime_batch_dispatch(bt, k, ctypes.byref(d3), None) == E["DEVICE_BUSY"]  # capacity 3
    done = ctypes.c_void_p()
    assert rt.ac_runtime_batch_submit(bt, ctypes.byref(done)) == OK
    assert rt.ac_runtime_batch_submit(bt, None) == E["INVALID_ARGUMENT"]
    assert rt.ac_runtime_batch_abort(bt) == E["INVALID_ARGUMENT"]
    assert rt.ac_runtime_event_wait(done, 5_000_000_000) == OK
    assert rt.ac_runtime_event_wait(ev1, 5_000_000_000) == OK
    assert np.array_equal(read(rt, B, n), a + 1) and np.array_equal(read(rt, C, n), a + 2)
    assert np.array_equal(read(rt, D, n), a + 1)
    st = ac_rt.desc(ac_rt.BatchStats)
    assert rt.ac_runtime_batch_get_stats(bt, ctypes.byref(st)) == OK
    # A->B elided (nothing before it), B->C reads what B was written: a barrier, A->D touches neither
    assert (st.dispatches, st.barriers, st.elided_barriers, st.flushes) == (3, 1, 2, 1)
    times = (ctypes.c_uint64 * 3)()
    cnt = ctypes.c_uint32()
    assert rt.ac_runtime_batch_get_dispatch_times(bt, times, 2, ctypes.byref(cnt)) == E["INVALID_ARGUMENT"]
    assert rt.ac_runtime_batch_get_dispatch_times(bt, times, 3, ctypes.byref(cnt)) == OK and cnt.value == 3
    wall, gpu = ctypes.c_uint64(), ctypes.c_uint64()
    assert rt.ac_runtime_event_get_timing(done, ctypes.byref(wall), ctypes.byref(gpu)) == OK
    assert all(t > 0 for t in times) and sum(times) <= gpu.value + 1000
    rt.ac_runtime_batch_destroy(bt)
    for e in (ev1, done):  # the events outlive their batch
        assert rt.ac_runtime_event_destroy(e) == OK

    # explicit barriers: counted as recorded, nothing elided; legacy begin holds 8 dispatches
    bd = ac_rt.desc(ac_rt.BatchDesc, max_dispatches=4, flags=ac_rt.FLAG_EXPLICIT)
    assert rt.ac_runtime_batch_begin_ex(ctx, ctypes.byref(bd), ctypes.byref(bt)) == OK
    assert rt.ac_runtime_batch_dispatch(bt, k, ctypes.byref(d1), None) == OK
    assert rt.ac_runtime_batch_barrier(bt) == OK
    assert rt.ac_runtime_batch_dispatch(bt, k, ctypes.byref(d2), None) == OK
    assert rt.ac_runtime_batch_submit(bt, None) == OK
    assert rt.ac_runtime_batch_get_stats(bt, ctypes.byref(st)) == OK
    assert (st.dispatches, st.barriers, st.elided_barriers) == (2, 1, 0)
    times = (ctypes.c_uint64 * 2)()
    assert rt.ac_runtime_batch_get_dispatch_times(bt, times, 2, ctypes.byref(cnt)) == E["FEATURE_NOT_SUPPORTED"]
    rt.ac_runtime_batch_destroy(bt)
    assert rt.ac_runtime_batch_begin(ctx, ctypes.byref(bt)) == OK
    for i in range(8):
        assert rt.ac_runtime_batch_dispatch(bt, k, ctypes.byref(d3), None) == OK
    assert rt.ac_runtime_batch_dispatch(bt, k, ctypes.byref(d3), None) == E["DEVICE_BUSY"]
    assert rt.ac_runtime_batch_submit(bt, None) == OK
    rt.ac_runtime_batch_destroy(bt)
    assert np.array_equal(read(rt, D, n), a + 1)

    for h in (A, B, C, D):
        assert rt.ac_runtime_buffer_destroy(h) == OK
    assert rt.ac_runtime_kernel_destroy(k) == OK
    assert rt.ac_runtime_context_destroy(ctx) == OK


def test_batch_ranges_abort_and_retained_buffers(rt, image):
    ctx = new_ctx(rt)
    k = make(rt, ctx, image, "ac_add_one", 2, 4)
    n = 1024
    a = np.arange(n, dtype=np.float32)
    src, dst = new_buf(rt, ctx, a.nbytes, a), new_buf(rt, ctx, a.nbytes)
    assert rt.ac_runtime_buffer_fill(dst, 0, a.nbytes, 0) == OK
    bd = ac_rt.desc(ac_rt.BatchDesc, max_dispatches=8)
    bt = ctypes.c_void_p()
    assert rt.ac_runtime_batch_begin_ex(ctx, ctypes.byref(bd), ctypes.byref(bt)) == OK
    push = struct.pack("<I", 256)

    def bind(pairs):
        arr = (ac_rt.BufferBinding * len(pairs))(*[ac_rt.BufferBinding(b.value, o, r) for b, o, r in pairs])
        return arr

    g = ac_rt.Dim3(1, 1, 1)
    assert rt.ac_runtime_batch_dispatch_bindings(bt, k, bind([(src, 2, 1024), (dst, 0, 1024)]), 2, push, 4, g) == \
        E["BUFFER_ALIGNMENT_INVALID"]
    assert rt.ac_runtime_batch_dispatch_bindings(bt, k, bind([(src, 0, 0), (dst, 0, 1024)]), 2, push, 4, g) == \
        E["INVALID_BUFFER_SIZE"]
    assert rt.ac_runtime_batch_dispatch_bindings(bt, k, bind([(src, 3200, 1024), (dst, 0, 1024)]), 2, push, 4, g) == \
        E["INVALID_BUFFER_SIZE"]
    assert rt.ac_runtime_batch_dispatch_bindings(bt, k, bind([(src, 0, 1024)]), 1, push, 4, g) == \
        E["KERNEL_ARG_INVALID"]
    # elements 100..355 of src -> elements 512..767 of dst
    assert rt.ac_runtime_batch_dispatch_bindings(bt, k, bind([(src, 400, 1024), (dst, 2048, 1024)]), 2, push, 4, g) \
        == OK
    # the source handle goes away before the batch runs: the recorded launch keeps its memory
    assert rt.ac_runtime_buffer_destroy(src) == OK
    assert rt.ac_runtime_batch_submit(bt, None) == OK
    got = read(rt, dst, n)
    want = np.zeros(n, np.float32)
    want[512:768] = a[100:356] + 1
    assert np.array_equal(got, want)
    rt.ac_runtime_batch_destroy(bt)

    # an aborted batch never runs what it recorded
    src = new_buf(rt, ctx, a.nbytes, a)
    assert rt.ac_runtime_batch_begin_ex(ctx, ctypes.byref(bd), ctypes.byref(bt)) == OK
    d = launch(k, [src, dst], struct.pack("<I", n), (n // 256, 1, 1))
    assert rt.ac_runtime_batch_dispatch(bt, k, ctypes.byref(d), None) == OK
    assert rt.ac_runtime_batch_abort(bt) == OK
    assert rt.ac_runtime_batch_abort(bt) == OK
    assert rt.ac_runtime_batch_submit(bt, None) == E["INVALID_ARGUMENT"]
    assert rt.ac_runtime_batch_dispatch(bt, k, ctypes.byref(d), None) == E["INVALID_ARGUMENT"]
    assert rt.ac_runtime_context_destroy(ctx) == E["RESOURCE_IN_USE"]
    rt.ac_runtime_batch_destroy(bt)
    assert np.array_equal(read(rt, dst, n), want)
    for h in (src, dst):
        assert rt.ac_runtime_buffer_destroy(h) == OK
    assert rt.ac_runtime_kernel_destroy(k) == OK
    assert rt.ac_runtime_context_destroy(ctx) == OK


def test_pipeline_cache(rt):
    ctx = new_ctx(rt)
    size = ctypes.c_size_t(0)
    assert rt.ac_runtime_pipeline_cache_get_data(ctx, None, ctypes.byref(size)) == OK and size.value > 0
    small = ctypes.c_size_t(size.value - 1)
    data = ctypes.create_string_buffer(size.value)
    assert rt.ac_runtime_pipeline_cache_get_data(ctx, data, ctypes.byref(small)) == E["INVALID_BUFFER_SIZE"]
    got = ctypes.c_size_t(size.value)
    assert rt.ac_runtime_pipeline_cache_get_data(ctx, data, ctypes.byref(got)) == OK and got.value == size.value
    assert b"gfx950" in data.raw
    ctx2 = new_ctx(rt)
    assert rt.ac_runtime_pipeline_cache_merge(ctx2, data, size.value) == OK
    other = bytearray(data.raw)
    i = other.find(b"gfx950")
    other[i:i + 6] = b"gfx942"
    assert rt.ac_runtime_pipeline_cache_merge(ctx2, bytes(other), size.value) == E["INVALID_ARGUMENT"]
    assert rt.ac_runtime_pipeline_cache_merge(ctx2, data, size.value - 4) == E["INVALID_ARGUMENT"]
    assert rt.ac_runtime_pipeline_cache_merge(ctx2, None, 0) == E["NULL_POINTER"]
    assert rt.ac_runtime_context_destroy(ctx2) == OK
    assert rt.ac_runtime_context_destroy(ctx) == OK
