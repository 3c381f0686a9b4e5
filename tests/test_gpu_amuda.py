"""libamuda_hip.so on the GPU, the flow of the reference's tests/test_amuda_bitnet_exact.c: ac_init, buffers,
ac_ops_bitnet_gemv_i2_s_exact on the 2560 x 6912 ffn_down shape with x = sin(0.05 k) / 2, ac_event_wait, sync to
host; every row within the reference's own bar (|y - y_ref| <= 1e-3 against its sequential f32 dequantize-and-sum),
and within 1e-5 relative L2 of a float64 sum. bitnet_raw_vec_dot_i2_s (host memory) against the oracle's exact
integers for the three kernel types."""
import ctypes

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

from test_amuda_abi import AcBuffer, AcContext, AcEvent, load  # noqa: E402


@pytest.fixture(scope="module")
def amuda():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    lib = load()
    lib.ac_init.argtypes = [ctypes.POINTER(ctypes.POINTER(AcContext))]
    lib.ac_buffer_alloc.argtypes = [ctypes.POINTER(AcContext), ctypes.c_size_t, ctypes.POINTER(ctypes.POINTER(AcBuffer))]
    lib.ac_buffer_sync_to_host.argtypes = [ctypes.POINTER(AcContext), ctypes.POINTER(AcBuffer)]
    lib.ac_buffer_free.argtypes = [ctypes.POINTER(AcContext), ctypes.POINTER(AcBuffer)]
    lib.ac_event_wait.argtypes = [ctypes.POINTER(AcContext), ctypes.POINTER(AcEvent)]
    lib.ac_event_get_duration_us.argtypes = [ctypes.POINTER(AcEvent)]
    lib.ac_event_get_duration_us.restype = ctypes.c_uint64
    lib.ac_event_free.argtypes = [ctypes.POINTER(AcContext), ctypes.POINTER(AcEvent)]
    lib.ac_destroy.argtypes = [ctypes.POINTER(AcContext)]
    return lib


def random_i2s(rng, m, k):
    codes = rng.integers(0, 3, (m, k)).astype(np.uint8)  # valid codes 0..2 (weights -1, 0, +1)
    blk = codes.reshape(m, k // 128, 4, 32)             # weight 32 g + i of a block -> byte i, bits 6 - 2 g
    packed = (blk[:, :, 0] << 6) | (blk[:, :, 1] << 4) | (blk[:, :, 2] << 2) | blk[:, :, 3]
    return packed.reshape(m, k // 4).astype(np.uint8), codes


def test_bitnet_gemv_i2_s_exact_reference_flow(amuda):
    lib = amuda
    ctx = ctypes.POINTER(AcContext)()
    assert lib.ac_init(ctypes.byref(ctx)) == 0
    assert ctx.contents.vendor_id == 0x1002 and ctx.contents.max_compute_units > 0 and not ctx.contents.is_uma_supported
    M, K = 2560, 6912
    rng = np.random.default_rng(2560)
    wp, codes = random_i2s(rng, M, K)
    codes[0, :7] = 3  # code 3 maps to 0 in this entry (amuda map2bit), whatever the integer path does
    blk = codes.reshape(M, K // 128, 4, 32)
    wp = ((blk[:, :, 0] << 6) | (blk[:, :, 1] << 4) | (blk[:, :, 2] << 2) | blk[:, :, 3]).reshape(M, K // 4)
    wp = wp.astype(np.uint8)
    scale = np.float32(2.2931101)
    x = (np.sin(np.arange(K, dtype=np.float32) * np.float32(0.05)) * np.float32(0.5)).astype(np.float32)
    bx, bw, by = (ctypes.POINTER(AcBuffer)() for _ in range(3))
    assert lib.ac_buffer_alloc(ctx, K * 4, ctypes.byref(bx)) == 0
    assert lib.ac_buffer_alloc(ctx, wp.nbytes, ctypes.byref(bw)) == 0
    assert lib.ac_buffer_alloc(ctx, M * 4, ctypes.byref(by)) == 0
    ctypes.memmove(bx.contents.host_ptr, x.ctypes.data, x.nbytes)
    ctypes.memmove(bw.contents.host_ptr, wp.ctypes.data, wp.nbytes)
    ev = ctypes.c_void_p()
    rc = lib.ac_ops_bitnet_gemv_i2_s_exact(ctx, M, K, bx, bw, ctypes.c_float(scale), by, ctypes.byref(ev))
    assert rc == 0 and ev.value
    evp = ctypes.cast(ev, ctypes.POINTER(AcEvent))
    assert lib.ac_event_wait(ctx, evp) == 0
    assert lib.ac_event_get_duration_us(evp) == evp.contents.duration_us
    assert lib.ac_buffer_sync_to_host(ctx, by) == 0
    y = np.ctypeslib.as_array(ctypes.cast(by.contents.host_ptr, ctypes.POINTER(ctypes.c_float)), (M,)).copy()
    # the reference test's own check: dequantize with map2bit {-1, 0, 1, 0}, sequential f32 sum, times the scale
    m2b = np.array([-1.0, 0.0, 1.0, 0.0], np.float32)
    deq = m2b[codes]
    y_seq = np.zeros(M, np.float32)
    for j in range(K):
        y_seq += deq[:, j] * x[j]
    y_seq *= scale
    assert np.max(np.abs(y - y_seq)) <= 1e-3
    y64 = (deq.astype(np.float64) @ x.astype(np.float64)) * float(scale)
    assert np.linalg.norm(y - y64) / np.linalg.norm(y64) < 1e-5
    assert lib.ac_event_free(ctx, evp) == 0
    for b in (bx, bw, by):
        assert lib.ac_buffer_free(ctx, b) == 0
    assert lib.ac_destroy(ctx) == 0


@pytest.mark.parametrize("kernel_type,n,nrc", [(0, 6912, 5), (1, 2560, 9), (2, 128, 3), (0, 2560, 1)])
def test_raw_vec_dot(amuda, orc, kernel_type, n, nrc):
    rng = np.random.default_rng(n + nrc + kernel_type)
    rows = 1 if kernel_type == 1 else nrc
    wp, codes = random_i2s(rng, rows, n)
    cols = nrc if kernel_type == 1 else 1
    q = rng.integers(-127, 128, (cols, n)).astype(np.int8)
    s = np.zeros(nrc, np.float32)
    amuda.bitnet_raw_vec_dot_i2_s(n, s.ctypes.data, wp.ctypes.data, q.ctypes.data, nrc, kernel_type)
    # exact integers sum (c - 1) q (ggml_bitnet_mad.cpp:191-231), as the oracle's I2_S restatement computes them
    _, ints = orc.i2s_gemv(wp, rows, n, q, np.ones(cols, np.float32), 1.0)
    want = ints.reshape(-1).astype(np.float32)
    assert np.array_equal(s, want)
