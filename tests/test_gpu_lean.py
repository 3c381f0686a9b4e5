"""The dedicated K = 4096 Q4_0 GEMV kernels against the generic one-column kernel whose block integers the oracle
checks, at the shapes they serve (Llama-3-8B: 14336 x 4096 gate/up rows, the stacked 28672 x 4096 gate|up, 6144 x
4096 q|k|v, 4096 x 4096 o):
  k_mmv_q4_0_k4096 (the headline kernel), k_mmv_q4_0_k4096_swiglu (stacked and over two matrices),
  k_mmv_q4_0_k4096_ep (ADD epilogue; ROPE + KV stores, stacked and over three matrices).
amv_debug_gemv_generic(1) makes the same calls run the generic kernel (k_mmv_q4_0 of the same rows per wave,
split and epilogue). The dedicated kernels keep its arithmetic and summation order, so every output (f32 values,
SWIGLU products, Q8_0 activation rows, f16 cache rows) must be equal bit for bit; the generic kernel's block
integers equal the oracle's, and the f32 outputs are within the reference's per-output gate of the oracle."""
import numpy as np
import pytest

from parity import dequant_act, per_output_gate

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


@pytest.fixture(scope="module")
def ops():
    from ameva_compute_amd import ops
    return ops


def gpu(x, dev):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


class generic:
    """Runs the enclosed GEMV calls on the generic kernel (parity instrumentation of the C ABI)."""

    def __init__(self, ops):
        self.lib = ops.lib()

    def __enter__(self):
        torch.cuda.synchronize()
        self.lib.amv_debug_gemv_generic(1)

    def __exit__(self, *exc):
        torch.cuda.synchronize()
        self.lib.amv_debug_gemv_generic(0)


def q4_0_weight(orc, rng, n, k):
    return orc.quantize_q4_0((rng.standard_normal((n, k)) * 0.02).astype(np.float32))


@pytest.mark.parametrize("n", [14336, 4096, 6144, 1024, 2])
def test_headline_kernel_equals_generic_and_oracle(dev, ops, orc, n):
    k = 4096
    rng = np.random.default_rng(n + 1)
    wg = q4_0_weight(orc, rng, n, k)
    x = rng.standard_normal((1, k)).astype(np.float32)
    a_ref = orc.quantize_q8_0(x, orc.Q8_X86)
    w = ops.QWeight.from_ggml(ops.Q4_0, gpu(wg, dev), n, k)
    act, _ = ops.quantize_act(gpu(x, dev), ops.Q8_0, ops.Q8_X86)
    y = ops.mul_mat_q(w, act, 1)
    with generic(ops):
        y_gen = ops.mul_mat_q(w, act, 1)
    assert torch.equal(y, y_gen)
    y_ref, s_ref = orc.mul_mat(ops.Q4_0, wg, n, k, a_ref, 1, with_blocks=True)
    assert np.array_equal(ops.block_sums(w, act, 1).cpu().numpy(), s_ref)
    worst = per_output_gate(y.cpu().numpy(), orc.dequantize(ops.Q4_0, wg, k), dequant_act(a_ref, 8, k),
                            what=f"k_mmv_q4_0_k4096 {n}x{k}")
    print(f"{n}x{k}: worst per-output error {worst:.2e} of sum |w a|")


def test_add_epilogue_kernel_equals_generic(dev, ops, orc):
    n, k = 4096, 4096
    rng = np.random.default_rng(11)
    w = ops.QWeight.from_ggml(ops.Q4_0, gpu(q4_0_weight(orc, rng, n, k), dev), n, k)
    act, _ = ops.quantize_act(gpu(rng.standard_normal((1, k)).astype(np.float32), dev), ops.Q8_0)
    e = gpu(rng.standard_normal(n).astype(np.float32), dev)
    v, eo = ops.mul_mat_vec_ep(w, act, ops.EP_ADD, e)
    with generic(ops):
        v_g, eo_g = ops.mul_mat_vec_ep(w, act, ops.EP_ADD, e)
    assert torch.equal(v, v_g) and torch.equal(eo, eo_g)
    assert torch.equal(v, ops.mul_mat_q(w, act, 1).reshape(-1))


@pytest.mark.parametrize("F", [14336, 64])
def test_swiglu_kernels_equal_generic(dev, ops, orc, F):
    """Stacked gate|up (two outputs per wave from 16384 rows) and the two-matrix form: the values, the SWIGLU
    products and the Q8_0 row of the product."""
    k = 4096
    rng = np.random.default_rng(F + 3)
    wg = q4_0_weight(orc, rng, 2 * F, k)
    w = ops.QWeight.from_ggml(ops.Q4_0, gpu(wg, dev), 2 * F, k)
    wgate = ops.QWeight.from_ggml(ops.Q4_0, gpu(np.ascontiguousarray(wg[:F]), dev), F, k)
    wup = ops.QWeight.from_ggml(ops.Q4_0, gpu(np.ascontiguousarray(wg[F:]), dev), F, k)
    act, _ = ops.quantize_act(gpu(rng.standard_normal((1, k)).astype(np.float32), dev), ops.Q8_0)
    lib = ops.lib()
    st = torch.cuda.current_stream().cuda_stream

    def seg():
        h = torch.empty(F, dtype=torch.float32, device=dev)
        a = torch.empty(lib.amv_act_bytes(ops.Q8_0, 1, F), dtype=torch.uint8, device=dev)
        cnt = torch.zeros(ops.swiglu_counter_words(2 * F), dtype=torch.int32, device=dev)
        rc = lib.amv_gemv_swiglu_q8_seg(ops.Q4_0, wgate.data.data_ptr(), wup.data.data_ptr(), F, k, act.data_ptr(),
                                        h.data_ptr(), a.data_ptr(), ops.Q8_0, ops.Q8_X86, cnt.data_ptr(), st)
        assert rc == 0, lib.amv_last_error()
        return h, a

    v, h, a = ops.gemv_swiglu_act(w, act)
    hs, as_ = seg()
    with generic(ops):
        v_g, h_g, a_g = ops.gemv_swiglu_act(w, act)
        hs_g, as_g = seg()
    assert torch.equal(v, v_g) and torch.equal(h, h_g) and torch.equal(a, a_g)
    assert torch.equal(hs, hs_g) and torch.equal(as_, as_g)
    assert torch.equal(hs, h) and torch.equal(as_, a)
    # the gate and up rows are the plain GEMV's values, which are within the gate of the oracle
    assert torch.equal(v, ops.mul_mat_q(w, act, 1).reshape(-1))


def test_rope_kv_kernels_equal_generic(dev, ops, orc):
    """q|k|v + ROPE + both cache rows, stacked and over three matrices (the plugin's form)."""
    n_head, n_head_kv, D, H = 32, 8, 128, 4096
    n, nq, kv = (n_head + 2 * n_head_kv) * D, n_head * D, n_head_kv * D
    rng = np.random.default_rng(21)
    wg = q4_0_weight(orc, rng, n, H)
    w = ops.QWeight.from_ggml(ops.Q4_0, gpu(wg, dev), n, H)
    parts = [ops.QWeight.from_ggml(ops.Q4_0, gpu(np.ascontiguousarray(wg[a:b]), dev), b - a, H)
             for a, b in ((0, nq), (nq, nq + kv), (nq + kv, n))]
    act, _ = ops.quantize_act(gpu(rng.standard_normal((1, H)).astype(np.float32), dev), ops.Q8_0)
    CTX = 64
    kc0 = gpu(rng.standard_normal((CTX, kv)).astype(np.float16), dev)
    vc0 = gpu(rng.standard_normal((CTX, kv)).astype(np.float16), dev)
    pos = torch.tensor([4095], dtype=torch.int32, device=dev)
    idx = torch.tensor([33], dtype=torch.int64, device=dev)
    lib = ops.lib()
    st = torch.cuda.current_stream().cuda_stream

    def stacked():
        kc, vc = kc0.clone(), vc0.clone()
        qkv = ops.gemv_rope_kv(w, act, n_head, n_head_kv, pos, kc, vc, idx)
        return qkv, kc, vc

    def segmented():
        kc, vc = kc0.clone(), vc0.clone()
        outs = [torch.empty(p.n_rows, dtype=torch.float32, device=dev) for p in parts]
        rc = lib.amv_gemv_rope_kv_seg(ops.Q4_0, parts[0].data.data_ptr(), parts[1].data.data_ptr(),
                                      parts[2].data.data_ptr(), H, act.data_ptr(), outs[0].data_ptr(),
                                      outs[1].data_ptr(), outs[2].data_ptr(), n_head, n_head_kv, D, pos.data_ptr(),
                                      500000.0, 1.0, 1.0, kc.data_ptr(), vc.data_ptr(), kv, idx.data_ptr(), CTX, None,
                                      st)
        assert rc == 0, lib.amv_last_error()
        return torch.cat(outs), kc, vc

    lean = [stacked(), segmented()]
    with generic(ops):
        gen = [stacked(), segmented()]
    for (q1, k1, v1), (q2, k2, v2) in zip(lean, gen):
        assert torch.equal(q1, q2)
        assert torch.equal(k1.view(torch.int16), k2.view(torch.int16))
        assert torch.equal(v1.view(torch.int16), v2.view(torch.int16))
    assert torch.equal(lean[0][0], lean[1][0])


@pytest.mark.parametrize("n", [1024, 2, 14336])
def test_read_probe_reads_every_weight_word(dev, ops, n):
    """amv_debug_gemv_read_probe (the bench's read ceiling of the headline mapping) folds every quant word of a row
    and every scale word of its row pair; with loads = 0 it writes the row index and reads nothing."""
    rng = np.random.default_rng(n + 17)
    raw = rng.integers(0, 2**32, size=n * 2304 // 4, dtype=np.uint32)
    words = raw[: n * 512].reshape(n, 512)
    scales = raw[n * 512:].reshape(n // 2, 128)
    want = np.bitwise_xor.reduce(words, axis=1) ^ np.repeat(np.bitwise_xor.reduce(scales, axis=1), 2)
    w = gpu(raw.view(np.uint8), dev)
    out = torch.full((n,), -1, dtype=torch.int32, device=dev)
    s = torch.cuda.current_stream().cuda_stream
    assert ops.lib().amv_debug_gemv_read_probe(w.data_ptr(), n, 4096, out.data_ptr(), 1, s) == 0
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy().view(np.uint32), want)
    assert ops.lib().amv_debug_gemv_read_probe(w.data_ptr(), n, 4096, out.data_ptr(), 0, s) == 0
    torch.cuda.synchronize()
    np.testing.assert_array_equal(out.cpu().numpy(), np.arange(n, dtype=np.int32))
    assert ops.lib().amv_debug_gemv_read_probe(w.data_ptr(), n + 1, 4096, out.data_ptr(), 1, s) != 0
