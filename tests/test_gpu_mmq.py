"""GPU parity of the prefill MUL_MAT (int8 MFMA) against the CPU oracle, through the C ABI: the MFMA's per-block
integer sums bit-exact, f32 output within 1e-3 relative L2, and at the BASELINE size (M = 512, 14336 x 4096) the
MFMA path agrees with the decode GEMV column by column."""
import numpy as np
import pytest

from parity import TOL_F16_OPERANDS, dequant_act, per_output_gate

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

TOL_F32 = 1e-3


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


@pytest.fixture(scope="module")
def ops():
    from ameva_compute_amd import ops
    return ops


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def gpu(x, dev):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dev)


def weights(orc, rng, wtype, n, k):
    wf = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    return orc.quantize_q4_0(wf) if wtype == 2 else orc.quantize_q8_0(wf, orc.Q8_REF)


@pytest.mark.parametrize("atype", [8, 1008])
@pytest.mark.parametrize("wtype", [2, 8])
@pytest.mark.parametrize("m,n,k", [(8, 16, 32), (40, 200, 1024), (17, 129, 96), (128, 256, 4096), (512, 64, 14336),
                                   (65, 129, 96), (300, 200, 1056), (130, 64, 32), (512, 1000, 4096),
                                   (8, 64, 128), (16, 300, 1024), (32, 130, 4096), (17, 129, 1024), (24, 48, 512)])
def test_mmq_block_sums_and_output(dev, ops, orc, wtype, m, n, k, atype):
    """The batched kernels on both activation layouts: the streamed small-batch kernel (m <= 32, k % 128 == 0; Q4_0
    with an even row count), the tiled int8 kernels, the exact form above 64 tokens: the per-block integers bit for
    bit and the f32 output within the bar, ragged rows / tokens / odd block counts included."""
    rng = np.random.default_rng(m * 1000 + n + k + wtype)
    wg = weights(orc, rng, wtype, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    a_ref = orc.quantize_q8_0(x, orc.Q8_X86)
    y_ref, s_ref = orc.mul_mat(wtype, wg, n, k, a_ref, m, with_blocks=True)
    w = ops.QWeight.from_ggml(wtype, gpu(wg, dev), n, k)
    act, ag = ops.quantize_act(gpu(x, dev), atype, ggml=True)
    assert np.array_equal(ag.cpu().numpy(), a_ref)  # the MMA layout's quantization is ggml's, byte for byte
    sums = ops.block_sums(w, act, m, kernel="mmq").cpu().numpy()
    assert np.array_equal(sums, s_ref)
    y = ops.mul_mat_q(w, act, m, kernel="mmq").cpu().numpy()
    assert rel_l2(y, y_ref) < TOL_F32
    per_output_gate(y, orc.dequantize(wtype, wg, k), dequant_act(a_ref, 8, k), what=f"mmq {wtype} {m}x{n}x{k}")


@pytest.mark.parametrize("wtype", [2, 8])
def test_mmq_full_size(dev, ops, orc, wtype):
    """BASELINE config 2 shape at M = 512: against the oracle, and against the GEMV column by column."""
    rng = np.random.default_rng(5 + wtype)
    m, n, k = 512, 14336, 4096
    wf = gpu((rng.standard_normal((n, k)) * 0.02).astype(np.float32), dev)
    if wtype == 2:
        wg = ops.quantize_q4_0(wf)
    else:
        _, wg = ops.quantize_act(wf, ops.Q8_0, ops.Q8_REF, ggml=True)
    w = ops.QWeight.from_ggml(wtype, wg, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    act, ag = ops.quantize_act(gpu(x, dev), ops.Q8_0_MMA, ggml=True)
    y = ops.mul_mat_q(w, act, m, kernel="mmq")                   # f16 MFMA kernel (m > 64)
    y_mmv = ops.mul_mat_q(w, act, m, kernel="mmv")               # the GEMV on the layout's Q8_0 prefix
    assert rel_l2(y.cpu().numpy(), y_mmv.cpu().numpy()) < 1e-5
    act8, _ = ops.quantize_act(gpu(x, dev), ops.Q8_0)
    y8 = ops.mul_mat_q(w, act8, m, kernel="mmq")                 # int8 MFMA kernel
    assert rel_l2(y.cpu().numpy(), y8.cpu().numpy()) < 1e-5
    y_ref = orc.mul_mat(wtype, wg.cpu().numpy(), n, k, ag.cpu().numpy(), m)
    assert rel_l2(y.cpu().numpy(), y_ref) < TOL_F32
    # output by output, the batched product and the GEMV of the same rows are both within the reference's gate
    w_deq, a_deq = orc.dequantize(wtype, wg.cpu().numpy(), k), dequant_act(ag.cpu().numpy(), 8, k)
    per_output_gate(y.cpu().numpy(), w_deq, a_deq, what="mmq M=512")
    per_output_gate(y_mmv.cpu().numpy(), w_deq, a_deq, what="GEMV columns M=512")


def test_routing_matches_reference_threshold(dev, ops, orc):
    """MUL_MAT picks the MFMA kernel from 8 columns on (AMEVA_QGEMM_MIN_M), the GEMV below; both give the oracle."""
    rng = np.random.default_rng(21)
    n, k = 300, 2048
    wg = weights(orc, rng, 2, n, k)
    w = ops.QWeight.from_ggml(2, gpu(wg, dev), n, k)
    for m in (1, 7, 8, 16):
        x = rng.standard_normal((m, k)).astype(np.float32)
        y = ops.mul_mat(w, gpu(x, dev)).cpu().numpy()
        y_ref = orc.mul_mat(2, wg, n, k, orc.quantize_q8_0(x, orc.Q8_X86), m)
        assert rel_l2(y, y_ref) < TOL_F32


def random_q4k(rng, n, k):
    """Random bytes are valid Q4_K blocks once the fp16 d, dmin are small finite values (6-bit scales and mins and
    nibbles then take every value, the worst case of the exact-sum bounds)."""
    y = rng.integers(0, 256, (n, k // 256, 144), dtype=np.uint8)
    for off in (0, 2):
        v = rng.uniform(0.0, 0.002, (n, k // 256)).astype(np.float16)
        y[:, :, off:off + 2] = v.view(np.uint8).reshape(n, k // 256, 2)
    return y.reshape(n, -1)


@pytest.mark.parametrize("m,n,k", [(8, 64, 256), (16, 300, 1024), (70, 129, 512), (512, 256, 4096),
                                   (512, 64, 14336), (130, 14336 // 8, 4096), (300, 200, 768), (65, 64, 256),
                                   (512, 2048, 4096)])
def test_mmq_q4k_block_sums_and_output(dev, ops, orc, m, n, k):
    """Batched Q4_K on the f16 matrix cores: the per-super-block integers (sum sc * dot, sum m * bsum) bit-exact
    against the oracle, f32 within 1e-3; the Q8_K prefix of the extended activations is the plain Q8_K layout."""
    rng = np.random.default_rng(m + n + k)
    wg = random_q4k(rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[0, :300] *= 40.0  # large activations: |q| = 127 across whole blocks
    a_ref = orc.quantize_q8_K(x)
    y_ref, s_ref = orc.mul_mat(ops.Q4_K, wg, n, k, a_ref, m, with_blocks=True)
    w = ops.QWeight.from_ggml(ops.Q4_K, gpu(wg, dev), n, k)
    act, ag = ops.quantize_act(gpu(x, dev), ops.Q8_K_MMA, ggml=True)
    assert np.array_equal(ag.cpu().numpy(), a_ref)
    plain, _ = ops.quantize_act(gpu(x, dev), ops.Q8_K)
    assert torch.equal(act[: plain.numel()], plain)
    sums = ops.block_sums(w, act, m, kernel="mmq").cpu().numpy()
    assert np.array_equal(sums, s_ref)
    y = ops.mul_mat_q(w, act, m, kernel="mmq").cpu().numpy()
    assert rel_l2(y, y_ref) < TOL_F32
    y_v = ops.mul_mat_q(w, act, m, kernel="mmv").cpu().numpy()  # the GEMV on the same buffer's Q8_K prefix
    assert rel_l2(y, y_v) < 1e-5
    w_deq, a_deq = orc.dequantize(ops.Q4_K, wg, k), dequant_act(a_ref, 15, k)
    per_output_gate(y, w_deq, a_deq, what=f"mmq Q4_K {m}x{n}x{k}")
    per_output_gate(y_v, w_deq, a_deq, what=f"GEMV Q4_K columns {m}x{n}x{k}")


def deq_f16_region(act, m, k, q4k):
    """The f16 region of a DEQ (or MMA) activation buffer, [m, k] halves (offsets of amv_q8k_mma_layout /
    amv_q8_0_mma_layout)."""
    base = m * k + (m * (k // 256) * 4 + m * (k // 16) * 4 if q4k else m * (k // 32) * 8)
    off = (base + 15) // 16 * 16
    return act[off: off + 2 * m * k].cpu().numpy().view(np.float16).reshape(m, k)


@pytest.mark.parametrize("wtype", [2, 8, 12])
@pytest.mark.parametrize("m,n,k", [(65, 129, 256), (130, 64, 512), (300, 200, 1024), (512, 1000, 4096),
                                   (200, 4096, 14336 // 256 * 256)])
def test_scaled_gemm_matches_oracle_and_exact_form(dev, ops, orc, wtype, m, n, k):
    """The scaled batched MUL_MAT (DEQ layouts: f16 (q - 8) d_w / (d sc) q - dmin m against f16 q_a d_a, one MFMA
    accumulation across k): the activation's f16 copies are exactly f16(q * d) of its own plain prefix, the plain
    prefix is ggml's quantization, and the f32 result is within 1e-3 relative L2 of the oracle and of the exact-sum
    form; block sums are refused on the scaled layout."""
    q4k = wtype == ops.Q4_K
    rng = np.random.default_rng(m + n + k + wtype)
    wg = random_q4k(rng, n, k) if q4k else weights(orc, rng, wtype, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[0, :100] *= 30.0
    a_ref = orc.quantize_q8_K(x) if q4k else orc.quantize_q8_0(x, orc.Q8_X86)
    y_ref = orc.mul_mat(wtype, wg, n, k, a_ref, m)
    w = ops.QWeight.from_ggml(wtype, gpu(wg, dev), n, k)
    deq_t, mma_t = (ops.Q8_K_DEQ, ops.Q8_K_MMA) if q4k else (ops.Q8_0_DEQ, ops.Q8_0_MMA)
    act_d, ag = ops.quantize_act(gpu(x, dev), deq_t, ggml=True)
    assert np.array_equal(ag.cpu().numpy(), a_ref)
    act_e, _ = ops.quantize_act(gpu(x, dev), mma_t)
    plain_n = m * k + (m * (k // 256) * 4 + m * (k // 16) * 4 if q4k else m * (k // 32) * 8)
    assert torch.equal(act_d[:plain_n], act_e[:plain_n])
    q = act_d[: m * k].cpu().numpy().view(np.int8).reshape(m, k).astype(np.float32)
    if q4k:
        d = act_d[m * k: m * k + m * (k // 256) * 4].cpu().numpy().view(np.float32).reshape(m, k // 256)
        d = np.repeat(d, 256, axis=1)
    else:
        meta = act_d[m * k: m * k + m * (k // 32) * 8].cpu().numpy().view(np.float32).reshape(m, k // 32, 2)
        d = np.repeat(meta[:, :, 0], 32, axis=1)
    # q * d rounded to f16 once (the exact product), or through f32 first (the compiler may fuse the product and the
    # conversion into one mixed-precision fma); for Q8_0 the f32 product is exact and both agree
    # (compared as values: q = 0 times a negative Q8_K scale is -0 on the CPU, +0 from the fused form)
    once = (q.astype(np.float64) * d.astype(np.float64)).astype(np.float16)
    twice = (q * d).astype(np.float16)
    got = deq_f16_region(act_d, m, k, q4k)
    assert np.all((got == once) | (got == twice))
    y_d = ops.mul_mat_q(w, act_d, m, kernel="mmq", act_t=deq_t).cpu().numpy()
    y_e = ops.mul_mat_q(w, act_e, m, kernel="mmq", act_t=mma_t).cpu().numpy()
    e_ref, e_ex = rel_l2(y_d, y_ref), rel_l2(y_d, y_e)
    print(f"scaled form: rel L2 {e_ref:.2e} against the oracle, {e_ex:.2e} against the exact form")
    assert e_ref < TOL_F32 and e_ex < TOL_F32
    # each operand rounded once to f16: per output within 2^-10 sum |w a| (the exact form within 1e-5)
    w_deq, a_deq = orc.dequantize(wtype, wg, k), dequant_act(a_ref, 15 if q4k else 8, k)
    per_output_gate(y_d, w_deq, a_deq, tol=TOL_F16_OPERANDS, what="scaled form")
    per_output_gate(y_e, w_deq, a_deq, what="exact form")
    sums = torch.empty(m * n * (k // 256 * 2 if q4k else k // 32), dtype=torch.int32, device=dev)
    rc = ops.lib().amv_mul_mat_q_act_block_sums(wtype, w.data.data_ptr(), n, k, act_d.data_ptr(), deq_t, m,
                                                sums.data_ptr(), torch.cuda.current_stream().cuda_stream)
    assert rc != 0 and b"exact layout" in ops.lib().amv_last_error()


def test_split_k_under_graph_capture(dev, ops, orc):
    """The scaled GEMM split over k (4096 x 14336 at 200 tokens) inside a captured graph: every replay equals the
    eager result bit for bit (the partials are summed in a fixed order), also with eager calls of a larger batch
    between the replays (the library's split-k workspace has a fixed size, allocated by the first uncaptured call
    that splits k, and never moves)."""
    rng = np.random.default_rng(77)
    n, k, m = 4096, 14336, 200
    wg = weights(orc, rng, ops.Q4_0, n, k)
    w = ops.QWeight.from_ggml(ops.Q4_0, gpu(wg, dev), n, k)
    x = gpu(rng.standard_normal((m, k)).astype(np.float32), dev)
    act, _ = ops.quantize_act(x, ops.Q8_0_DEQ)
    y_eager = ops.mul_mat_q(w, act, m, kernel="mmq", act_t=ops.Q8_0_DEQ)
    out = torch.empty_like(y_eager)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ops.mul_mat_q(w, act, m, out, kernel="mmq", act_t=ops.Q8_0_DEQ)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        ops.mul_mat_q(w, act, m, out, kernel="mmq", act_t=ops.Q8_0_DEQ)
    big_m = 512
    xb = gpu(rng.standard_normal((big_m, k)).astype(np.float32), dev)
    actb, _ = ops.quantize_act(xb, ops.Q8_0_DEQ)
    for rep in range(3):
        out.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, y_eager), rep
        # eager work between the replays, the larger batch asking for a larger workspace
        yb = ops.mul_mat_q(w, actb, big_m, kernel="mmq", act_t=ops.Q8_0_DEQ)
        torch.cuda.synchronize()
        assert torch.isfinite(yb).all()
    assert torch.equal(ops.mul_mat_q(w, act, m, kernel="mmq", act_t=ops.Q8_0_DEQ), y_eager)


@pytest.mark.parametrize("m", [8, 16, 40])
def test_mul_mat_q_plain_q8k_for_q4k(dev, ops, orc, m):
    """amv_mul_mat_q, and amv_mul_mat_q_act with act_type AMV_T_Q8_K, on a plain Q8_K activation (no f16 copies) for
    Q4_K weights: small batches go to the tiled int8 kernel, which reads only the plain layout (the small-batch
    kernels need AMV_ACT_Q8_K_MMA); both equal, within the per-output gate of the oracle."""
    from ameva_compute_amd._lib import lib
    rng = np.random.default_rng(300 + m)
    n, k = 96, 1024
    wg = random_q4k(rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    y_ref = orc.mul_mat(ops.Q4_K, wg, n, k, orc.quantize_q8_K(x), m)
    w = ops.QWeight.from_ggml(ops.Q4_K, gpu(wg, dev), n, k)
    plain, _ = ops.quantize_act(gpu(x, dev), ops.Q8_K)
    out = torch.empty((m, n), dtype=torch.float32, device=dev)
    st = torch.cuda.current_stream().cuda_stream
    assert lib().amv_mul_mat_q(ops.Q4_K, w.data.data_ptr(), n, k, plain.data_ptr(), m, out.data_ptr(), n, st) == 0
    assert rel_l2(out.cpu().numpy(), y_ref) < TOL_F32
    out2 = torch.empty_like(out)
    rc = lib().amv_mul_mat_q_act(ops.Q4_K, w.data.data_ptr(), n, k, plain.data_ptr(), ops.Q8_K, m, out2.data_ptr(), n,
                                 st)
    assert rc == 0, lib().amv_last_error()
    assert torch.equal(out2, out)
    per_output_gate(out.cpu().numpy(), orc.dequantize(ops.Q4_K, wg, k), dequant_act(orc.quantize_q8_K(x), 15, k),
                    what=f"Q4_K plain Q8_K m={m}")


@pytest.mark.parametrize("wtype,atype,m,n,k", [
    (2, "Q8_0", 512, 4096, 14336),     # exact tiled, k split: the residual joins in the sum of the partials
    (2, "Q8_0", 130, 256, 4096),       # exact tiled, one k range: the residual in the epilogue
    (12, "Q8_K", 512, 1024, 4096),     # exact Q4_K tiled
    (12, "Q8_K_MMA", 16, 512, 1024),   # small-batch Q4_K kernel + a second launch
    (2, "Q8_0", 16, 256, 1024),        # streamed small-batch kernel + a second launch
    (2, "Q8_0_DEQ", 130, 256, 4096),   # scaled form + a second launch
])
def test_mul_mat_q_add(dev, ops, orc, wtype, atype, m, n, k):
    """amv_mul_mat_q_act_add equals amv_mul_mat_q_act followed by the ADD, bit for bit, on every path."""
    rng = np.random.default_rng(m + n + k + wtype)
    if wtype == 2:
        wg = orc.quantize_q4_0((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    else:
        wg = random_q4k(rng, n, k)
    w = ops.QWeight.from_ggml(wtype, gpu(wg, dev), n, k)
    at = getattr(ops, atype)
    act, _ = ops.quantize_act(gpu(rng.standard_normal((m, k)).astype(np.float32), dev), at)
    res = gpu(rng.standard_normal((m, n)).astype(np.float32), dev)
    y = ops.mul_mat_q(w, act, m, kernel="mmq", act_t=at)
    got = ops.mul_mat_q_add(w, act, m, res, act_t=at)
    assert torch.equal(got, y + res)
    with pytest.raises(Exception, match="overlaps"):
        ops.mul_mat_q_add(w, act, m, got, act_t=at, out=got)


def random_q6k(rng, n, k):
    """Random bytes are valid Q6_K blocks once the fp16 d is a small finite value (codes, int8 sub-block scales and
    high bits then take every value)."""
    y = rng.integers(0, 256, (n, k // 256, 210), dtype=np.uint8)
    v = rng.uniform(0.0, 0.002, (n, k // 256)).astype(np.float16)
    y[:, :, 208:210] = v.view(np.uint8).reshape(n, k // 256, 2)
    return y.reshape(n, -1)


@pytest.mark.parametrize("m,n,k", [(8, 64, 256), (16, 300, 1024), (17, 129, 512), (32, 512, 4096), (24, 33, 256),
                                   (1, 70, 512), (16, 8192, 1024), (32, 100, 2048)])
@pytest.mark.parametrize("atype", ["Q8_K", "Q8_K_MMA"])
def test_mmq_q6k_small_batch(dev, ops, orc, m, n, k, atype):
    """The streamed small-batch Q6_K kernel (k_mmq_q6k_sb, m <= 32; sub-block sums from v_mfma_i32_16x16x32_i8 with
    the other sub-block's activation slots zeroed): each super-block's integer I = sum_s sc_s sum q a bit-exact against
    the oracle, every output within the per-output gate, on both activation layouts; ragged rows and tokens, one or
    two 16-row tiles per wave, one or two token tiles."""
    rng = np.random.default_rng(m * 7 + n + k)
    wg = random_q6k(rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[0, :100] *= 30.0  # |q| = 127 in whole sub-blocks
    a_ref = orc.quantize_q8_K(x)
    y_ref, s_ref = orc.mul_mat(ops.Q6_K, wg, n, k, a_ref, m, with_blocks=True)
    w = ops.QWeight.from_ggml(ops.Q6_K, gpu(wg, dev), n, k)
    at = getattr(ops, atype)
    act, ag = ops.quantize_act(gpu(x, dev), at, ggml=True)
    assert np.array_equal(ag.cpu().numpy(), a_ref)
    sums = torch.empty(m * n * (k // 256), dtype=torch.int32, device=dev)
    rc = ops.lib().amv_mul_mat_q_act_block_sums(ops.Q6_K, w.data.data_ptr(), n, k, act.data_ptr(), at, m,
                                                sums.data_ptr(), torch.cuda.current_stream().cuda_stream)
    assert rc == 0, ops.lib().amv_last_error()
    assert np.array_equal(sums.cpu().numpy().reshape(s_ref.shape), s_ref)
    y = ops.mul_mat_q(w, act, m, kernel="mmq", act_t=at).cpu().numpy()
    assert rel_l2(y, y_ref) < TOL_F32
    per_output_gate(y, orc.dequantize(ops.Q6_K, wg, k), dequant_act(a_ref, 15, k), what=f"Q6_K m={m} {n}x{k}")
    res = gpu(rng.standard_normal((m, n)).astype(np.float32), dev)  # the residual form: a second launch adds it
    assert torch.equal(ops.mul_mat_q_add(w, act, m, res, act_t=at), torch.from_numpy(y).to(dev) + res)
