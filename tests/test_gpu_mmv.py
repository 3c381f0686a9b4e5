"""GPU parity of the quantizers, the weight repack and the decode GEMV against the CPU oracle, through the C ABI.

Bars: Q8_0 / Q4_0 / Q8_K bytes and per-block int32 sums bit-exact; f32 GEMV output within 1e-3 relative L2 of the
oracle (the observed error is ~1e-7: only the f32 summation order differs) and, output by output, within the
reference's gate |got - ref| <= 1e-5 sum |w a| (tests/parity.py).
"""
import numpy as np
import pytest

from parity import dequant_act, per_output_gate

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


def q8_edge_rows(k, rng):
    x = rng.standard_normal((6, k)).astype(np.float32)
    x[1, :32] = 0.0                                  # all-zero block: d = 0, q = 0
    x[2, :32] = np.arange(32, dtype=np.float32) - 15.5  # ties of x * 127/amax
    x[3, :] *= 1e-3
    x[4, k - 32:] = 127.0 * (np.arange(32) % 3 - 1)   # exact +-127
    x[5, :32] = np.float32(2.0) ** -20 * (np.arange(32) - 16)  # tiny block (fp16 subnormal d)
    return x


@pytest.mark.parametrize("rule", [0, 1, 2])
def test_quantize_q8_0_bytes(dev, ops, orc, rule):
    rng = np.random.default_rng(100 + rule)
    for k in (32, 4096, 14336):
        x = q8_edge_rows(k, rng)
        act, g = ops.quantize_act(gpu(x, dev), ops.Q8_0, rule, ggml=True)
        want = orc.quantize_q8_0(x, rule)
        got = g.cpu().numpy()
        assert np.array_equal(got, want), (k, np.argwhere(got != want)[:5])
        # the kernels' layout holds the same int8 values and the fp16-rounded d
        a = act.cpu().numpy()
        m = x.shape[0]
        qs = a[: m * k].view(np.int8).reshape(m, k // 32, 32)
        wb = want.reshape(m, k // 32, 34)
        assert np.array_equal(qs, wb[:, :, 2:].view(np.int8))
        meta = a[m * k:].view(np.int32).reshape(m, k // 32, 2)
        d16 = orc.fp16_to_fp32(wb[:, :, 0].astype(np.uint16) | (wb[:, :, 1].astype(np.uint16) << 8))
        assert np.array_equal(meta[:, :, 0].view(np.float32), d16)
        assert np.array_equal(meta[:, :, 1], qs.astype(np.int32).sum(axis=2))
        # without the ggml blocks the plain layout comes from the four-elements-per-lane kernel: the same bytes
        act2, _ = ops.quantize_act(gpu(x, dev), ops.Q8_0, rule)
        assert torch.equal(act2, act)


def test_quantize_q8_K_bytes(dev, ops, orc):
    rng = np.random.default_rng(7)
    x = rng.standard_normal((5, 4096)).astype(np.float32)
    x[1, :256] = 0.0
    x[2, 256:512] = 3.0          # ties for the max: the first element wins
    x[2, 300] = -3.0
    x[3] *= 1e-4
    x[4, :256] = 0.0  # exact ties (iscale = 1): round half to even, as the oracle's known answers pin
    x[4, 0] = -127.0
    x[4, 1:11] = [2.5, 3.5, -2.5, -3.5, 0.5, 1.5, -0.5, 126.5, -126.5, 64.5]
    _, g = ops.quantize_act(gpu(x, dev), ops.Q8_K, ggml=True)
    want = orc.quantize_q8_K(x)
    assert np.array_equal(g.cpu().numpy(), want)


def test_quantize_q4_0_bytes(dev, ops, orc):
    rng = np.random.default_rng(8)
    x = (rng.standard_normal((33, 4096)) * 0.02).astype(np.float32)
    x[0, :32] = 0.0
    x[1, 3] = -0.5                # magnitude tie: the first (index 3, -0.5) wins
    x[1, 5] = 0.5
    x[2, :32] = np.linspace(-1, 1, 32, dtype=np.float32)
    got = ops.quantize_q4_0(gpu(x, dev)).cpu().numpy()
    assert np.array_equal(got, orc.quantize_q4_0(x))


@pytest.mark.parametrize("wtype", [2, 8, 12, 14])
def test_repack_round_trip(dev, ops, wtype):
    rng = np.random.default_rng(9)
    be, bb = ops.BLOCK[wtype]
    for n, k in ((1, be), (37, be * 3), (128, 4096)):
        raw = rng.integers(0, 256, n * (k // be) * bb, dtype=np.uint8)
        w = ops.QWeight.from_ggml(wtype, gpu(raw, dev), n, k)
        assert w.nbytes == raw.size
        assert np.array_equal(w.to_ggml().cpu().numpy(), raw)


@pytest.mark.parametrize("n", [1, 6, 37])
def test_q4_0_repacked_layout(dev, ops, n):
    """The documented Q4_0 layout: qs[n][k/32][16] | scales of rows 2p, 2p+1 side by side per block, odd last row
    as a plain run."""
    rng = np.random.default_rng(n)
    k = 96
    nb = k // 32
    raw = rng.integers(0, 256, (n, nb, 18), dtype=np.uint8)
    w = ops.QWeight.from_ggml(2, gpu(raw.reshape(n, -1), dev), n, k)
    r = w.data.cpu().numpy().reshape(-1)
    assert np.array_equal(r[: n * nb * 16].reshape(n, nb, 16), raw[:, :, 2:])
    d = r[n * nb * 16:].view(np.uint16)
    dg = raw[:, :, :2].copy().view(np.uint16).reshape(n, nb)
    ne = n & ~1
    assert np.array_equal(d[: ne * nb].reshape(ne // 2, nb, 2), dg[:ne].reshape(ne // 2, 2, nb).transpose(0, 2, 1))
    if n % 2:
        assert np.array_equal(d[ne * nb:], dg[ne])


def _q4_0_case(orc, rng, n, k):
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    return orc.quantize_q4_0(w)


def _q8_0_case(orc, rng, n, k):
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    return orc.quantize_q8_0(w, orc.Q8_REF)


SHAPES = [(1, 32), (3, 64), (37, 96), (129, 2080), (4096, 4096), (14336, 4096), (4096, 14336)]


@pytest.mark.parametrize("wtype", [2, 8])
@pytest.mark.parametrize("n,k", SHAPES)
def test_gemv_parity(dev, ops, orc, wtype, n, k):
    rng = np.random.default_rng(n * 7 + k)
    wg = _q4_0_case(orc, rng, n, k) if wtype == 2 else _q8_0_case(orc, rng, n, k)
    x = rng.standard_normal((1, k)).astype(np.float32)
    a_ref = orc.quantize_q8_0(x, orc.Q8_X86)
    y_ref, s_ref = orc.mul_mat(wtype, wg, n, k, a_ref, 1, with_blocks=True)
    w = ops.QWeight.from_ggml(wtype, gpu(wg, dev), n, k)
    act, _ = ops.quantize_act(gpu(x, dev), ops.Q8_0, ops.Q8_X86)
    y = ops.mul_mat_q(w, act, 1).cpu().numpy()
    sums = ops.block_sums(w, act, 1).cpu().numpy()
    assert np.array_equal(sums, s_ref)
    assert rel_l2(y, y_ref) < TOL_F32
    per_output_gate(y, orc.dequantize(wtype, wg, k), dequant_act(a_ref, 8, k), what=f"GEMV {wtype} {n}x{k}")


@pytest.mark.parametrize("wtype", [2, 8])
def test_gemv_multi_column(dev, ops, orc, wtype):
    rng = np.random.default_rng(55)
    n, k, m = 300, 1024, 5
    wg = _q4_0_case(orc, rng, n, k) if wtype == 2 else _q8_0_case(orc, rng, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    a_ref = orc.quantize_q8_0(x, orc.Q8_X86)
    y_ref, s_ref = orc.mul_mat(wtype, wg, n, k, a_ref, m, with_blocks=True)
    w = ops.QWeight.from_ggml(wtype, gpu(wg, dev), n, k)
    y = ops.mul_mat(w, gpu(x, dev)).cpu().numpy()
    act, _ = ops.quantize_act(gpu(x, dev), ops.Q8_0)
    sums = ops.block_sums(w, act, m).cpu().numpy()
    assert np.array_equal(sums, s_ref)
    assert rel_l2(y, y_ref) < TOL_F32
    per_output_gate(y, orc.dequantize(wtype, wg, k), dequant_act(a_ref, 8, k), what="GEMV m=5")


def test_gemv_full_size_linearity(dev, ops):
    """Size-independent property at the BASELINE shape: the output is linear in the activation block sums, so
    scaling every activation by 2 (exact in the quantizer: d doubles, q unchanged) doubles the output exactly."""
    rng = np.random.default_rng(77)
    n, k = 14336, 4096
    wf = gpu((rng.standard_normal((n, k)) * 0.02).astype(np.float32), dev)
    w = ops.QWeight.from_ggml(ops.Q4_0, ops.quantize_q4_0(wf), n, k)
    x = gpu(rng.standard_normal((1, k)).astype(np.float32), dev)
    y1 = ops.mul_mat(w, x)
    y2 = ops.mul_mat(w, x * 2)
    assert torch.equal(y2, y1 * 2)


@pytest.mark.parametrize("wtype", [2, 8])
@pytest.mark.parametrize("n,k,m,pad", [(14336, 4096, 1, 0), (4096, 14336, 1, 0), (3, 64, 1, 0), (257, 640, 3, 0),
                                       (129, 2048, 8, 36), (64, 128, 2, 4)])
def test_gemv_raw_blocks(dev, ops, orc, wtype, n, k, m, pad):
    """amv_mul_mat_vec_raw: ggml's blocks read in place (the raw-layout MUL_MAT), rows of k/32 blocks plus `pad` bytes
    (a row view of a wider tensor keeps its parent's stride): block integers bit-exact, f32 within the gates."""
    rng = np.random.default_rng(n + k + m + pad + wtype)
    wg = _q4_0_case(orc, rng, n, k) if wtype == 2 else _q8_0_case(orc, rng, n, k)
    rb = wg.shape[1] + pad
    rows = np.zeros((n, rb), np.uint8)
    rows[:, : wg.shape[1]] = wg
    x = rng.standard_normal((m, k)).astype(np.float32)
    a_ref = orc.quantize_q8_0(x, orc.Q8_X86)
    y_ref, s_ref = orc.mul_mat(wtype, wg, n, k, a_ref, m, with_blocks=True)
    wd = gpu(rows.reshape(-1), dev)
    act, _ = ops.quantize_act(gpu(x, dev), ops.Q8_0, ops.Q8_X86)
    s = torch.cuda.current_stream().cuda_stream
    y = torch.empty((m, n), dtype=torch.float32, device=dev)
    sums = torch.empty((m, n, k // 32), dtype=torch.int32, device=dev)
    L = ops.lib()
    assert L.amv_mul_mat_vec_raw(wtype, wd.data_ptr(), rb, n, k, act.data_ptr(), m, y.data_ptr(), n, None, s) == 0
    assert L.amv_mul_mat_vec_raw(wtype, wd.data_ptr(), rb, n, k, act.data_ptr(), m, None, n, sums.data_ptr(), s) == 0
    torch.cuda.synchronize()
    assert np.array_equal(sums.cpu().numpy(), s_ref)
    y = y.cpu().numpy()
    assert rel_l2(y, y_ref) < TOL_F32
    per_output_gate(y, orc.dequantize(wtype, wg, k), dequant_act(a_ref, 8, k), what=f"raw {wtype} {n}x{k} m={m}")
    # the repacked GEMV of the same weight agrees within the same gates
    w = ops.QWeight.from_ggml(wtype, gpu(wg, dev), n, k)
    y2 = ops.mul_mat_q(w, act, m).cpu().numpy()
    assert rel_l2(y, y2) < 1e-6


def test_gemv_raw_blocks_refuses_bad_shapes(dev, ops):
    L = ops.lib()
    s = torch.cuda.current_stream().cuda_stream
    w = torch.zeros(64 * 1024, dtype=torch.uint8, device=dev)
    a = torch.zeros(64 * 1024, dtype=torch.uint8, device=dev)
    y = torch.zeros(1024, dtype=torch.float32, device=dev)
    assert L.amv_mul_mat_vec_raw(2, w.data_ptr(), 36, 4, 96, a.data_ptr(), 1, y.data_ptr(), 4, None, s) != 0  # k % 64
    assert L.amv_mul_mat_vec_raw(2, w.data_ptr(), 36, 4, 64, a.data_ptr(), 9, y.data_ptr(), 4, None, s) != 0  # m > 8
    assert L.amv_mul_mat_vec_raw(2, w.data_ptr(), 38, 4, 64, a.data_ptr(), 1, y.data_ptr(), 4, None, s) != 0  # stride
    assert L.amv_mul_mat_vec_raw(12, w.data_ptr(), 144, 4, 256, a.data_ptr(), 1, y.data_ptr(), 4, None, s) != 0  # Q4_K
