"""GPU parity of the prefill MUL_MAT (int8 MFMA) against the CPU oracle, through the C ABI: the MFMA's per-block
integer sums bit-exact, f32 output within 1e-3 relative L2, and at the BASELINE size (M = 512, 14336 x 4096) the
MFMA path agrees with the decode GEMV column by column."""
import numpy as np
import pytest

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
                                   (65, 129, 96), (300, 200, 1056), (130, 64, 32), (512, 1000, 4096)])
def test_mmq_block_sums_and_output(dev, ops, orc, wtype, m, n, k, atype):
    """Both kernels (int8 MFMA on plain Q8_0 activations; f16 MFMA on AMV_ACT_Q8_0_MMA for m > 64): the per-block
    integers bit for bit and the f32 output within the bar, ragged rows / tokens / odd block counts included."""
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
