"""GPU parity of the K-quant GEMVs, BitNet I2_S, RMS_NORM (+MUL +Q8_0), ROPE, SWIGLU and FLASH_ATTN_EXT decode
against the CPU oracle, through the C ABI.

Bars: integer block sums and I2_S integer outputs bit-exact; Q8_0 bytes of the fused quantization bit-exact; f32
outputs within 1e-3 relative L2 of the oracle; attention with the f16 KV cache within 2e-3.
"""
import numpy as np
import pytest

from parity import dequant_act, per_output_gate

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

TOL_F32 = 1e-3
TOL_FA = 2e-3


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


def random_kquant(rng, t, n, k):
    """Random bytes are valid Q4_K / Q6_K blocks once the fp16 scales are small finite values."""
    bb = 144 if t == 12 else 210
    y = rng.integers(0, 256, (n, k // 256, bb), dtype=np.uint8)
    def put(off):
        v = rng.uniform(0.0, 0.002, (n, k // 256)).astype(np.float16)
        y[:, :, off:off + 2] = v.view(np.uint8).reshape(n, k // 256, 2)
    if t == 12:
        put(0)
        put(2)
    else:
        put(208)
    return y.reshape(n, -1)


KSHAPES = [(1, 256), (37, 512), (300, 2048), (4096, 4096), (14336, 4096), (4096, 14336)]


@pytest.mark.parametrize("wtype", [12, 14])
@pytest.mark.parametrize("n,k", KSHAPES)
def test_kquant_gemv_parity(dev, ops, orc, wtype, n, k):
    rng = np.random.default_rng(n + k + wtype)
    wg = random_kquant(rng, wtype, n, k)
    x = rng.standard_normal((1, k)).astype(np.float32)
    a_ref = orc.quantize_q8_K(x)
    y_ref, s_ref = orc.mul_mat(wtype, wg, n, k, a_ref, 1, with_blocks=True)
    w = ops.QWeight.from_ggml(wtype, gpu(wg, dev), n, k)
    act, ag = ops.quantize_act(gpu(x, dev), ops.Q8_K, ggml=True)
    assert np.array_equal(ag.cpu().numpy(), a_ref)
    y = ops.mul_mat_q(w, act, 1).cpu().numpy()
    sums = ops.block_sums(w, act, 1).cpu().numpy()
    assert np.array_equal(sums, s_ref)
    assert rel_l2(y, y_ref) < TOL_F32
    per_output_gate(y, orc.dequantize(wtype, wg, k), dequant_act(a_ref, 15, k), what=f"GEMV {wtype} {n}x{k}")


@pytest.mark.parametrize("wtype", [12, 14])
def test_kquant_quantizer_valid_and_gemv(dev, ops, orc, wtype):
    """The library's own K-quant rule yields valid blocks: the oracle's dequantization (pinned by known answers)
    reproduces the input within the 4- / 6-bit error, and the GEMV on those bytes matches the oracle."""
    rng = np.random.default_rng(3)
    n, k = 512, 4096
    wf = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    wg = ops.quantize_k(gpu(wf, dev), wtype).cpu().numpy()
    deq = orc.dequantize(wtype, wg, k)
    err = rel_l2(deq, wf)
    assert err < (0.12 if wtype == 12 else 0.03), err
    x = rng.standard_normal((1, k)).astype(np.float32)
    y_ref = orc.mul_mat(wtype, wg, n, k, orc.quantize_q8_K(x), 1)
    y = ops.mul_mat(ops.QWeight.from_ggml(wtype, gpu(wg, dev), n, k), gpu(x, dev)).cpu().numpy()
    assert rel_l2(y, y_ref) < TOL_F32


# ----------------------------------------------------------------------------------------------------- I2_S
def pack_i2s(codes):
    n, k = codes.shape
    w = np.zeros((n, k // 4), np.uint8)
    for b in range(k // 128):
        for g in range(4):
            w[:, 32 * b:32 * b + 32] |= (codes[:, 128 * b + 32 * g:128 * b + 32 * g + 32] << (6 - 2 * g)).astype(np.uint8)
    return w


@pytest.mark.parametrize("n,k,m", [(6912, 2560, 1), (2560, 6912, 1), (6912, 2560, 128), (2560, 6912, 128), (3, 128, 2),
                                   (129, 256, 5), (100, 384, 70), (64, 128, 8), (1000, 1280, 2000)])
def test_i2s_parity(dev, ops, orc, n, k, m):
    """m < 8: the GEMV; m >= 8: the int8-MFMA kernel k_i2s_mmq_p (BASELINE config 3 batch 128): 64 x 64 tiles whose
    k blocks the 4 waves share, unsplit when the tiles fill the GPU (6912 x 2560: 5 blocks per wave in two chunks;
    1000 x 1280 at m = 2000 with ragged row and token tiles) or with k split over workgroups and the partials added
    in a second launch (2560 x 6912: 3 splits of 18 blocks; the small shapes). Integer outputs bit-exact and the f32
    outputs bit-exact too (the same f32 operations as the CPU on the same integer)."""
    rng = np.random.default_rng(n * 3 + k + m)
    codes = rng.integers(0, 3, (n, k))
    w = pack_i2s(codes)
    scale = np.float32(1.37)
    tensor = np.concatenate([w.reshape(-1), np.frombuffer(scale.tobytes(), np.uint8), np.zeros(28, np.uint8)])
    x = rng.standard_normal((m, k)).astype(np.float32)
    x[0, :7] = 0.0
    q_ref, deq_ref = orc.i2s_quantize_act(x)
    out_ref, sums_ref = orc.i2s_gemv(w, n, k, q_ref, deq_ref, float(scale))
    tg = gpu(tensor, dev)
    assert ops.i2s_tensor_scale(tg, n, k) == scale
    act = ops.i2s_quantize_act(gpu(x, dev))
    a = act.cpu().numpy()
    assert np.array_equal(a[: m * k].view(np.int8).reshape(m, k), q_ref)
    meta = a[m * k:].view(np.int32).reshape(m, 2)
    assert np.array_equal(meta[:, 0].view(np.float32), deq_ref)
    assert np.array_equal(meta[:, 1], q_ref.astype(np.int32).sum(axis=1))
    sums = ops.i2s_gemv_sums(tg, n, k, act, m).cpu().numpy()
    assert np.array_equal(sums, sums_ref.astype(np.int32))
    out = ops.i2s_gemv(tg, n, k, act, m, float(scale)).cpu().numpy()
    assert np.array_equal(out.view(np.uint32), out_ref.view(np.uint32))  # same f32 operations: bit-exact


def test_i2s_on_reference_fixture(dev, ops, orc):
    """The reference's upstream I2_S fixture (2 rows x 128, scale trailer 1.625) through the GPU GEMV: the integer
    sums equal the dot of the fixture's independent expected f32 weights (divided by the scale) with q."""
    import os
    gold = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
    data = np.fromfile(os.path.join(gold, "fixture_i2s_upstream.bin"), np.uint8)
    expected = np.fromfile(os.path.join(gold, "expected_i2s_upstream_f32.bin"), np.float32).reshape(2, 128)
    rng = np.random.default_rng(11)
    x = rng.standard_normal((1, 128)).astype(np.float32)
    tg = gpu(data, dev)
    scale = ops.i2s_tensor_scale(tg, 2, 128)
    assert scale == 1.625
    act = ops.i2s_quantize_act(gpu(x, dev))
    q = act.cpu().numpy()[:128].view(np.int8).astype(np.int64)
    want = (expected.astype(np.float64) / scale) @ q
    sums = ops.i2s_gemv_sums(tg, 2, 128, act, 1).cpu().numpy()[0]
    assert np.array_equal(sums, want.astype(np.int64))


# ---------------------------------------------------------------------------------------------- RMS_NORM
@pytest.mark.parametrize("m,n", [(1, 4096), (7, 4096), (3, 14336), (2, 2560)])
def test_rms_norm_fused(dev, ops, orc, m, n):
    rng = np.random.default_rng(m * n)
    x = (rng.standard_normal((m, n)) * 2).astype(np.float32)
    w = rng.standard_normal(n).astype(np.float32)
    y_ref, o_ref = orc.rms_norm(x, 1e-5, w)
    y, o, act = ops.rms_norm(gpu(x, dev), 1e-5, gpu(w, dev), quantize=True)
    y, o, a = y.cpu().numpy(), o.cpu().numpy(), act.cpu().numpy()
    assert rel_l2(y, y_ref) < 1e-6 and rel_l2(o, o_ref) < 1e-6
    # the fused quantization equals ggml's quantize_row_q8_0 (x86 rule) of the GPU's own o, byte for byte
    ref_blocks = orc.quantize_q8_0(o, orc.Q8_X86).reshape(m, n // 32, 34)
    qs = a[: m * n].view(np.int8).reshape(m, n // 32, 32)
    assert np.array_equal(qs, ref_blocks[:, :, 2:].view(np.int8))
    meta = a[m * n:].view(np.int32).reshape(m, n // 32, 2)
    d16 = orc.fp16_to_fp32(ref_blocks[:, :, 0].astype(np.uint16) | (ref_blocks[:, :, 1].astype(np.uint16) << 8))
    assert np.array_equal(meta[:, :, 0].view(np.float32), d16)
    y2 = ops.rms_norm(gpu(x, dev), 1e-5).cpu().numpy()
    assert np.array_equal(y2, y)
    # the quantized y * w alone (no y, no o stored), Q8_0 and Q8_K: the same bytes as quantizing the stored o
    from ameva_compute_amd._lib import lib
    for at, bs in ((ops.Q8_0, 32), (ops.Q8_K, 256)):
        if n % bs:
            continue
        act2 = torch.empty(lib().amv_act_bytes(at, m, n), dtype=torch.uint8, device=dev)
        xg, wg = gpu(x, dev), gpu(w, dev)
        assert lib().amv_rms_norm_act(xg.data_ptr(), m, n, 1e-5, wg.data_ptr(), None, None, act2.data_ptr(), at,
                                      ops.Q8_X86, ops._stream()) == 0
        ref, _ = ops.quantize_act(gpu(o, dev), at, ops.Q8_X86)
        assert torch.equal(act2, ref)


# ---------------------------------------------------------------------------------------------- ROPE
@pytest.mark.parametrize("mode", [0, 2])
@pytest.mark.parametrize("n_head,ne0,n_dims", [(32, 128, 128), (8, 128, 128), (4, 64, 32)])
def test_rope(dev, ops, orc, mode, n_head, ne0, n_dims):
    rng = np.random.default_rng(n_head + ne0 + mode)
    pos = np.array([0, 1, 5, 511, 4095, 70000], np.int32)
    x = rng.standard_normal((len(pos), n_head, ne0)).astype(np.float32)
    y_ref = orc.rope(x, pos, n_dims, mode, 500000.0)
    xg = gpu(x, dev)
    y = ops.rope(xg, gpu(pos, dev), n_dims, mode, 500000.0).cpu().numpy()
    assert rel_l2(y, y_ref) < 1e-5
    assert np.array_equal(y[0], x[0])
    ops.rope(xg, gpu(pos, dev), n_dims, mode, 500000.0, out=xg)  # in place
    assert np.array_equal(xg.cpu().numpy(), y)


def test_swiglu(dev, ops, orc):
    rng = np.random.default_rng(12)
    g = (rng.standard_normal(14336) * 5).astype(np.float32)
    u = rng.standard_normal(14336).astype(np.float32)
    y = ops.swiglu(gpu(g, dev), gpu(u, dev)).cpu().numpy()
    assert rel_l2(y, orc.swiglu(g, u)) < 1e-6


@pytest.mark.parametrize("n_rows,F,act_type,offset", [(512, 14336, "Q8_0", 0), (512, 14336, "Q8_K", 0),
                                                       (7, 512, "Q8_K", 0), (9, 96, "Q8_0", 0), (5, 96, "Q8_0", 1)])
def test_swiglu_rows_quantized(dev, ops, orc, n_rows, F, act_type, offset):
    """SWIGLU over the two halves of a stacked gate|up output with the activation of the next MUL_MAT fused: y within
    1e-6 of the oracle, the Q8_0 / Q8_K bytes equal amv_quantize_act of y (offset 1: rows not 16-byte aligned, the
    one-element-per-thread kernel)."""
    at = getattr(ops, act_type)
    rng = np.random.default_rng(n_rows + F + offset)
    gu = (rng.standard_normal((n_rows, 2 * F + offset)) * 3).astype(np.float32)
    t = gpu(gu, dev)
    g, u = t[:, offset:offset + F], t[:, offset + F:]
    y, act = ops.swiglu_rows(g, u, quantize=True, act_type=at)
    assert rel_l2(y.cpu().numpy(), orc.swiglu(gu[:, offset:offset + F], gu[:, offset + F:])) < 1e-6
    ref, _ = ops.quantize_act(y, at, ops.Q8_X86)
    assert torch.equal(act, ref)


# ---------------------------------------------------------------------------------------------- FA decode
@pytest.mark.parametrize("n_head,n_head_kv,n_kv,stride", [(32, 8, 4096, 4096), (32, 8, 1000, 4096), (8, 8, 17, 64),
                                                          (16, 8, 300, 300), (8, 1, 1, 8), (32, 4, 2049, 2100)])
def test_flash_attn_decode(dev, ops, orc, n_head, n_head_kv, n_kv, stride):
    rng = np.random.default_rng(n_head * 31 + n_kv)
    D = 128
    q = rng.standard_normal((n_head, D)).astype(np.float32)
    k = rng.standard_normal((n_head_kv, stride, D)).astype(np.float16)
    v = rng.standard_normal((n_head_kv, stride, D)).astype(np.float16)
    scale = 1.0 / np.sqrt(D)
    ref = orc.flash_attn_decode(q, k[:, :n_kv].view(np.uint16), v[:, :n_kv].view(np.uint16), scale)
    out = ops.flash_attn_decode(gpu(q, dev), gpu(k.view(np.uint16), dev).view(torch.float16),
                                gpu(v.view(np.uint16), dev).view(torch.float16), scale, n_kv=n_kv).cpu().numpy()
    assert rel_l2(out, ref) < TOL_FA
    # llama.cpp's token-major cache [kv_size][n_head_kv][D] viewed per head: same result
    kt = gpu(np.ascontiguousarray(k.transpose(1, 0, 2)), dev)
    vt = gpu(np.ascontiguousarray(v.transpose(1, 0, 2)), dev)
    out_t = ops.flash_attn_decode(gpu(q, dev), kt.permute(1, 0, 2), vt.permute(1, 0, 2), scale, n_kv=n_kv).cpu().numpy()
    assert np.array_equal(out_t, out)


def test_flash_attn_decode_fused_quant(dev, ops, orc):
    """The Q8_0 output of the combine equals ggml's quantize_row_q8_0 of the attention output, byte for byte."""
    rng = np.random.default_rng(8)
    n_head, n_head_kv, n_kv, D = 32, 8, 777, 128
    q = rng.standard_normal((n_head, D)).astype(np.float32)
    k = rng.standard_normal((n_head_kv, n_kv, D)).astype(np.float16)
    v = rng.standard_normal((n_head_kv, n_kv, D)).astype(np.float16)
    act = torch.empty(ops.lib().amv_act_bytes(ops.Q8_0, 1, n_head * D), dtype=torch.uint8, device=dev)
    out = ops.flash_attn_decode(gpu(q, dev), gpu(k, dev), gpu(v, dev), 0.0884, act=act).cpu().numpy()
    ref = orc.quantize_q8_0(out.reshape(1, -1), orc.Q8_X86).reshape(-1, 34)
    a = act.cpu().numpy()
    assert np.array_equal(a[: n_head * D].view(np.int8).reshape(-1, 32), ref[:, 2:].view(np.int8))
    d16 = orc.fp16_to_fp32(ref[:, 0].astype(np.uint16) | (ref[:, 1].astype(np.uint16) << 8))
    assert np.array_equal(a[n_head * D:].view(np.int32).reshape(-1, 2)[:, 0].view(np.float32), d16)


def test_flash_attn_decode_mask(dev, ops, orc):
    rng = np.random.default_rng(99)
    n_head, n_head_kv, n_kv, D = 32, 8, 1024, 128
    q = rng.standard_normal((n_head, D)).astype(np.float32)
    k = rng.standard_normal((n_head_kv, n_kv, D)).astype(np.float16)
    v = rng.standard_normal((n_head_kv, n_kv, D)).astype(np.float16)
    mask = np.zeros(n_kv, np.float16)
    mask[700:] = -np.inf          # padding of the cache: whole splits masked out
    mask[::7] = -1.5
    scale = 1.0 / np.sqrt(D)
    ref = orc.flash_attn_decode(q, k.view(np.uint16), v.view(np.uint16), scale, mask.view(np.uint16))
    out = ops.flash_attn_decode(gpu(q, dev), gpu(k, dev), gpu(v, dev), scale, mask=gpu(mask, dev)).cpu().numpy()
    assert rel_l2(out, ref) < TOL_FA


def test_glue_ops(dev, ops, orc):
    rng = np.random.default_rng(5)
    a = rng.standard_normal((7, 4096)).astype(np.float32)
    b = rng.standard_normal((1, 4096)).astype(np.float32)
    assert np.array_equal(ops.add(gpu(a, dev), gpu(b, dev)).cpu().numpy(), a + b)
    assert np.array_equal(ops.mul(gpu(a, dev), gpu(b, dev)).cpu().numpy(), a * b)
    cache = torch.zeros((16, 1024), dtype=torch.float16, device=dev)
    src = rng.standard_normal((3, 1024)).astype(np.float32)
    idx = torch.tensor([5, 0, 15], dtype=torch.int64, device=dev)
    ops.set_rows_f16(cache, gpu(src, dev), idx)
    c = cache.cpu().numpy()
    assert np.array_equal(c[[5, 0, 15]].view(np.uint16), orc.fp32_to_fp16(src))
    assert not c[1:5].any()
    with pytest.raises(IndexError):
        ops.set_rows_f16(cache, gpu(src, dev), torch.tensor([5, 16, 0], dtype=torch.int64, device=dev))
    emb = (rng.standard_normal((50, 256)) * 0.02).astype(np.float32)
    embq = orc.quantize_q4_0(emb)
    ids = np.array([3, 49, 0, 3], np.int32)
    got = ops.get_rows(gpu(embq, dev), ops.Q4_0, 256, gpu(ids, dev)).cpu().numpy()
    assert np.array_equal(got, orc.dequantize(ops.Q4_0, embq, 256)[ids])


# ---------------------------------------------------------------------------------------------- GEMV epilogues
def _weight(rng, orc, t, n, k):
    if t in (12, 14):
        return random_kquant(rng, t, n, k)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    return orc.quantize_q4_0(w) if t == 2 else orc.quantize_q8_0(w, orc.Q8_REF)


@pytest.mark.parametrize("wtype", [2, 8, 12, 14])
@pytest.mark.parametrize("n,k", [(37, 512), (4096, 4096), (2 * 14336, 4096)])
def test_gemv_epilogues(dev, ops, orc, wtype, n, k):
    """Each epilogue's output equals the separate node applied to the plain GEMV's value: ADD bit for bit (the same
    f32 addition), the SWIGLU forms within 1e-6 of the oracle's silu (expf of the GPU against the CPU's); the
    write-through dst equals the plain GEMV bit for bit."""
    rng = np.random.default_rng(n + k + wtype)
    wg = _weight(rng, orc, wtype, n, k)
    w = ops.QWeight.from_ggml(wtype, gpu(wg, dev), n, k)
    x = rng.standard_normal((1, k)).astype(np.float32)
    act, _ = ops.quantize_act(gpu(x, dev), ops.act_type(wtype), ops.Q8_X86)
    v = ops.mul_mat_q(w, act, 1, kernel="mmv").reshape(-1)
    vn = v.cpu().numpy()
    e = (rng.standard_normal(n) * 3).astype(np.float32)
    eg = gpu(e, dev)
    d, o = ops.mul_mat_vec_ep(w, act, ops.EP_ADD, eg)
    assert torch.equal(d, v) and np.array_equal(o.cpu().numpy(), vn + e)
    d, o = ops.mul_mat_vec_ep(w, act, ops.EP_SILU_MUL, eg, write_dst=False)
    assert d is None and rel_l2(o.cpu().numpy(), orc.swiglu(vn, e)) < 1e-6
    d, o = ops.mul_mat_vec_ep(w, act, ops.EP_MUL_SILU, eg)
    assert torch.equal(d, v) and rel_l2(o.cpu().numpy(), orc.swiglu(e, vn)) < 1e-6
    F = n // 2
    if n % 2 == 0:
        d, o = ops.mul_mat_vec_ep(w, act, ops.EP_SWIGLU_STACKED)
        assert torch.equal(d, v) and o.numel() == F
        assert rel_l2(o.cpu().numpy(), orc.swiglu(vn[:F], vn[F:])) < 1e-6
        # the stacked form against the graph's two MUL_MATs + SWIGLU, and the epilogue against amv_swiglu
        assert torch.equal(o, ops.swiglu(v[:F].contiguous(), v[F:].contiguous()))
    d, o0 = ops.mul_mat_vec_ep(w, act, ops.EP_NONE)
    assert torch.equal(d, v) and o0 is d


def test_gemv_epilogue_errors(dev, ops, orc):
    from ameva_compute_amd._lib import AmevaError
    rng = np.random.default_rng(3)
    w = ops.QWeight.from_ggml(2, gpu(_weight(rng, orc, 2, 33, 64), dev), 33, 64)
    act, _ = ops.quantize_act(gpu(rng.standard_normal((1, 64)).astype(np.float32), dev), ops.Q8_0, ops.Q8_X86)
    with pytest.raises(AmevaError, match="even number of rows"):
        ops.mul_mat_vec_ep(w, act, ops.EP_SWIGLU_STACKED)
    with pytest.raises(AmevaError, match="needs its operand"):
        ops.mul_mat_vec_ep(w, act, ops.EP_ADD)
    with pytest.raises(AmevaError, match="unknown"):
        ops.mul_mat_vec_ep(w, act, 9)


# ---------------------------------------------------------------------------------------------- ROPE + KV store
@pytest.mark.parametrize("mode", [0, 2])
@pytest.mark.parametrize("n_head,n_head_kv,D,n_tok", [(32, 8, 128, 1), (32, 8, 128, 5), (8, 2, 64, 3),
                                                      (32, 8, 128, 512), (4, 1, 256, 40)])
def test_rope_kv_store(dev, ops, orc, mode, n_head, n_head_kv, D, n_tok):
    """Equals amv_rope followed by the two SET_ROWS bit for bit, and the oracle's rope within 1e-5 (512 tokens: a
    prefill chunk, every head of a token in one workgroup)."""
    rng = np.random.default_rng(n_head + D + n_tok + mode)
    CTX = max(64, n_tok)
    n_all = n_head + 2 * n_head_kv
    kvw = n_head_kv * D
    pos = rng.integers(0, 100000, n_tok).astype(np.int32)
    idx = rng.permutation(CTX)[:n_tok].astype(np.int64)
    x = rng.standard_normal((n_tok, n_all, D)).astype(np.float32)
    kc0 = rng.standard_normal((CTX, kvw)).astype(np.float16)
    vc0 = rng.standard_normal((CTX, kvw)).astype(np.float16)
    base = 500000.0
    # fused
    qkv = gpu(x, dev)
    kc, vc = gpu(kc0, dev), gpu(vc0, dev)
    ops.rope_kv_store(qkv, gpu(pos, dev), n_head, n_head_kv, kc, vc, gpu(idx, dev), D, mode, base)
    # unfused: ROPE of the q and k heads, then SET_ROWS of k and v
    qk = gpu(x[:, :n_head + n_head_kv], dev)
    qk_r = ops.rope(qk, gpu(pos, dev), D, mode, base)
    kc2, vc2 = gpu(kc0, dev), gpu(vc0, dev)
    ops.set_rows_f16(kc2, qk_r[:, n_head:].reshape(n_tok, kvw).contiguous(), gpu(idx, dev))
    ops.set_rows_f16(vc2, gpu(x[:, n_head + n_head_kv:].reshape(n_tok, kvw), dev), gpu(idx, dev))
    assert torch.equal(qkv[:, :n_head + n_head_kv], qk_r)
    assert torch.equal(qkv[:, n_head + n_head_kv:], gpu(x[:, n_head + n_head_kv:], dev))
    assert torch.equal(kc, kc2) and torch.equal(vc, vc2)
    ref = orc.rope(x[:, :n_head + n_head_kv], pos, D, mode, base)
    assert rel_l2(qkv[:, :n_head + n_head_kv].cpu().numpy(), ref) < 1e-5
    untouched = np.setdiff1d(np.arange(CTX), idx)
    assert np.array_equal(kc.cpu().numpy()[untouched].view(np.uint16), kc0[untouched].view(np.uint16))


@pytest.mark.parametrize("n_dims", [128, 64])
def test_rope_kv_store_strided_cache(dev, ops, n_dims):
    """A cache of odd row stride (f16 pairs stored as halfwords) and partial rotation (n_dims < D) give the same
    values as a contiguous cache."""
    n_head, n_head_kv, D, n_tok, CTX = 8, 2, 128, 9, 16
    kvw = n_head_kv * D
    x = torch.randn((n_tok, n_head + 2 * n_head_kv, D), device=dev)
    pos = torch.arange(100, 100 + n_tok, dtype=torch.int32, device=dev)
    idx = torch.arange(n_tok, dtype=torch.int64, device=dev) + 3
    kc = torch.zeros((CTX, kvw), dtype=torch.float16, device=dev)
    vc = torch.zeros_like(kc)
    q1 = x.clone()
    ops.rope_kv_store(q1, pos, n_head, n_head_kv, kc, vc, idx, n_dims, 0, 500000.0)
    kb = torch.zeros((CTX, kvw + 1), dtype=torch.float16, device=dev)
    vb = torch.zeros_like(kb)
    q2 = x.clone()
    ops.rope_kv_store(q2, pos, n_head, n_head_kv, kb[:, :kvw], vb[:, :kvw], idx, n_dims, 0, 500000.0)
    assert torch.equal(q1, q2)
    assert torch.equal(kb[:, :kvw], kc) and torch.equal(vb[:, :kvw], vc) and not kb[:, kvw].any()
    if n_dims < D:  # elements past n_dims are not rotated
        assert torch.equal(q1[:, :n_head + n_head_kv, n_dims:], x[:, :n_head + n_head_kv, n_dims:])


def test_rope_kv_store_bad_index(dev, ops):
    n_head, n_head_kv, D = 4, 2, 64
    qkv = torch.randn((1, n_head + 2 * n_head_kv, D), device=dev)
    kc = torch.zeros((8, n_head_kv * D), dtype=torch.float16, device=dev)
    vc = torch.zeros_like(kc)
    bad = torch.zeros(1, dtype=torch.int32, device=dev)
    ops.rope_kv_store(qkv, torch.tensor([3], dtype=torch.int32, device=dev), n_head, n_head_kv, kc, vc,
                      torch.tensor([8], dtype=torch.int64, device=dev), bad=bad)
    # one k head and one v head of each of the n_head_kv heads count the skipped row
    assert int(bad.item()) == 2 * n_head_kv
    assert not kc.any() and not vc.any()


# ---------------------------------------------------------------------------------------------- FA prefill
@pytest.mark.parametrize("n_tok,n_head,n_head_kv,n_kv,pos0,layout", [
    (512, 32, 8, 512, 0, "token"),      # config 4 prompt: 512 tokens from position 0
    (100, 8, 2, 300, 200, "token"),     # chunk of a longer prompt (tail tile, keys before the chunk)
    (64, 8, 1, 1000, -1, "head"),       # no causal limit, GQA 8, head-major cache
    (1, 4, 4, 1, 0, "head"),            # one token
    (45, 8, 4, 45, 0, "token"),         # GQA 2 (waves past the group's heads idle), partial tiles
])
def test_flash_attn_prefill(dev, ops, orc, n_tok, n_head, n_head_kv, n_kv, pos0, layout):
    rng = np.random.default_rng(n_tok + n_kv)
    D = 128
    q = rng.standard_normal((n_tok, n_head, D)).astype(np.float32)
    kh = orc.fp32_to_fp16(rng.standard_normal((n_head_kv, n_kv, D)))
    vh = orc.fp32_to_fp16(rng.standard_normal((n_head_kv, n_kv, D)))
    scale = 1.0 / np.sqrt(D)
    ref = orc.flash_attn_prefill(q, kh, vh, scale, causal_pos0=pos0)
    if layout == "token":  # llama.cpp cache [kv_size][n_head_kv * D], viewed head-major
        kt = gpu(np.ascontiguousarray(kh.transpose(1, 0, 2)), dev).view(torch.float16)
        vt = gpu(np.ascontiguousarray(vh.transpose(1, 0, 2)), dev).view(torch.float16)
        kg, vg = kt.permute(1, 0, 2), vt.permute(1, 0, 2)
    else:
        kg, vg = gpu(kh, dev).view(torch.float16), gpu(vh, dev).view(torch.float16)
    out = ops.flash_attn_prefill(gpu(q, dev), kg, vg, scale, causal_pos0=pos0).cpu().numpy()
    assert rel_l2(out, ref) < TOL_FA


def test_flash_attn_prefill_mask_and_fused_qkv_rows(dev, ops, orc):
    """ggml's KQ mask path (f16, -inf above the diagonal plus finite biases) and q read in place from fused q/k/v rows
    (token stride (n_head + 2 n_head_kv) * D)."""
    rng = np.random.default_rng(4)
    n_tok, n_head, n_head_kv, D = 70, 8, 2, 128
    n_kv = n_tok
    qkv = rng.standard_normal((n_tok, n_head + 2 * n_head_kv, D)).astype(np.float32)
    kh = orc.fp32_to_fp16(rng.standard_normal((n_head_kv, n_kv, D)))
    vh = orc.fp32_to_fp16(rng.standard_normal((n_head_kv, n_kv, D)))
    mf = (rng.standard_normal((n_tok, 80)) * 0.5).astype(np.float32)
    mf[np.triu_indices(n_tok, 1, 80)] = -np.inf
    mask = orc.fp32_to_fp16(mf)
    ref = orc.flash_attn_prefill(qkv[:, :n_head], kh, vh, 0.1, mask=mask[:, :n_kv])
    qg = gpu(qkv, dev)[:, :n_head]
    out = ops.flash_attn_prefill(qg, gpu(kh, dev).view(torch.float16), gpu(vh, dev).view(torch.float16), 0.1,
                                 mask=gpu(mask, dev).view(torch.float16)).cpu().numpy()
    assert rel_l2(out, ref) < TOL_FA
