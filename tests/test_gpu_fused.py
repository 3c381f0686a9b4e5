"""The fused decode launches against the unfused launches they replace, through the C ABI:
  GEMV + ROPE + KV stores (amv_gemv_rope_kv), GEMV + ADD + RMS_NORM + quantization (amv_gemv_add_rms_norm), stacked
  gate/up GEMV + SWIGLU + quantization (amv_gemv_swiglu_q8), FA decode with the split merge in its last workgroups
  and the key count read from device memory (amv_flash_attn_decode_ex).
Bar: identical bits (the fused kernels run the same arithmetic; the arrival counters only move work between
workgroups), Q8_0 and Q8_K activation rows included; every call is made twice on the same counters, which must have
reset themselves. The unfused ops are pinned against the oracle in test_gpu_ops / test_gpu_mmv."""
import numpy as np
import pytest

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


def weight(rng, orc, t, n, k):
    if t in (12, 14):
        bb = 144 if t == 12 else 210
        y = rng.integers(0, 256, (n, k // 256, bb), dtype=np.uint8)
        for off in ((0, 2) if t == 12 else (208,)):
            v = rng.uniform(0.0, 0.002, (n, k // 256)).astype(np.float16)
            y[:, :, off:off + 2] = v.view(np.uint8).reshape(n, k // 256, 2)
        return y.reshape(n, -1)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    return orc.quantize_q4_0(w) if t == 2 else orc.quantize_q8_0(w, orc.Q8_REF)


def act_of(ops, x, t):
    return ops.quantize_act(x.reshape(1, -1).contiguous(), t, ops.Q8_X86)[0]


# (weight type, n_rows, k, activation type of the output): Llama shapes, a K split over the waves of a workgroup
# (few rows), an odd row count, the K-quants with Q8_K outputs
ADD_NORM_CASES = [(2, 4096, 4096, 8), (2, 4096, 14336, 8), (12, 4096, 14336, 15), (14, 512, 256, 15),
                  (8, 96, 128, 8), (2, 256, 512, 15), (12, 1024, 4096, 8), (2, 128, 8192, 8)]


@pytest.mark.parametrize("wtype,n,k,act_t", ADD_NORM_CASES)
def test_gemv_add_rms_norm(dev, ops, orc, wtype, n, k, act_t):
    rng = np.random.default_rng(n + k + act_t)
    w = ops.QWeight.from_ggml(wtype, gpu(weight(rng, orc, wtype, n, k), dev), n, k)
    x = gpu(rng.standard_normal(k).astype(np.float32), dev)
    act = act_of(ops, x, ops.act_type(wtype))
    e = gpu((rng.standard_normal(n) * 2).astype(np.float32), dev)
    nw = gpu((1 + 0.1 * rng.standard_normal(n)).astype(np.float32), dev)
    cnt = torch.zeros(ops.add_norm_counter_words(n), dtype=torch.int32, device=dev)
    # unfused: GEMV, ADD, RMS_NORM + MUL, quantization
    v_ref = ops.mul_mat_q(w, act, 1, kernel="mmv").reshape(-1)
    eo_ref = ops.add(v_ref.reshape(1, -1), e.reshape(1, -1)).reshape(-1)
    y_ref, o_ref = ops.rms_norm(eo_ref, 1e-5, nw)
    a_ref = act_of(ops, o_ref, act_t)
    for _ in range(2):
        v, eo, y, o, a = ops.gemv_add_rms_norm(w, act, e, 1e-5, nw, act_t, counters=cnt)
        torch.cuda.synchronize()
        assert torch.equal(v, v_ref) and torch.equal(eo, eo_ref)
        assert torch.equal(y, y_ref.reshape(-1)) and torch.equal(o, o_ref.reshape(-1))
        assert torch.equal(a, a_ref)
        assert not cnt.any()


@pytest.mark.parametrize("wtype,F,k,act_t", [(2, 14336, 4096, 8), (12, 14336, 4096, 15), (8, 64, 256, 8),
                                             (14, 256, 512, 15), (2, 32, 64, 8), (12, 512, 256, 15),
                                             (2, 64, 8192, 8), (12, 256, 8192, 15), (12, 8192, 256, 15)])
def test_gemv_swiglu_act(dev, ops, orc, wtype, F, k, act_t):
    rng = np.random.default_rng(F + k + wtype)
    n = 2 * F
    w = ops.QWeight.from_ggml(wtype, gpu(weight(rng, orc, wtype, n, k), dev), n, k)
    act = act_of(ops, gpu(rng.standard_normal(k).astype(np.float32), dev), ops.act_type(wtype))
    v_ref, h_ref = ops.mul_mat_vec_ep(w, act, ops.EP_SWIGLU_STACKED)
    # the stacked launches (1 or, from 16384 rows, 2 outputs per wave) sum every row as the plain GEMV does
    assert torch.equal(v_ref, ops.mul_mat_q(w, act, 1, kernel="mmv").reshape(-1))
    a_ref = act_of(ops, h_ref, act_t)
    cnt = torch.zeros(ops.swiglu_counter_words(n), dtype=torch.int32, device=dev)
    for _ in range(2):
        v, h, a = ops.gemv_swiglu_act(w, act, act_t, counters=cnt)
        torch.cuda.synchronize()
        assert torch.equal(v, v_ref) and torch.equal(h, h_ref) and torch.equal(a, a_ref)
        assert not cnt.any()


@pytest.mark.parametrize("wtype", [2, 12])
@pytest.mark.parametrize("n_head,n_head_kv,D", [(32, 8, 128), (8, 2, 64)])
def test_gemv_rope_kv(dev, ops, orc, wtype, n_head, n_head_kv, D):
    rng = np.random.default_rng(n_head + D + wtype)
    H = 4096 if wtype == 2 else 512
    n = (n_head + 2 * n_head_kv) * D
    kv = n_head_kv * D
    w = ops.QWeight.from_ggml(wtype, gpu(weight(rng, orc, wtype, n, H), dev), n, H)
    act = act_of(ops, gpu(rng.standard_normal(H).astype(np.float32), dev), ops.act_type(wtype))
    CTX = 40
    kc = gpu(rng.standard_normal((CTX, kv)).astype(np.float16), dev)
    vc = gpu(rng.standard_normal((CTX, kv)).astype(np.float16), dev)
    pos = torch.tensor([12345], dtype=torch.int32, device=dev)
    idx = torch.tensor([17], dtype=torch.int64, device=dev)
    # unfused: GEMV, then ROPE + both SET_ROWS
    qkv_ref = ops.mul_mat_q(w, act, 1, kernel="mmv").reshape(-1)
    kc_ref, vc_ref = kc.clone(), vc.clone()
    ops.rope_kv_store(qkv_ref.reshape(1, n_head + 2 * n_head_kv, D), pos, n_head, n_head_kv, kc_ref, vc_ref, idx,
                      freq_base=500000.0)
    qkv = ops.gemv_rope_kv(w, act, n_head, n_head_kv, pos, kc, vc, idx)
    torch.cuda.synchronize()
    assert torch.equal(qkv, qkv_ref.reshape(-1))
    assert torch.equal(kc.view(torch.int16), kc_ref.view(torch.int16))
    assert torch.equal(vc.view(torch.int16), vc_ref.view(torch.int16))
    # a cache row outside the cache: nothing stored, one count per k and v head
    bad = torch.zeros(1, dtype=torch.int32, device=dev)
    kc2, vc2 = kc.clone(), vc.clone()
    ops.gemv_rope_kv(w, act, n_head, n_head_kv, pos, kc2, vc2, torch.tensor([CTX], dtype=torch.int64, device=dev),
                     bad=bad)
    torch.cuda.synchronize()
    assert torch.equal(kc2, kc) and torch.equal(vc2, vc) and int(bad.item()) == 2 * n_head_kv


@pytest.mark.parametrize("n_head,n_head_kv,n_kv_max,n_kv,act_t", [(32, 8, 4096, 4096, 8), (32, 8, 4096, 3001, 15),
                                                                  (32, 8, 1024, 1, 8), (8, 8, 300, 257, 8),
                                                                  (16, 2, 9000, 8191, 15), (8, 1, 64, 50, 8),
                                                                  (64, 8, 2048, 1999, 15)])
def test_flash_attn_decode_ex(dev, ops, orc, n_head, n_head_kv, n_kv_max, n_kv, act_t):
    """Key count from device memory, split merge as a second launch or in the split's last workgroups: both equal
    amv_flash_attn_decode at that key count, and their Q8_0 / Q8_K rows equal amv_quantize_act of the output."""
    rng = np.random.default_rng(n_head + n_kv)
    D = 128
    q = gpu(rng.standard_normal((n_head, D)).astype(np.float32), dev)
    k = gpu(rng.standard_normal((n_kv_max, n_head_kv * D)).astype(np.float16), dev)
    v = gpu(rng.standard_normal((n_kv_max, n_head_kv * D)).astype(np.float16), dev)
    kh = k.view(n_kv_max, n_head_kv, D).permute(1, 0, 2)
    vh = v.view(n_kv_max, n_head_kv, D).permute(1, 0, 2)
    scale = 1.0 / np.sqrt(D)
    ref = ops.flash_attn_decode(q, kh, vh, scale, n_kv=n_kv)
    a_ref = act_of(ops, ref, act_t)
    nkd = torch.tensor([n_kv], dtype=torch.int32, device=dev)
    cnt = torch.zeros(32 * n_head_kv, dtype=torch.int32, device=dev)
    act = torch.empty(ops.lib().amv_act_bytes(act_t, 1, n_head * D), dtype=torch.uint8, device=dev)
    for one in (False, True, True):
        act.zero_()
        out = ops.flash_attn_decode_ex(q, kh, vh, scale, n_kv_max, nkd, act=act, act_t=act_t, counters=cnt,
                                       one_launch=one)
        torch.cuda.synchronize()
        assert torch.equal(out, ref), one
        assert torch.equal(act, a_ref), one
        assert not cnt.any()
    # without n_kv_dev the launch's n_kv_max keys are used
    full = ops.flash_attn_decode_ex(q, kh, vh, scale, n_kv_max, None)
    assert torch.equal(full, ops.flash_attn_decode(q, kh, vh, scale, n_kv=n_kv_max))


@pytest.mark.parametrize("wtype", [2, 12])
@pytest.mark.parametrize("n_head,n_head_kv,D", [(32, 8, 128), (8, 2, 64)])
def test_gemv_rope_kv_seg(dev, ops, orc, wtype, n_head, n_head_kv, D):
    """q, k, v as three matrices (each repacked on its own, as the plugin holds separate ggml weights): the same bits
    as the stacked launch over their rows, in the three outputs and both cache rows."""
    rng = np.random.default_rng(n_head * 3 + D + wtype)
    H = 4096 if wtype == 2 else 512
    n = (n_head + 2 * n_head_kv) * D
    nq, kv = n_head * D, n_head_kv * D
    wg = weight(rng, orc, wtype, n, H)
    w = ops.QWeight.from_ggml(wtype, gpu(wg, dev), n, H)
    parts = [ops.QWeight.from_ggml(wtype, gpu(np.ascontiguousarray(wg[a:b]), dev), b - a, H)
             for a, b in ((0, nq), (nq, nq + kv), (nq + kv, n))]
    act = act_of(ops, gpu(rng.standard_normal(H).astype(np.float32), dev), ops.act_type(wtype))
    CTX = 40
    kc = gpu(rng.standard_normal((CTX, kv)).astype(np.float16), dev)
    vc = gpu(rng.standard_normal((CTX, kv)).astype(np.float16), dev)
    kc_ref, vc_ref = kc.clone(), vc.clone()
    pos = torch.tensor([777], dtype=torch.int32, device=dev)
    idx = torch.tensor([5], dtype=torch.int64, device=dev)
    qkv_ref = ops.gemv_rope_kv(w, act, n_head, n_head_kv, pos, kc_ref, vc_ref, idx)
    outs = [torch.empty(p.n_rows, dtype=torch.float32, device=dev) for p in parts]
    lib = ops.lib()
    rc = lib.amv_gemv_rope_kv_seg(wtype, parts[0].data.data_ptr(), parts[1].data.data_ptr(), parts[2].data.data_ptr(),
                                  H, act.data_ptr(), outs[0].data_ptr(), outs[1].data_ptr(), outs[2].data_ptr(),
                                  n_head, n_head_kv, D, pos.data_ptr(), 500000.0, 1.0, 1.0, kc.data_ptr(),
                                  vc.data_ptr(), kv, idx.data_ptr(), CTX, None, torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.amv_last_error()
    torch.cuda.synchronize()
    assert torch.equal(torch.cat(outs), qkv_ref)
    assert torch.equal(kc.view(torch.int16), kc_ref.view(torch.int16))
    assert torch.equal(vc.view(torch.int16), vc_ref.view(torch.int16))


@pytest.mark.parametrize("wtype,F,k,act_t", [(2, 14336, 4096, 8), (12, 14336, 4096, 15), (2, 64, 4096, 8),
                                             (12, 512, 256, 15)])
def test_gemv_swiglu_act_seg(dev, ops, orc, wtype, F, k, act_t):
    """gate and up as two matrices: the same SWIGLU values and activation row as the stacked launch."""
    rng = np.random.default_rng(F + k + wtype + 1)
    wg = weight(rng, orc, wtype, 2 * F, k)
    w = ops.QWeight.from_ggml(wtype, gpu(wg, dev), 2 * F, k)
    wgate = ops.QWeight.from_ggml(wtype, gpu(np.ascontiguousarray(wg[:F]), dev), F, k)
    wup = ops.QWeight.from_ggml(wtype, gpu(np.ascontiguousarray(wg[F:]), dev), F, k)
    act = act_of(ops, gpu(rng.standard_normal(k).astype(np.float32), dev), ops.act_type(wtype))
    _, h_ref, a_ref = ops.gemv_swiglu_act(w, act, act_t)
    h = torch.empty(F, dtype=torch.float32, device=dev)
    a = torch.empty(ops.lib().amv_act_bytes(act_t, 1, F), dtype=torch.uint8, device=dev)
    cnt = torch.zeros(ops.swiglu_counter_words(2 * F), dtype=torch.int32, device=dev)
    lib = ops.lib()
    for _ in range(2):
        rc = lib.amv_gemv_swiglu_q8_seg(wtype, wgate.data.data_ptr(), wup.data.data_ptr(), F, k, act.data_ptr(),
                                        h.data_ptr(), a.data_ptr(), act_t, 0, cnt.data_ptr(),
                                        torch.cuda.current_stream().cuda_stream)
        assert rc == 0, lib.amv_last_error()
        torch.cuda.synchronize()
        assert torch.equal(h, h_ref) and torch.equal(a, a_ref)
        assert not cnt.any()
