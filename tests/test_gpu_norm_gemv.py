"""The decode GEMVs with the RMS_NORM before them folded in (amv_rms_norm_gemv_rope_kv, amv_rms_norm_gemv_swiglu_q8 and
their _seg forms over separate matrices) against the two launches they replace: amv_rms_norm_act (RMS_NORM * norm_w +
Q8_0 for Q4_0 weights, Q8_K for Q4_K), then amv_gemv_rope_kv / amv_gemv_swiglu_q8 over that activation. Bar:
identical bits in every output (qkv, both cache rows, the gate/up values, SWIGLU and its Q8_0 / Q8_K row), for each
workgroup size, each Q8_0 rounding rule and inputs whose norm is tiny, large or has exact zeros; every call twice on
the same counters, which must reset themselves. The two-launch path is pinned against the oracle in test_gpu_ops /
test_gpu_fused."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

H = 4096


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


def q4_weight(ops, orc, rng, n, dev, wt=2):
    if wt == 12:  # random Q4_K blocks, d and dmin in [0, 2e-3)
        y = rng.integers(0, 256, (n, H // 256, 144), dtype=np.uint8)
        for off in (0, 2):
            v = rng.uniform(0.0, 0.002, (n, H // 256)).astype(np.float16)
            y[:, :, off:off + 2] = v.view(np.uint8).reshape(n, H // 256, 2)
        return ops.QWeight.from_ggml(12, gpu(y.reshape(n, -1), dev), n, H)
    w = (rng.standard_normal((n, H)) * 0.02).astype(np.float32)
    return ops.QWeight.from_ggml(2, gpu(orc.quantize_q4_0(w), dev), n, H)


def row(rng, kind):
    x = rng.standard_normal(H).astype(np.float32)
    if kind == "tiny":
        x *= 1e-4
    elif kind == "large":
        x *= 300.0
    elif kind == "zeros":
        x[::3] = 0.0
        x[1000:1100] = 0.0  # whole zero blocks: Q8_0 d = 0
    return x


def norm_act(ops, x, nw, eps, rule, atype=8):
    lib, st = ops.lib(), torch.cuda.current_stream().cuda_stream
    act = torch.empty(lib.amv_act_bytes(atype, 1, H), dtype=torch.uint8, device=x.device)
    o = torch.empty(H, dtype=torch.float32, device=x.device)
    ops.check(lib.amv_rms_norm_act(x.data_ptr(), 1, H, eps, nw.data_ptr(), None, o.data_ptr(), act.data_ptr(),
                                   atype, rule, st), "rms_norm")
    return act


@pytest.fixture(params=[0, 256, 512, 1024, -256, -512], ids=lambda t: f"nt{t}")
def threads(request, ops):
    ops.lib().amv_debug_norm_gemv_threads(request.param)
    yield request.param
    ops.lib().amv_debug_norm_gemv_threads(0)


@pytest.mark.parametrize("wt", [2, 12])
@pytest.mark.parametrize("kind,rule", [("normal", 0), ("tiny", 1), ("large", 2), ("zeros", 0)])
def test_norm_gemv_swiglu(dev, ops, orc, threads, wt, kind, rule):
    if wt == 12 and threads < 0:
        pytest.skip("four outputs per wave: the Q4_0 kernel's instrumentation")
    rng = np.random.default_rng(7 + rule + len(kind) + wt)
    # Q4_K: the Llama shape only (below ~8 K outputs the plain Q4_K launch splits K over waves, another f32 order)
    F = 14336 if kind == "normal" or wt == 12 else 1024
    n = 2 * F
    w = q4_weight(ops, orc, rng, n, dev, wt)
    at = ops.act_type(wt)
    x = gpu(row(rng, kind), dev)
    nw = gpu((1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32), dev)
    eps = 1e-5
    act = norm_act(ops, x, nw, eps, rule, at)
    v_ref, h_ref, a_ref = ops.gemv_swiglu_act(w, act, at, rule)
    lib, st = ops.lib(), torch.cuda.current_stream().cuda_stream
    cnt = torch.zeros(ops.swiglu_counter_words(n), dtype=torch.int32, device=dev)
    # the same rows as two matrices (llama.cpp's gate and up tensors)
    wg = ops.QWeight.from_ggml(wt, w.to_ggml().reshape(n, -1)[:F].contiguous(), F, H)
    wu = ops.QWeight.from_ggml(wt, w.to_ggml().reshape(n, -1)[F:].contiguous(), F, H)
    for seg in (False, True, False):
        v = torch.full_like(v_ref, float("nan"))
        h = torch.full_like(h_ref, float("nan"))
        a = torch.zeros_like(a_ref)
        if seg:
            ops.check(lib.amv_rms_norm_gemv_swiglu_q8_seg(x.data_ptr(), nw.data_ptr(), eps, rule, wt,
                                                          wg.data.data_ptr(), wu.data.data_ptr(), F, H, h.data_ptr(),
                                                          a.data_ptr(), cnt.data_ptr(), st), "norm + gate/up seg")
        else:
            ops.check(lib.amv_rms_norm_gemv_swiglu_q8(x.data_ptr(), nw.data_ptr(), eps, rule, wt, w.data.data_ptr(),
                                                      n, H, v.data_ptr(), h.data_ptr(), a.data_ptr(), cnt.data_ptr(),
                                                      st), "norm + gate/up")
        torch.cuda.synchronize()
        if not seg:
            assert torch.equal(v, v_ref)
        assert torch.equal(h, h_ref) and torch.equal(a, a_ref)
        assert not cnt.any()


@pytest.mark.parametrize("wt", [2, 12])
@pytest.mark.parametrize("n_head,n_head_kv,D,kind,rule", [(32, 8, 128, "normal", 0), (8, 2, 64, "large", 1),
                                                           (32, 8, 128, "zeros", 2)])
def test_norm_gemv_rope_kv(dev, ops, orc, threads, wt, n_head, n_head_kv, D, kind, rule):
    if threads < 0:
        pytest.skip("-NT changes the gate/up launches only")
    if wt == 12 and n_head != 32:
        pytest.skip("the plain Q4_K launch splits K over waves at this size: another f32 summation order")
    rng = np.random.default_rng(n_head + D + rule + wt)
    n = (n_head + 2 * n_head_kv) * D
    kv = n_head_kv * D
    w = q4_weight(ops, orc, rng, n, dev, wt)
    x = gpu(row(rng, kind), dev)
    nw = gpu((1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32), dev)
    eps = 1e-5
    CTX = 40
    kc = gpu(rng.standard_normal((CTX, kv)).astype(np.float16), dev)
    vc = gpu(rng.standard_normal((CTX, kv)).astype(np.float16), dev)
    pos = torch.tensor([4095], dtype=torch.int32, device=dev)
    idx = torch.tensor([23], dtype=torch.int64, device=dev)
    act = norm_act(ops, x, nw, eps, rule, ops.act_type(wt))
    kc_ref, vc_ref = kc.clone(), vc.clone()
    qkv_ref = ops.gemv_rope_kv(w, act, n_head, n_head_kv, pos, kc_ref, vc_ref, idx)
    lib, st = ops.lib(), torch.cuda.current_stream().cuda_stream
    gg = w.to_ggml().reshape(n, -1)
    nq = n_head * D
    parts = [ops.QWeight.from_ggml(wt, gg[a:b].contiguous(), b - a, H) for a, b in ((0, nq), (nq, nq + kv), (nq + kv, n))]
    for bad_row, seg in ((False, False), (True, False), (False, True)):
        qkv = torch.full_like(qkv_ref, float("nan"))
        kc2, vc2 = kc.clone(), vc.clone()
        bad = torch.zeros(1, dtype=torch.int32, device=dev)
        ix = torch.tensor([CTX], dtype=torch.int64, device=dev) if bad_row else idx
        if seg:
            o = [qkv[:nq], qkv[nq:nq + kv], qkv[nq + kv:]]
            ops.check(lib.amv_rms_norm_gemv_rope_kv_seg(x.data_ptr(), nw.data_ptr(), eps, rule, wt,
                                                        *[p_.data.data_ptr() for p_ in parts], H,
                                                        *[t.data_ptr() for t in o], n_head, n_head_kv, D,
                                                        pos.data_ptr(), 500000.0, 1.0, 1.0, kc2.data_ptr(),
                                                        vc2.data_ptr(), kv, ix.data_ptr(), CTX, bad.data_ptr(), st),
                      "norm + qkv seg")
        else:
            ops.check(lib.amv_rms_norm_gemv_rope_kv(x.data_ptr(), nw.data_ptr(), eps, rule, wt, w.data.data_ptr(), n,
                                                    H, qkv.data_ptr(), n_head, n_head_kv, D, pos.data_ptr(), 500000.0,
                                                    1.0, 1.0, kc2.data_ptr(), vc2.data_ptr(), kv, ix.data_ptr(), CTX,
                                                    bad.data_ptr(), st), "norm + qkv")
        torch.cuda.synchronize()
        assert torch.equal(qkv, qkv_ref)
        if bad_row:  # a cache row outside the cache: nothing stored, one count per k and v head
            assert torch.equal(kc2, kc) and torch.equal(vc2, vc) and int(bad.item()) == 2 * n_head_kv
        else:
            assert torch.equal(kc2.view(torch.int16), kc_ref.view(torch.int16))
            assert torch.equal(vc2.view(torch.int16), vc_ref.view(torch.int16))
            assert int(bad.item()) == 0


def test_norm_gemv_refuses_bad_shapes(dev, ops, orc):
    rng = np.random.default_rng(3)
    lib, st = ops.lib(), torch.cuda.current_stream().cuda_stream
    w = q4_weight(ops, orc, rng, 64, dev)
    x = torch.zeros(2 * H, dtype=torch.float32, device=dev)
    out = torch.empty(4096, dtype=torch.float32, device=dev)
    a = torch.empty(8192, dtype=torch.uint8, device=dev)
    cnt = torch.zeros(4096, dtype=torch.int32, device=dev)
    p = lambda t: t.data_ptr()  # noqa: E731
    # k other than 4096, a Q6_K weight, a row count that is not whole output blocks, a misaligned x
    assert lib.amv_rms_norm_gemv_swiglu_q8(p(x), p(x), 1e-5, 0, 2, p(w.data), 64, 2048, p(out), p(out), p(a),
                                           p(cnt), st) != 0
    assert lib.amv_rms_norm_gemv_swiglu_q8(p(x), p(x), 1e-5, 0, 14, p(w.data), 64, H, p(out), p(out), p(a),
                                           p(cnt), st) != 0
    assert lib.amv_rms_norm_gemv_swiglu_q8(p(x), p(x), 1e-5, 0, 12, p(w.data), 64, H, p(out), p(out), p(a),
                                           p(cnt), st) != 0  # Q4_K: F must be whole 256-blocks
    assert lib.amv_rms_norm_gemv_swiglu_q8(p(x), p(x), 1e-5, 0, 2, p(w.data), 96, H, p(out), p(out), p(a),
                                           p(cnt), st) != 0
    assert lib.amv_rms_norm_gemv_swiglu_q8(p(x) + 4, p(x), 1e-5, 0, 2, p(w.data), 64, H, p(out), p(out), p(a),
                                           p(cnt), st) != 0
    torch.cuda.synchronize()
