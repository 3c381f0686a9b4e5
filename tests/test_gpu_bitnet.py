"""The BitNet b1.58 per-token engine on the GPU (libac_bitnet_hip.so, the reference's ac_bitnet_engine.cpp) and its
kernels, against the oracle's restatement of the CPU token step (llama_bitnet_core.cpp:886-1300):
  kernels  norm + int8 (relu2 / silu / plain, with and without the norm): the normalized values within 1e-6 of the
           CPU's and the int8 values within one step where the CPU's f32 sum of squares rounds the scale apart;
           RoPE + cache rows bit for bit against the rotation of the same table; f32-cache attention and the f16 LM
           head within 1e-5; the I2_S GEMV with the residual add bit for bit against GEMV then add;
  engine   a small model (2 layers, ReLU^2 FFN with sub norms) and a BitNet b1.58 2B-shaped layer decoded token by token
           from position 0: residual stream and logits within 1e-3 relative L2 of the CPU token step (int8
           activations re-quantized at every layer make exact equality a matter of the last bit of each norm's sum);
           the same tokens through a second engine give identical results (the captured step is deterministic); the
           reference's error rules."""
import ctypes
import os

import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

from test_oracle_bitnet import i2s_pack  # noqa: E402

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(os.path.dirname(HERE), "ameva_compute_amd", "libac_bitnet_hip.so")


class CfgC(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in ("n_embd", "n_ffn", "n_heads", "n_kv_heads", "head_dim", "n_ctx",
                                               "n_layers")] + \
               [("norm_eps", ctypes.c_float), ("rope_theta", ctypes.c_float), ("relu2_ffn", ctypes.c_int32)]


class LayerC(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in ("attn_norm", "attn_sub_norm", "ffn_norm", "ffn_sub_norm", "wq", "wk",
                                               "wv", "wo", "w_gate", "w_up", "w_down")] + \
               [(n, ctypes.c_float) for n in ("scale_wq", "scale_wk", "scale_wv", "scale_wo", "scale_w_gate",
                                              "scale_w_up", "scale_w_down")]


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


@pytest.fixture(scope="module")
def eng():
    lib = ctypes.CDLL(LIB)
    P = ctypes.c_void_p
    lib.ac_bitnet_engine_create.restype = P
    lib.ac_bitnet_engine_configure.argtypes = [P, ctypes.POINTER(CfgC)]
    lib.ac_bitnet_engine_upload_layer.argtypes = [P, ctypes.c_uint32, ctypes.POINTER(LayerC)]
    lib.ac_bitnet_engine_upload_output.argtypes = [P, P, P, ctypes.c_uint32]
    lib.ac_bitnet_engine_eval_token.argtypes = [P, ctypes.c_uint32, P, P, P, ctypes.c_uint32]
    lib.ac_bitnet_engine_lm_head.argtypes = [P, P, P]
    lib.ac_bitnet_engine_last_error.argtypes = [P]
    lib.ac_bitnet_engine_last_error.restype = ctypes.c_char_p
    lib.ac_bitnet_engine_destroy.argtypes = [P]
    return lib


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def L():
    from ameva_compute_amd._lib import lib
    return lib()


def stream():
    return torch.cuda.current_stream().cuda_stream


def g(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


@pytest.mark.parametrize("mode,do_norm,n", [(0, 1, 2560), (1, 1, 6912), (2, 0, 512), (0, 0, 2560), (1, 0, 6912)])
def test_norm_q8(dev, orc, mode, do_norm, n):
    rng = np.random.default_rng(mode * 10 + do_norm + n)
    a = rng.standard_normal(n).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)
    if mode == 1:
        x = np.maximum(a, 0) * np.maximum(a, 0) * b
    elif mode == 2:
        x = (a / (1 + np.exp(-a))) * b
    else:
        x = a.copy()
    x = x.astype(np.float32)
    want = orc.bitnet_rms_norm(x, w, 1e-5) if do_norm else x
    q_want = np.empty(n, np.int8)
    d_want = orc.lib().orc_i2s_quantize_act(want.ctypes.data, q_want.ctypes.data, n)
    y = torch.empty(n, dtype=torch.float32, device=dev)
    act = torch.empty(n + 16, dtype=torch.uint8, device=dev)
    ga, gb, gw = g(a, dev), g(b, dev), g(w, dev)
    assert L().amv_bitnet_norm_q8(ga.data_ptr(), gb.data_ptr(), gw.data_ptr(), n, 1e-5, mode, do_norm, y.data_ptr(),
                                  act.data_ptr(), stream()) == 0
    torch.cuda.synchronize()
    yv = y.cpu().numpy()
    if do_norm:
        assert rel(yv, want) < 1e-6
    else:
        assert rel(yv, want) < 1e-6 if mode == 2 else np.array_equal(yv, want)  # silu: GPU expf against glibc's
    av = act.cpu().numpy()
    q = av[:n].view(np.int8)
    d, s = np.frombuffer(av[n:n + 8].tobytes(), np.float32)[0], np.frombuffer(av[n + 4:n + 8].tobytes(), np.int32)[0]
    diff = np.abs(q.astype(int) - q_want.astype(int))
    assert diff.max() <= 1 and np.count_nonzero(diff) <= max(2, n // 500)
    assert abs(d - d_want) <= 1e-6 * d_want and s == int(q.astype(np.int64).sum())


def test_rope_kv_and_cache_rows(dev):
    rng = np.random.default_rng(5)
    H, KVH, hd, ctx, pos = 20, 5, 128, 40, 17
    q = rng.standard_normal((H, hd)).astype(np.float32)
    k = rng.standard_normal((KVH, hd)).astype(np.float32)
    v = rng.standard_normal((KVH, hd)).astype(np.float32)
    half = hd // 2
    th = np.float32(pos) / np.power(np.float32(10000.0), (2 * np.arange(half, dtype=np.float32)) / np.float32(hd))
    cs = np.concatenate([np.cos(th), np.sin(th)]).astype(np.float32)
    gq, gk, gv, gcs = g(q, dev), g(k, dev), g(v, dev), g(cs, dev)
    kc = torch.zeros((ctx, KVH * hd), dtype=torch.float32, device=dev)
    vc = torch.zeros_like(kc)
    p = torch.tensor([pos], dtype=torch.int32, device=dev)
    assert L().amv_bitnet_rope_kv(gq.data_ptr(), gk.data_ptr(), gv.data_ptr(), gcs.data_ptr(), kc.data_ptr(),
                                  vc.data_ptr(), p.data_ptr(), H, KVH, hd, ctx, stream()) == 0
    c, s = cs[:half], cs[half:]

    def rot(x):
        x0, x1 = x[:, :half], x[:, half:]
        return np.concatenate([x0 * c - x1 * s, x1 * c + x0 * s], axis=1).astype(np.float32)
    assert np.array_equal(gq.cpu().numpy(), rot(q))
    kcn, vcn = kc.cpu().numpy(), vc.cpu().numpy()
    assert np.array_equal(kcn[pos], rot(k).reshape(-1)) and np.array_equal(vcn[pos], v.reshape(-1))
    assert not np.delete(kcn, pos, axis=0).any() and not np.delete(vcn, pos, axis=0).any()


def test_f32_cache_attention_and_f16_head(dev, orc):
    from ameva_compute_amd import ops
    rng = np.random.default_rng(6)
    H, KVH, hd, ctx = 20, 5, 128, 300
    for pos in (0, 1, 77, 299):
        q = rng.standard_normal((H, hd)).astype(np.float32)
        kc = rng.standard_normal((ctx, KVH * hd)).astype(np.float32)
        vc = rng.standard_normal((ctx, KVH * hd)).astype(np.float32)
        want = orc.bitnet_attention(q, kc, vc, pos, KVH)
        gkc, gvc = g(kc, dev), g(vc, dev)
        kview = gkc.view(ctx, KVH, hd).permute(1, 0, 2)
        vview = gvc.view(ctx, KVH, hd).permute(1, 0, 2)
        nkv = torch.tensor([pos + 1], dtype=torch.int32, device=dev)
        out = ops.flash_attn_decode_kv(g(q, dev), kview, vview, 0, 1.0 / float(np.sqrt(np.float32(hd))),
                                       n_kv_max=ctx, n_kv_dev=nkv)
        assert rel(out.cpu().numpy(), want) < 1e-5, pos
    W = (rng.standard_normal((1000, 2560)) * 0.05).astype(np.float16)
    x = rng.standard_normal(2560).astype(np.float32)
    y = torch.empty(1000, dtype=torch.float32, device=dev)
    gW, gx = g(W.view(np.uint16), dev), g(x, dev)
    assert L().amv_gemv_f16(gW.data_ptr(), 1000, 2560, gx.data_ptr(), y.data_ptr(), stream()) == 0
    assert rel(y.cpu().numpy(), orc.bitnet_gemv_f16(W.view(np.uint16), x)) < 1e-5


def test_i2s_gemv_residual_add(dev):
    rng = np.random.default_rng(7)
    n, k = 2560, 6912
    w = i2s_pack(rng.integers(0, 3, (n, k)).astype(np.uint8))
    x = rng.standard_normal(k).astype(np.float32)
    r = rng.standard_normal(n).astype(np.float32)
    gw, gx = g(w, dev), g(x, dev)
    act = torch.empty(k + 16, dtype=torch.uint8, device=dev)
    assert L().amv_i2s_quantize_act(gx.data_ptr(), 1, k, act.data_ptr(), stream()) == 0
    plain = torch.empty(n, dtype=torch.float32, device=dev)
    assert L().amv_i2s_gemv(gw.data_ptr(), n, k, act.data_ptr(), 1, 1.7, plain.data_ptr(), n, stream()) == 0
    acc = g(r, dev)
    assert L().amv_i2s_gemv_acc(gw.data_ptr(), n, k, act.data_ptr(), 1.7, acc.data_ptr(), stream()) == 0
    assert torch.equal(acc, g(r, dev) + plain)


def fused(a, b, nw, k, mode, do_norm, ws, rows, scales, dsts, acc, cs=None, pos=None, n_ctx=0):
    n = len(ws)
    W = (ctypes.c_void_p * 3)(*[t.data_ptr() for t in ws])
    Rw = (ctypes.c_int64 * 3)(*rows)
    S = (ctypes.c_float * 3)(*scales)
    D = (ctypes.c_void_p * 3)(*[t.data_ptr() for t in dsts])
    p = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    return L().amv_bitnet_gemv_fused(p(a), p(b), p(nw), k, 1e-5, mode, do_norm, n, W, Rw, S, D, acc, p(cs), p(pos),
                                     n_ctx, stream())


def unfused_act(dev, a, b, nw, k, mode, do_norm):
    act = torch.empty(k + 16, dtype=torch.uint8, device=dev)
    assert L().amv_bitnet_norm_q8(a.data_ptr(), None if b is None else b.data_ptr(),
                                  None if nw is None else nw.data_ptr(), k, 1e-5, mode, do_norm, None, act.data_ptr(),
                                  stream()) == 0
    return act


@pytest.mark.parametrize("k,rows,mode,do_norm,with_w,acc", [
    (2560, (2560,), 0, 1, True, 1), (2560, (2560,), 0, 0, False, 1), (2560, (6912, 6912), 0, 1, True, 0),
    (6912, (2560,), 1, 1, True, 1), (6912, (2560,), 2, 0, False, 1), (6912, (2560,), 1, 1, False, 0),
    (12288, (999,), 0, 1, True, 0), (256, (3, 5, 7), 2, 1, True, 1), (4096, (130, 1), 1, 1, True, 0)])
def test_fused_norm_gemv_equals_the_separate_kernels(dev, k, rows, mode, do_norm, with_w, acc):
    """One launch (the activation per workgroup in LDS, stacked matrices) = amv_bitnet_norm_q8 then one amv_i2s_gemv
    (or _acc) per matrix, bit for bit."""
    rng = np.random.default_rng(k + sum(rows) + 10 * mode + do_norm)
    a = g(rng.standard_normal(k).astype(np.float32), dev)
    b = g(rng.standard_normal(k).astype(np.float32), dev) if mode else None
    nw = g((1 + 0.1 * rng.standard_normal(k)).astype(np.float32), dev) if with_w else None
    ws = [g(i2s_pack(rng.integers(0, 3, (r, k)).astype(np.uint8)), dev) for r in rows]
    scales = [0.5 + 0.25 * i for i in range(len(rows))]
    base = [g(rng.standard_normal(r).astype(np.float32), dev) for r in rows]
    got = [t.clone() for t in base]
    assert fused(a, b, nw, k, mode, do_norm, ws, rows, scales, got, acc) == 0
    act = unfused_act(dev, a, b, nw, k, mode, do_norm)
    for w, r, sc, t0, t1 in zip(ws, rows, scales, base, got):
        want = t0.clone()
        if acc:
            assert L().amv_i2s_gemv_acc(w.data_ptr(), r, k, act.data_ptr(), sc, want.data_ptr(), stream()) == 0
        else:
            assert L().amv_i2s_gemv(w.data_ptr(), r, k, act.data_ptr(), 1, sc, want.data_ptr(), r, stream()) == 0
        torch.cuda.synchronize()
        assert torch.equal(t1, want)


@pytest.mark.parametrize("E,H,KVH,pos", [(2560, 20, 5, 17), (256, 2, 1, 0), (1024, 8, 8, 39), (8192, 64, 8, 5)])
def test_fused_qkv_rope_equals_the_separate_kernels(dev, E, H, KVH, pos):
    rng = np.random.default_rng(E + pos)
    hd, ctx, kv = 128, 40, KVH * 128
    x = g(rng.standard_normal(E).astype(np.float32), dev)
    nw = g((1 + 0.1 * rng.standard_normal(E)).astype(np.float32), dev)
    ws = [g(i2s_pack(rng.integers(0, 3, (r, E)).astype(np.uint8)), dev) for r in (H * hd, kv, kv)]
    sc = [1.3, 0.9, 1.1]
    th = np.float32(pos) / np.power(np.float32(10000.0), (2 * np.arange(64, dtype=np.float32)) / np.float32(hd))
    cs = g(np.concatenate([np.cos(th), np.sin(th)]).astype(np.float32), dev)
    p = torch.tensor([pos], dtype=torch.int32, device=dev)
    q1 = torch.empty(H * hd, dtype=torch.float32, device=dev)
    kc1, vc1 = torch.zeros((ctx, kv), device=dev), torch.zeros((ctx, kv), device=dev)
    assert fused(x, None, nw, E, 0, 1, ws, (H * hd, kv, kv), sc, [q1, kc1, vc1], 0, cs, p, ctx) == 0
    act = unfused_act(dev, x, None, nw, E, 0, 1)
    q2, k2, v2 = (torch.empty(r, dtype=torch.float32, device=dev) for r in (H * hd, kv, kv))
    for w, r, s_, o in zip(ws, (H * hd, kv, kv), sc, (q2, k2, v2)):
        assert L().amv_i2s_gemv(w.data_ptr(), r, E, act.data_ptr(), 1, s_, o.data_ptr(), r, stream()) == 0
    kc2, vc2 = torch.zeros((ctx, kv), device=dev), torch.zeros((ctx, kv), device=dev)
    assert L().amv_bitnet_rope_kv(q2.data_ptr(), k2.data_ptr(), v2.data_ptr(), cs.data_ptr(), kc2.data_ptr(),
                                  vc2.data_ptr(), p.data_ptr(), H, KVH, hd, ctx, stream()) == 0
    torch.cuda.synchronize()
    assert torch.equal(q1, q2) and torch.equal(kc1, kc2) and torch.equal(vc1, vc2)
    assert kc1[pos].abs().sum() > 0 and not torch.cat([kc1[:pos], kc1[pos + 1:]]).any()


def test_fused_argument_errors(dev):
    t = torch.zeros(1024, device=dev)
    w = torch.zeros(1024, dtype=torch.uint8, device=dev)
    assert fused(t, None, None, 100, 0, 1, [w], (4,), [1.0], [t], 0) != 0          # k % 128
    assert fused(t, None, None, 128, 1, 1, [w], (4,), [1.0], [t], 0) != 0          # relu2 without b
    assert fused(t, None, None, 256, 0, 1, [w, w], (4, 4), [1.0, 1.0], [t, t], 0, cs=t, pos=t, n_ctx=4) != 0  # rope: 3
    assert b"RoPE" in L().amv_last_error()


def random_model(rng, cfg, n_layers, n_vocab, relu2=True):
    E, F, kv = cfg["n_embd"], cfg["n_ffn"], cfg["n_kv_heads"] * cfg["head_dim"]
    r = lambda a, b: i2s_pack(rng.integers(0, 3, (a, b)).astype(np.uint8))  # noqa: E731
    nrm = lambda n: (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)  # noqa: E731
    layers = []
    for _ in range(n_layers):
        layers.append(dict(attn_norm=nrm(E), attn_sub_norm=nrm(E), ffn_norm=nrm(E),
                           ffn_sub_norm=nrm(F) if relu2 else None, wq=r(E, E), wk=r(kv, E), wv=r(kv, E), wo=r(E, E),
                           w_gate=r(F, E), w_up=r(F, E), w_down=r(E, F), scale_wq=1.3, scale_wk=0.9, scale_wv=1.1,
                           scale_wo=0.05, scale_w_gate=0.7, scale_w_up=0.8, scale_w_down=0.02))
    out_norm = nrm(E)
    head = (rng.standard_normal((n_vocab, E)) * 0.05).astype(np.float16).view(np.uint16)
    return layers, out_norm, head


def make_engine(eng, cfg, layers, out_norm, head):
    h = eng.ac_bitnet_engine_create()
    assert h, eng.ac_bitnet_engine_last_error(None)
    c = CfgC(cfg["n_embd"], cfg["n_ffn"], cfg["n_heads"], cfg["n_kv_heads"], cfg["head_dim"], cfg["n_ctx"],
             len(layers), cfg["norm_eps"], cfg["rope_theta"], int(cfg["relu2"]))
    assert eng.ac_bitnet_engine_configure(h, ctypes.byref(c)) == 0, eng.ac_bitnet_engine_last_error(h)
    for i, Ld in enumerate(layers):
        lc = LayerC()
        for n in ("attn_norm", "attn_sub_norm", "ffn_norm", "ffn_sub_norm", "wq", "wk", "wv", "wo", "w_gate", "w_up",
                  "w_down"):
            a = Ld.get(n)
            setattr(lc, n, None if a is None else a.ctypes.data)
        for n in ("scale_wq", "scale_wk", "scale_wv", "scale_wo", "scale_w_gate", "scale_w_up", "scale_w_down"):
            setattr(lc, n, Ld[n])
        assert eng.ac_bitnet_engine_upload_layer(h, i, ctypes.byref(lc)) == 0, eng.ac_bitnet_engine_last_error(h)
    assert eng.ac_bitnet_engine_upload_output(h, out_norm.ctypes.data, head.ctypes.data, head.shape[0]) == 0
    return h


@pytest.mark.parametrize("shape", ["small", "bitnet_2b_layer"])
def test_engine_matches_cpu_token_step(dev, eng, orc, shape):
    rng = np.random.default_rng(11)
    if shape == "small":
        cfg = dict(n_embd=256, n_ffn=512, n_heads=2, n_kv_heads=1, head_dim=128, n_ctx=32, norm_eps=1e-5,
                   rope_theta=10000.0, relu2=True)
        n_layers, n_vocab, n_tok = 2, 1000, 6
    else:
        cfg = dict(n_embd=2560, n_ffn=6912, n_heads=20, n_kv_heads=5, head_dim=128, n_ctx=64, norm_eps=1e-5,
                   rope_theta=500000.0, relu2=True)
        n_layers, n_vocab, n_tok = 1, 4096, 3
    layers, out_norm, head = random_model(rng, cfg, n_layers, n_vocab)
    m = orc.BitnetModel(cfg, layers, out_norm, head)
    h = make_engine(eng, cfg, layers, out_norm, head)
    h2 = make_engine(eng, cfg, layers, out_norm, head)
    try:
        E = cfg["n_embd"]
        for pos in range(n_tok):
            x = (rng.standard_normal(E) * 0.5).astype(np.float32)
            want_x, want_l = m.token(pos, x)
            got_x = np.empty(E, np.float32)
            got_l = np.empty(n_vocab, np.float32)
            assert eng.ac_bitnet_engine_eval_token(h, pos, x.ctypes.data, got_x.ctypes.data, got_l.ctypes.data, 0) == 0
            assert rel(got_x, want_x) < 1e-3 and rel(got_l, want_l) < 1e-3, (pos, rel(got_x, want_x), rel(got_l, want_l))
            # a second engine replaying its own captured step gives the same bits
            x2 = np.empty(E, np.float32)
            l2 = np.empty(n_vocab, np.float32)
            assert eng.ac_bitnet_engine_eval_token(h2, pos, x.ctypes.data, x2.ctypes.data, l2.ctypes.data, 0) == 0
            assert np.array_equal(x2, got_x) and np.array_equal(l2, got_l)
        # the LM head alone on the CPU's normalized x
        xn = orc.bitnet_rms_norm(want_x, out_norm, cfg["norm_eps"])
        lh = np.empty(n_vocab, np.float32)
        assert eng.ac_bitnet_engine_lm_head(h, xn.ctypes.data, lh.ctypes.data) == 0
        assert rel(lh, orc.bitnet_gemv_f16(head, xn)) < 1e-5
    finally:
        eng.ac_bitnet_engine_destroy(h)
        eng.ac_bitnet_engine_destroy(h2)


def test_engine_error_rules(dev, eng):
    h = eng.ac_bitnet_engine_create()
    try:
        x = np.zeros(256, np.float32)
        assert eng.ac_bitnet_engine_eval_token(h, 0, x.ctypes.data, None, None, 0) == -106  # before Configure
        bad = CfgC(250, 512, 2, 1, 128, 16, 1, 1e-5, 1e4, 1)
        assert eng.ac_bitnet_engine_configure(h, ctypes.byref(bad)) == -106
        assert b"unsupported model shape" in eng.ac_bitnet_engine_last_error(h)
        odd = CfgC(256, 512, 4, 1, 64, 16, 1, 1e-5, 1e4, 1)  # head_dim 64: a valid model outside the MI355X kernels
        assert eng.ac_bitnet_engine_configure(h, ctypes.byref(odd)) == -108
        good = CfgC(256, 512, 2, 1, 128, 16, 1, 1e-5, 1e4, 1)
        assert eng.ac_bitnet_engine_configure(h, ctypes.byref(good)) == 0
        assert eng.ac_bitnet_engine_configure(h, ctypes.byref(good)) == -106  # twice
        lc = LayerC()
        assert eng.ac_bitnet_engine_upload_layer(h, 0, ctypes.byref(lc)) == -106  # tensors missing
        assert eng.ac_bitnet_engine_upload_layer(h, 1, ctypes.byref(lc)) == -106  # out of range
        rng = np.random.default_rng(0)
        cfg = dict(n_embd=256, n_ffn=512, n_heads=2, n_kv_heads=1, head_dim=128, n_ctx=16, norm_eps=1e-5,
                   rope_theta=1e4, relu2=True)
        layers, out_norm, head = random_model(rng, cfg, 1, 10, relu2=False)  # no ffn_sub_norm with relu2_ffn
        lc = LayerC()
        for n in ("attn_norm", "ffn_norm", "wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down"):
            setattr(lc, n, layers[0][n].ctypes.data)
        assert eng.ac_bitnet_engine_upload_layer(h, 0, ctypes.byref(lc)) == -106
        assert b"ffn_sub_norm" in eng.ac_bitnet_engine_last_error(h)
        lg = np.zeros(10, np.float32)
        assert eng.ac_bitnet_engine_eval_token(h, 16, x.ctypes.data, None, None, 0) == -106   # pos >= n_ctx
        assert eng.ac_bitnet_engine_eval_token(h, 0, x.ctypes.data, None, lg.ctypes.data, 0) == -106  # no LM head
        assert eng.ac_bitnet_engine_lm_head(h, x.ctypes.data, lg.ctypes.data) == -106
        assert eng.ac_bitnet_engine_eval_token(h, 0, x.ctypes.data, None, None, 0) == -106  # layer not uploaded
    finally:
        eng.ac_bitnet_engine_destroy(h)


@pytest.mark.parametrize("do_norm,acc", [(1, 1), (0, 1), (1, 0)])
def test_fa_merge_fold_equals_the_merge_launch(dev, do_norm, acc):
    """The BitNet engine's short-context output projection: the attention splits alone (amv_flash_attn_split_kv) and
    their merge in the projection's prologue (amv_bitnet_gemv_fa_merge) = split + merge (amv_flash_attn_decode_kv)
    + amv_bitnet_gemv_fused on the merged row, bit for bit, over an f32 cache with the key count in device memory.
    Counts run downward, so the splits past each count hold an earlier call's partials (masked, never read)."""
    rng = np.random.default_rng(31 + do_norm + 2 * acc)
    H, KVH, hd, nk = 20, 5, 128, 256
    E, kv = H * hd, KVH * hd
    scale = 1.0 / float(np.sqrt(np.float32(hd)))
    q = g(rng.standard_normal((H, hd)).astype(np.float32), dev)
    kc = g(rng.standard_normal((nk, kv)).astype(np.float32), dev)
    vc = g(rng.standard_normal((nk, kv)).astype(np.float32), dev)
    nw = g((1 + 0.1 * rng.standard_normal(E)).astype(np.float32), dev) if do_norm else None
    w = g(i2s_pack(rng.integers(0, 3, (E, E)).astype(np.uint8)), dev)
    base = g(rng.standard_normal(E).astype(np.float32), dev)
    wsb = L().amv_flash_attn_workspace_bytes(H, KVH, nk, hd)
    ws = torch.empty(wsb // 4, dtype=torch.float32, device=dev)
    att = torch.empty(E, dtype=torch.float32, device=dev)
    nkv = torch.zeros(1, dtype=torch.int32, device=dev)
    ns, sl = ctypes.c_int32(0), ctypes.c_int32(0)
    st = stream()
    for n in (256, 200, 129, 128, 65, 64, 37, 2, 1):
        nkv.fill_(n)
        want = base.clone()
        assert L().amv_flash_attn_decode_kv(0, q.data_ptr(), kc.data_ptr(), vc.data_ptr(), None, att.data_ptr(), H, KVH,
                                            nk, nkv.data_ptr(), hd, kv * 4, hd * 4, kv * 4, hd * 4, scale,
                                            ws.data_ptr(), wsb, None, None, 8, 0, st) == 0
        assert fused(att, None, nw, E, 0, do_norm, [w], (E,), (0.05,), [want], acc) == 0
        got = base.clone()
        assert L().amv_flash_attn_split_kv(0, q.data_ptr(), kc.data_ptr(), vc.data_ptr(), None, H, KVH, nk,
                                           nkv.data_ptr(), hd, kv * 4, hd * 4, kv * 4, hd * 4, scale, ws.data_ptr(),
                                           wsb, 0, ctypes.byref(ns), ctypes.byref(sl), st) == 0
        assert (ns.value, sl.value) == (4, 64)
        assert L().amv_bitnet_gemv_fa_merge(ws.data_ptr(), ns.value, sl.value, nk, nkv.data_ptr(),
                                            None if nw is None else nw.data_ptr(), E, 1e-5, do_norm, w.data_ptr(), E,
                                            0.05, got.data_ptr(), acc, st) == 0
        torch.cuda.synchronize()
        assert torch.equal(got, want), n
    # more keys than 4 splits hold is refused
    assert L().amv_bitnet_gemv_fa_merge(ws.data_ptr(), 8, 64, 300, nkv.data_ptr(), None, E, 1e-5, 0, w.data_ptr(), E,
                                        0.05, base.data_ptr(), 1, st) != 0


def test_engine_fold_merge_equals_merge_launch(dev, eng, monkeypatch):
    """The engine at short contexts (the merge folded into the output projection) against the same engine with the
    merge launch kept (AMV_BITNET_FOLD_MERGE=0): every token's x and logits bit-identical, at positions on both
    sides of the fold's 256-key limit."""
    rng = np.random.default_rng(12)
    cfg = dict(n_embd=256, n_ffn=512, n_heads=2, n_kv_heads=1, head_dim=128, n_ctx=300, norm_eps=1e-5,
               rope_theta=10000.0, relu2=True)
    layers, out_norm, head = random_model(rng, cfg, 2, 1000)
    h = make_engine(eng, cfg, layers, out_norm, head)
    monkeypatch.setenv("AMV_BITNET_FOLD_MERGE", "0")
    h2 = make_engine(eng, cfg, layers, out_norm, head)
    try:
        E = cfg["n_embd"]
        for pos in range(258):  # consecutive positions: each token reads the cache rows the earlier ones wrote
            x = (rng.standard_normal(E) * 0.5).astype(np.float32)
            out = []
            for hh in (h, h2):
                xo = np.empty(E, np.float32)
                lo = np.empty(1000, np.float32)
                assert eng.ac_bitnet_engine_eval_token(hh, pos, x.ctypes.data, xo.ctypes.data, lo.ctypes.data, 0) == 0
                out.append((xo, lo))
            assert np.array_equal(out[0][0], out[1][0]) and np.array_equal(out[0][1], out[1][1]), pos
    finally:
        eng.ac_bitnet_engine_destroy(h)
        eng.ac_bitnet_engine_destroy(h2)
