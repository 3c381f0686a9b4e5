"""GPU tests through the ggml backend plugin (libggml-ameva.so): single-node graphs for every op of the hot path,
the counters the reference's own tests use as ground truth that a GPU kernel ran, lossless get_tensor of repacked
weights, the FAIL-FAST paths forced by failure injection, and one Llama-3-8B-shaped decoder layer (BASELINE config
4: hidden 4096, 32 / 8 heads of 128, RoPE theta 500000, FA decode over an f16 KV cache of 4096, SwiGLU 14336, Q4_0
weights) against the oracle's chain of the same ops."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

import ggml_plugin as gp  # noqa: E402
from parity import dequant_act, per_output_gate  # noqa: E402


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


@pytest.fixture(scope="module")
def plugin():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return gp.load()[1]


def quantize(orc, t, w):
    if t == gp.Q4_0:
        return orc.quantize_q4_0(w)
    if t == gp.Q8_0:
        return orc.quantize_q8_0(w, orc.Q8_REF)
    raise ValueError(t)


def random_kquant(rng, t, n, k):
    bb = 144 if t == gp.Q4_K else 210
    y = rng.integers(0, 256, (n, k // 256, bb), dtype=np.uint8)
    offs = (0, 2) if t == gp.Q4_K else (208,)
    for off in offs:
        v = rng.uniform(0.0, 0.002, (n, k // 256)).astype(np.float16)
        y[:, :, off:off + 2] = v.view(np.uint8).reshape(n, k // 256, 2)
    return y.reshape(n, -1)


@pytest.mark.parametrize("wt", [gp.Q4_0, gp.Q8_0, gp.Q4_K, gp.Q6_K])
@pytest.mark.parametrize("m", [1, 16, 100])
def test_mul_mat_node(plugin, orc, wt, m):
    rng = np.random.default_rng(wt * 10 + m)
    n, k = 512, 4096
    if wt in (gp.Q4_0, gp.Q8_0):
        wg = quantize(orc, wt, (rng.standard_normal((n, k)) * 0.02).astype(np.float32))
        aq = lambda x: orc.quantize_q8_0(x, orc.Q8_X86)  # noqa: E731
    else:
        wg = random_kquant(rng, wt, n, k)
        aq = orc.quantize_q8_K
    x = rng.standard_normal((m, k)).astype(np.float32)
    g = gp.Graph(wg.nbytes + 4096, 64 << 20)
    try:
        plugin.ggml_backend_ameva_reset_counters()
        W = g.tensor(wt, [k, n], "w", "w")
        X = g.tensor(gp.F32, [k, m], "c", "x")
        g.set(W, wg)
        g.set(X, x)
        Y = g.mul_mat(W, X)
        rep0 = gp.counter(plugin, "repacked_tensor_count")
        assert g.compute() == gp.STATUS_SUCCESS
        y = g.get(Y, np.float32, (m, n))
        assert rel_l2(y, orc.mul_mat(wt, wg, n, k, aq(x), m)) < 1e-3
        per_output_gate(y, orc.dequantize(wt, wg, k), dequant_act(aq(x), 15 if wt in (gp.Q4_K, gp.Q6_K) else 8, k),
                        what=f"plugin MUL_MAT {wt} m={m}")
        assert gp.counter(plugin, "f32_gpu_sgemm_dispatch_count") == 1
        assert gp.counter(plugin, "mmq_mul_mat_count") == (1 if m >= 8 else 0)
        assert gp.counter(plugin, "repacked_tensor_count") == rep0 + 1
        # the weight reads back in ggml layout, byte for byte
        assert np.array_equal(g.get(W, np.uint8), wg.reshape(-1))
        # a second run reuses the repacked weight
        assert g.compute() == gp.STATUS_SUCCESS
        assert np.array_equal(g.get(Y, np.float32, (m, n)), y)
    finally:
        g.free()


# The reference's placement matrix (tests/ameva_qmm_check.cpp:46-48, 103-166, 240-246): the weight in a compute
# buffer ("resident", repacked into scratch per use), in a WEIGHTS buffer ("weights", repacked in place once), in a
# WEIGHTS buffer written by two partial set_tensor calls that end inside a row ("split"), and a view of rows
# [3, 3 + N) of a weight of N + 5 rows ("view"); its shapes: one-column GEMVs, small batches below and above the
# MFMA crossover (M = 8), odd N and partial tiles, long rows, and K = 544 (17 blocks of 32, not whole K-quant
# super-blocks).
MMQ_PLUGIN_TYPES = (gp.Q4_0, gp.Q8_0, gp.Q4_K, gp.Q6_K)  # weight types with a batched (M >= 8) matrix-core kernel
QMM_SHAPES = [(1, 37, 256), (5, 64, 512), (8, 16, 256), (13, 33, 768), (1, 70, 2560), (3, 19, 4096), (40, 70, 512),
              (33, 130, 256), (1, 21, 544)]


@pytest.mark.parametrize("place", ["resident", "weights", "split", "view"])
@pytest.mark.parametrize("wt", [gp.Q4_0, gp.Q8_0, gp.Q4_K, gp.Q6_K])
def test_mul_mat_placement_matrix(plugin, orc, wt, place):
    be = gp.BLOCK[wt][0]
    ran = 0
    for M, N, K in QMM_SHAPES:
        if K % be:
            continue
        rng = np.random.default_rng(wt * 7919 + M * 131 + N * 17 + K)
        NW = N + 5 if place == "view" else N
        if wt in (gp.Q4_0, gp.Q8_0):
            wg = quantize(orc, wt, (rng.standard_normal((NW, K)) * 0.02).astype(np.float32))
            aq = lambda x: orc.quantize_q8_0(x, orc.Q8_X86)  # noqa: E731
        else:
            wg = random_kquant(rng, wt, NW, K)
            aq = orc.quantize_q8_K
        wg = wg.reshape(NW, -1)
        x = rng.standard_normal((M, K)).astype(np.float32)
        g = gp.Graph(wg.nbytes + 4096, 16 << 20)
        try:
            plugin.ggml_backend_ameva_reset_counters()
            W = g.tensor(wt, [K, NW], "c" if place == "resident" else "w", "w")
            X = g.tensor(gp.F32, [K, M], "c", "x")
            if place == "split":  # the first write ends inside a row and is not the whole tensor
                raw = np.ascontiguousarray(wg).reshape(-1)
                cut = raw.nbytes // 3 + 1
                buf = gp.ctypes.cast(W.buffer, gp.POINTER(gp.Buffer)).contents
                buf.iface.set_tensor(W.buffer, gp.ctypes.addressof(W), raw.ctypes.data, 0, cut)
                buf.iface.set_tensor(W.buffer, gp.ctypes.addressof(W), raw.ctypes.data + cut, cut, raw.nbytes - cut)
            else:
                g.set(W, wg)
            g.set(X, x)
            rb = wg.shape[1]
            src0 = g.view(W, wt, [K, N], [W.nb[0], rb, rb * N, rb * N], 3 * rb, "w_rows") if place == "view" else W
            Y = g.mul_mat(src0, X)
            assert not g.reason(Y), (M, N, K, g.reason(Y))
            rep0 = gp.counter(plugin, "repacked_tensor_count")
            assert g.compute() == gp.STATUS_SUCCESS, (M, N, K)
            y = g.get(Y, np.float32, (M, N))
            r0 = 3 if place == "view" else 0
            want = orc.mul_mat(wt, np.ascontiguousarray(wg[r0:r0 + N]), N, K, aq(x), M)
            assert rel_l2(y, want) < 1e-3, (M, N, K, rel_l2(y, want))
            per_output_gate(y, orc.dequantize(wt, np.ascontiguousarray(wg[r0:r0 + N]), K),
                            dequant_act(aq(x), 15 if wt in (gp.Q4_K, gp.Q6_K) else 8, K),
                            what=f"placement {place} {wt} {(M, N, K)}")
            repacked = place in ("weights", "split")
            assert gp.counter(plugin, "repacked_tensor_count") == rep0 + (1 if repacked else 0), (M, N, K)
            assert gp.counter(plugin, "f32_gpu_sgemm_dispatch_count") == 1
            batched = M >= 8 and wt in MMQ_PLUGIN_TYPES
            assert gp.counter(plugin, "mmq_mul_mat_count") == (1 if batched else 0), (M, N, K)
            # the buffer interface returns the uploaded ggml bytes, whole and from inside a row to inside a row
            assert np.array_equal(g.get(W, np.uint8), wg.reshape(-1)), (M, N, K)
            o, cnt = rb // 2 + 1, wg.nbytes - rb
            part = np.empty(cnt, np.uint8)
            buf = gp.ctypes.cast(W.buffer, gp.POINTER(gp.Buffer)).contents
            buf.iface.get_tensor(W.buffer, gp.ctypes.addressof(W), part.ctypes.data, o, cnt)
            assert np.array_equal(part, wg.reshape(-1)[o:o + cnt]), (M, N, K)
            ran += 1
        finally:
            g.free()
    assert ran >= 7


@pytest.mark.parametrize("wt", [gp.Q4_0, gp.Q4_K])
def test_mul_mat_view_of_repacked_weight(plugin, orc, wt):
    """A graph that reads a weight whole (which repacks it in place) and then rows [3, 3 + N) of it through a view:
    the view's rows come from a ggml-layout copy of the repacked parent, and both products match the oracle."""
    rng = np.random.default_rng(wt)
    NW, N, K, M = 133, 64, 512, 12
    if wt == gp.Q4_0:
        wg = quantize(orc, wt, (rng.standard_normal((NW, K)) * 0.02).astype(np.float32)).reshape(NW, -1)
        aq = lambda x: orc.quantize_q8_0(x, orc.Q8_X86)  # noqa: E731
    else:
        wg = random_kquant(rng, wt, NW, K)
        aq = orc.quantize_q8_K
    x = rng.standard_normal((M, K)).astype(np.float32)
    g = gp.Graph(wg.nbytes + 4096, 16 << 20)
    try:
        W = g.tensor(wt, [K, NW], "w", "w")
        X = g.tensor(gp.F32, [K, M], "c", "x")
        g.set(W, wg)
        g.set(X, x)
        rb = wg.shape[1]
        V = g.view(W, wt, [K, N], [W.nb[0], rb, rb * N, rb * N], 3 * rb, "w_rows")
        YW = g.mul_mat(W, X, "whole")
        YV = g.mul_mat(V, X, "rows")
        rep0 = gp.counter(plugin, "repacked_tensor_count")
        assert g.compute() == gp.STATUS_SUCCESS
        assert gp.counter(plugin, "repacked_tensor_count") == rep0 + 1
        a = aq(x)
        assert rel_l2(g.get(YW, np.float32, (M, NW)), orc.mul_mat(wt, wg, NW, K, a, M)) < 1e-3
        assert rel_l2(g.get(YV, np.float32, (M, N)), orc.mul_mat(wt, np.ascontiguousarray(wg[3:3 + N]), N, K, a, M)) < 1e-3
        assert np.array_equal(g.get(W, np.uint8), wg.reshape(-1))
    finally:
        g.free()


def test_activation_reuse_and_norm_fusion(plugin, orc):
    rng = np.random.default_rng(3)
    k, n = 4096, 256
    wa = quantize(orc, gp.Q4_0, (rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    wb = quantize(orc, gp.Q4_0, (rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    x = rng.standard_normal((1, k)).astype(np.float32) * 3
    nw = rng.standard_normal(k).astype(np.float32)
    g = gp.Graph(2 * wa.nbytes + 8192, 32 << 20)
    try:
        plugin.ggml_backend_ameva_reset_counters()
        WA, WB = g.tensor(gp.Q4_0, [k, n], "w", "wa"), g.tensor(gp.Q4_0, [k, n], "w", "wb")
        X, NW = g.tensor(gp.F32, [k, 1], "c", "x"), g.tensor(gp.F32, [k], "c", "nw")
        for t, a in ((WA, wa), (WB, wb), (X, x), (NW, nw)):
            g.set(t, a)
        N = g.rms_norm(X, 1e-5)
        M = g.mul(N, NW)
        YA, YB = g.mul_mat(WA, M), g.mul_mat(WB, M)
        assert g.compute() == gp.STATUS_SUCCESS
        y_ref, o_ref = orc.rms_norm(x, 1e-5, nw)
        o = g.get(M, np.float32, (1, k))
        assert rel_l2(g.get(N, np.float32, (1, k)), y_ref) < 1e-6 and rel_l2(o, o_ref) < 1e-6
        a = orc.quantize_q8_0(o, orc.Q8_X86)
        assert rel_l2(g.get(YA, np.float32), orc.mul_mat(gp.Q4_0, wa, n, k, a, 1)) < 1e-3
        assert rel_l2(g.get(YB, np.float32), orc.mul_mat(gp.Q4_0, wb, n, k, a, 1)) < 1e-3
        assert gp.counter(plugin, "fused_pair_count") == 1
        # the fused RMS_NORM + MUL also writes the Q8_0 row both GEMVs read: two reuses, no quantization launch
        assert gp.counter(plugin, "act_quant_reuse_count") == 2
        assert gp.counter(plugin, "gpu_op_count") == 4
    finally:
        g.free()


@pytest.mark.parametrize("form", ["add", "gate", "up", "gate_swapped"])
def test_mul_mat_epilogue_fusion(plugin, orc, form):
    """A one-row MUL_MAT followed by ADD or GLU SWIGLU (split) runs as the GEMV's epilogue: the fused node's value and
    the MUL_MAT's own output both match the unfused ops (ggml_swiglu_split(a, b) = silu(a) * b; swapped: silu(b) * a)."""
    rng = np.random.default_rng(len(form))
    k, n = 4096, 1024
    wg = quantize(orc, gp.Q4_0, (rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    x = rng.standard_normal((1, k)).astype(np.float32)
    e = (rng.standard_normal((1, n)) * 2).astype(np.float32)
    g = gp.Graph(wg.nbytes + 8192, 32 << 20)
    try:
        plugin.ggml_backend_ameva_reset_counters()
        W, X, E = g.tensor(gp.Q4_0, [k, n], "w", "w"), g.tensor(gp.F32, [k, 1], "c", "x"), g.tensor(gp.F32, [n, 1], "c", "e")
        for t, a in ((W, wg), (X, x), (E, e)):
            g.set(t, a)
        Y = g.mul_mat(W, X)
        if form == "add":
            Z = g.add(Y, E)
        elif form == "gate":
            Z = g.swiglu(Y, E)
        elif form == "up":
            Z = g.swiglu(E, Y)
        else:
            Z = g.swiglu(E, Y, swapped=True)  # silu(Y) * E with Y as src1
        assert g.compute() == gp.STATUS_SUCCESS
        y_ref = orc.mul_mat(gp.Q4_0, wg, n, k, orc.quantize_q8_0(x, orc.Q8_X86), 1).reshape(1, n)
        y = g.get(Y, np.float32, (1, n))
        assert rel_l2(y, y_ref) < 1e-3
        z = g.get(Z, np.float32, (1, n))
        ref = {"add": y + e, "gate": orc.swiglu(y, e), "up": orc.swiglu(e, y), "gate_swapped": orc.swiglu(y, e)}[form]
        assert rel_l2(z, ref) < 1e-6
        assert gp.counter(plugin, "fused_pair_count") == 1
        assert gp.counter(plugin, "gpu_op_count") == 2
    finally:
        g.free()


def test_rope_swiglu_get_rows_nodes(plugin, orc):
    rng = np.random.default_rng(4)
    g = gp.Graph(1 << 20, 16 << 20)
    try:
        x = rng.standard_normal((3, 32, 128)).astype(np.float32)
        pos = np.array([0, 17, 4095], np.int32)
        X, POS = g.tensor(gp.F32, [128, 32, 3]), g.tensor(gp.I32, [3])
        g.set(X, x)
        g.set(POS, pos)
        R = g.rope(X, POS, 128, 0, 500000.0)
        gt, up = rng.standard_normal(14336).astype(np.float32), rng.standard_normal(14336).astype(np.float32)
        G_, U_ = g.tensor(gp.F32, [14336, 1]), g.tensor(gp.F32, [14336, 1])
        g.set(G_, gt)
        g.set(U_, up)
        S = g.swiglu(G_, U_)
        emb = (rng.standard_normal((64, 4096)) * 0.02).astype(np.float32)
        embq = orc.quantize_q4_0(emb)
        E = g.tensor(gp.Q4_0, [4096, 64], "w", "tok_embd")
        g.set(E, embq)
        ids = np.array([5, 63, 0], np.int32)
        IDS = g.tensor(gp.I32, [3])
        g.set(IDS, ids)
        GR = g.get_rows(E, IDS)
        assert g.compute() == gp.STATUS_SUCCESS
        assert rel_l2(g.get(R, np.float32, (3, 32, 128)), orc.rope(x, pos, 128, 0, 500000.0)) < 1e-5
        assert rel_l2(g.get(S, np.float32), orc.swiglu(gt, up)) < 1e-6
        assert np.array_equal(g.get(GR, np.float32, (3, 4096)), orc.dequantize(gp.Q4_0, embq, 4096)[ids])
    finally:
        g.free()


def test_failure_injection_and_contract_fail_fast(plugin):
    rng = np.random.default_rng(5)
    g = gp.Graph(1 << 20, 8 << 20)
    try:
        X = g.tensor(gp.F32, [4096, 1])
        g.set(X, rng.standard_normal(4096).astype(np.float32))
        W = g.tensor(gp.Q4_0, [4096, 64], "w", "w")
        g.set(W, rng.integers(0, 256, 64 * 128 * 18, dtype=np.uint8).reshape(64, -1) & 0x0F)
        Y = g.mul_mat(W, X)
        plugin.ggml_backend_ameva_reset_counters()
        plugin.ggml_backend_ameva_set_failure_injection(6)  # AMEVA_FAIL_DISPATCH
        try:
            assert g.compute() == gp.STATUS_FAILED
            assert gp.counter(plugin, "f32_gpu_sgemm_dispatch_count") == 0
        finally:
            plugin.ggml_backend_ameva_set_failure_injection(0)
        plugin.ggml_backend_ameva_set_failure_injection(7)  # AMEVA_FAIL_WAIT_TIMEOUT
        try:
            assert g.compute() == gp.STATUS_FAILED
        finally:
            plugin.ggml_backend_ameva_set_failure_injection(0)
        assert g.compute() == gp.STATUS_SUCCESS
        # one unsupported node fails the whole graph before anything runs
        plugin.ggml_backend_ameva_reset_counters()
        bad = g._node(gp.OP_SOFT_MAX, gp.F32, [4096, 1], [X], "softmax")
        assert g.compute([Y, bad]) == gp.STATUS_FAILED
        assert gp.counter(plugin, "gpu_op_count") == 0
    finally:
        g.free()


@pytest.mark.parametrize("t", [gp.Q8_0, gp.Q4_0])
def test_quantized_kv_cache_nodes(plugin, orc, t):
    """SET_ROWS of a token's K and V rows into a Q8_0 / Q4_0 cache, then FLASH_ATTN_EXT over llama.cpp's views of that
    cache (the reference's quantized-cache path, ameva_set_rows_q.comp + ameva_flash_attn.comp:104-136): the written
    rows equal the oracle's quantizer bytes, and the attention equals the oracle's restatement of ggml's CPU kernel."""
    rng = np.random.default_rng(77 + t)
    NH, NKV, D, CTX, pos_t = 32, 8, 128, 512, 300
    bs = 34 if t == gp.Q8_0 else 18
    rb = D // 32 * bs                                     # one head row
    quant = (lambda a: orc.quantize_q8_0(a, orc.Q8_X86)) if t == gp.Q8_0 else orc.quantize_q4_0
    kf = rng.standard_normal((CTX, NKV * D)).astype(np.float32)
    vf = rng.standard_normal((CTX, NKV * D)).astype(np.float32)
    kc, vc = quant(kf), quant(vf)                         # [CTX, NKV * rb]
    knew = rng.standard_normal((1, NKV * D)).astype(np.float32)
    vnew = rng.standard_normal((1, NKV * D)).astype(np.float32)
    q = rng.standard_normal((NH, D)).astype(np.float32)
    mask = np.zeros(CTX, np.float16)
    mask[pos_t + 1:] = -np.inf
    g = gp.Graph(4096, 32 << 20)
    try:
        KC, VC = g.tensor(t, [NKV * D, CTX], "c", "k_cache"), g.tensor(t, [NKV * D, CTX], "c", "v_cache")
        g.set(KC, kc)
        g.set(VC, vc)
        KN, VN = g.tensor(gp.F32, [NKV * D, 1], "c", "k_new"), g.tensor(gp.F32, [NKV * D, 1], "c", "v_new")
        g.set(KN, knew)
        g.set(VN, vnew)
        IDX = g.tensor(gp.I64, [1], "c", "kv_idx")
        g.set(IDX, np.array([pos_t], np.int64))
        Q = g.tensor(gp.F32, [D, NH, 1], "c", "q")
        g.set(Q, q)
        MASK = g.tensor(gp.F16, [CTX, 1], "c", "mask")
        g.set(MASK, mask)
        g.set_rows(KC, KN, IDX)
        g.set_rows(VC, VN, IDX)
        kv_nb = [bs, NKV * rb, rb, NKV * rb * CTX]
        kview = g.view_nd(KC, gp.OP_VIEW, [D, CTX, NKV], kv_nb)
        vview = g.view_nd(VC, gp.OP_VIEW, [D, CTX, NKV], kv_nb)
        qp = g.view_nd(Q, gp.OP_PERMUTE, [D, 1, NH], [4, D * NH * 4, D * 4, D * NH * 4])
        att = g.flash_attn_ext(qp, kview, vview, MASK, 1.0 / np.sqrt(D))
        assert g.compute() == gp.STATUS_SUCCESS
        got = g.get(att, np.float32, (NH, D))
        kc2, vc2 = kc.copy(), vc.copy()
        kc2[pos_t], vc2[pos_t] = quant(knew)[0], quant(vnew)[0]
        assert np.array_equal(g.get(KC, np.uint8, kc.shape), kc2)
        assert np.array_equal(g.get(VC, np.uint8, vc.shape), vc2)
        kh = np.ascontiguousarray(kc2.reshape(CTX, NKV, rb).transpose(1, 0, 2))
        vh = np.ascontiguousarray(vc2.reshape(CTX, NKV, rb).transpose(1, 0, 2))
        want = orc.flash_attn_decode_q(t, q, kh, vh, 1.0 / np.sqrt(D), mask.view(np.uint16))
        assert rel_l2(got, want) < 1e-4
    finally:
        g.free()


@pytest.mark.parametrize("wt", [gp.Q4_0, gp.Q4_K])
def test_llama3_8b_decode_layer(plugin, orc, wt):
    """One decoder layer of Llama-3-8B shape, bs1 decode at position 4095 with 4095 cached tokens, Q4_0 weights (Q8_0
    activations) or Q4_K weights (Q8_K activations): the plugin runs it as 6 launches for Q4_0 (q/k/v with the
    RMS_NORM + MUL before it, ROPE and both SET_ROWS; the attention split and merge; o + ADD; gate/up with the
    RMS_NORM + MUL before it and SWIGLU; down + ADD), as 7 for Q4_K (the FFN RMS_NORM + MUL a launch of its own)."""
    rng = np.random.default_rng(2024)
    H, NH, NKV, D, FF, CTX = 4096, 32, 8, 128, 14336, 4096
    pos_t = CTX - 1
    eps, base = 1e-5, 500000.0
    def wq4(n, k):
        if wt == gp.Q4_K:  # random K-quant blocks, d and dmin in [0, 2e-4): weights of magnitude ~0.1
            y = random_kquant(rng, gp.Q4_K, n, k)
            for off in (0, 2):
                v = rng.uniform(0.0, 2e-4, (n, k // 256)).astype(np.float16)
                y.reshape(n, k // 256, 144)[:, :, off:off + 2] = v.view(np.uint8).reshape(n, k // 256, 2)
            return y
        return orc.quantize_q4_0((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    bpw = {gp.Q4_0: (32, 18), gp.Q4_K: (256, 144)}[wt]  # weights per block, bytes per block
    w = {"q": wq4(NH * D, H), "k": wq4(NKV * D, H), "v": wq4(NKV * D, H), "o": wq4(H, NH * D),
         "gate": wq4(FF, H), "up": wq4(FF, H), "down": wq4(H, FF)}
    attn_norm = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    ffn_norm = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    x = rng.standard_normal((1, H)).astype(np.float32)
    kc = rng.standard_normal((CTX, NKV * D)).astype(np.float16)  # llama.cpp cache rows [token][head * D]
    vc = rng.standard_normal((CTX, NKV * D)).astype(np.float16)
    wbytes = sum(a.nbytes for a in w.values()) + 16 * 4096
    g = gp.Graph(wbytes, 96 << 20)
    try:
        plugin.ggml_backend_ameva_reset_counters()
        T = {k_: g.tensor(wt, [a.shape[1] * bpw[0] // bpw[1], a.shape[0]], "w", k_) for k_, a in w.items()}
        for k_, a in w.items():
            g.set(T[k_], a)
        AN, FN = g.tensor(gp.F32, [H], "w", "attn_norm"), g.tensor(gp.F32, [H], "w", "ffn_norm")
        g.set(AN, attn_norm)
        g.set(FN, ffn_norm)
        KC, VC = g.tensor(gp.F16, [NKV * D, CTX], "c", "k_cache"), g.tensor(gp.F16, [NKV * D, CTX], "c", "v_cache")
        g.set(KC, kc)
        g.set(VC, vc)
        X = g.tensor(gp.F32, [H, 1], "c", "inp")
        g.set(X, x)
        POS = g.tensor(gp.I32, [1], "c", "pos")
        g.set(POS, np.array([pos_t], np.int32))
        IDX = g.tensor(gp.I64, [1], "c", "kv_idx")
        g.set(IDX, np.array([pos_t], np.int64))
        MASK = g.tensor(gp.F16, [CTX, 1], "c", "mask")
        g.set(MASK, np.zeros(CTX, np.float16))

        cur = g.mul(g.rms_norm(X, eps), AN)
        q = g.reshape_3d(g.mul_mat(T["q"], cur), D, NH, 1)
        k = g.reshape_3d(g.mul_mat(T["k"], cur), D, NKV, 1)
        v = g.mul_mat(T["v"], cur)
        q = g.rope(q, POS, D, 0, base)
        k = g.rope(k, POS, D, 0, base)
        k2 = g.view_nd(k, gp.OP_RESHAPE, [NKV * D, 1], [4, NKV * D * 4, NKV * D * 4, NKV * D * 4])
        g.set_rows(KC, k2, IDX)
        g.set_rows(VC, v, IDX)
        kv_nb = [2, NKV * D * 2, D * 2, NKV * D * 2 * CTX]
        kview = g.view_nd(KC, gp.OP_VIEW, [D, CTX, NKV], kv_nb)
        vview = g.view_nd(VC, gp.OP_VIEW, [D, CTX, NKV], kv_nb)
        qp = g.view_nd(q, gp.OP_PERMUTE, [D, 1, NH], [4, D * NH * 4, D * 4, D * NH * 4])
        att = g.flash_attn_ext(qp, kview, vview, MASK, 1.0 / np.sqrt(D))
        att2 = g.view_nd(att, gp.OP_RESHAPE, [H, 1], [4, H * 4, H * 4, H * 4])
        ffn_inp = g.add(g.mul_mat(T["o"], att2), X)
        cur = g.mul(g.rms_norm(ffn_inp, eps), FN)
        ff = g.swiglu(g.mul_mat(T["gate"], cur), g.mul_mat(T["up"], cur))
        out = g.add(g.mul_mat(T["down"], ff), ffn_inp)
        assert g.compute() == gp.STATUS_SUCCESS
        y = g.get(out, np.float32, (1, H))
        assert gp.counter(plugin, "f32_gpu_sgemm_dispatch_count") == 7
        # nodes run inside another node's launch: both RMS_NORM + MUL pairs (4; Q4_K: the attention pair and the
        # FFN norm's MUL, 3);
        # k, v, both ROPEs and both SET_ROWS in the q launch (6); up and SWIGLU in the gate launch (2); the residual
        # ADDs of o and down (2)
        assert gp.counter(plugin, "fused_pair_count") == (14 if wt == gp.Q4_0 else 13)
        # o reads the row the attention merge writes, down the one the gate/up launch writes (the q/k/v launch and,
        # for Q4_0, the gate/up launch compute theirs inside; Q4_K's gate/up reads the one its norm launch writes)
        assert gp.counter(plugin, "act_quant_reuse_count") == (2 if wt == gp.Q4_0 else 3)

        # the oracle's chain of the same ops
        def q8(a):
            return orc.quantize_q8_K(a) if wt == gp.Q4_K else orc.quantize_q8_0(a, orc.Q8_X86)
        def mm(name, a):
            n_, kk_ = w[name].shape[0], w[name].shape[1] * bpw[0] // bpw[1]
            return orc.mul_mat(wt, w[name], n_, kk_, q8(a), 1)
        _, c = orc.rms_norm(x, eps, attn_norm)
        qr = orc.rope(mm("q", c).reshape(1, NH, D), np.array([pos_t], np.int32), D, 0, base)
        kr = orc.rope(mm("k", c).reshape(1, NKV, D), np.array([pos_t], np.int32), D, 0, base)
        kc2, vc2 = kc.copy(), vc.copy()
        kc2[pos_t] = kr.reshape(-1).astype(np.float16)
        vc2[pos_t] = mm("v", c).reshape(-1).astype(np.float16)
        kh = np.ascontiguousarray(kc2.reshape(CTX, NKV, D).transpose(1, 0, 2))
        vh = np.ascontiguousarray(vc2.reshape(CTX, NKV, D).transpose(1, 0, 2))
        a_ = orc.flash_attn_decode(qr.reshape(NH, D), kh.view(np.uint16), vh.view(np.uint16), 1.0 / np.sqrt(D))
        f_in = mm("o", a_.reshape(1, H)) + x
        _, c2 = orc.rms_norm(f_in, eps, ffn_norm)
        y_ref = mm("down", orc.swiglu(mm("gate", c2), mm("up", c2))) + f_in
        # the KV cache row written by SET_ROWS is the f16 of the roped K / V
        assert np.array_equal(g.get(KC, np.uint16, (CTX, NKV * D))[:pos_t], kc[:pos_t].view(np.uint16))
        assert rel_l2(g.get(KC, np.float16, (CTX, NKV * D))[pos_t], kc2[pos_t]) < 1e-3
        err = rel_l2(y, y_ref)
        assert err < 2e-3, err
    finally:
        g.free()


def test_graph_replay(plugin, orc):
    """A graph computed again unchanged is captured as a HIP graph on its second computation and replayed after that:
    every call reads its own inputs (each result matches the oracle, and a replay of earlier inputs the earlier result
    bit for bit), each call books the same counters, and a weight rewritten between calls is read in its new values
    (the capture is dropped and the weight repacked again)."""
    rng = np.random.default_rng(77)
    n, k = 1024, 4096
    wg = quantize(orc, gp.Q4_0, (rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    xs = [rng.standard_normal((1, k)).astype(np.float32) for _ in range(3)]
    r = rng.standard_normal((1, n)).astype(np.float32)
    g = gp.Graph(wg.nbytes + 4096, 16 << 20)
    try:
        W = g.tensor(gp.Q4_0, [k, n], "w", "w")
        X = g.tensor(gp.F32, [k, 1], "c", "x")
        R = g.tensor(gp.F32, [n, 1], "c", "r")
        g.set(W, wg)
        g.set(R, r)
        Y = g.add(g.mul_mat(W, X), R)  # the ADD runs in the GEMV's epilogue
        first = {}
        for call, i in enumerate([0, 1, 0, 2, 1, 1]):
            g.set(X, xs[i])
            plugin.ggml_backend_ameva_reset_counters()
            assert g.compute() == gp.STATUS_SUCCESS
            assert gp.counter(plugin, "f32_gpu_sgemm_dispatch_count") == 1
            assert gp.counter(plugin, "fused_pair_count") == 1
            y = g.get(Y, np.float32, (1, n))
            want = orc.mul_mat(gp.Q4_0, wg, n, k, orc.quantize_q8_0(xs[i], orc.Q8_X86), 1) + r
            assert rel_l2(y, want) < 1e-3, (call, i)
            if i in first:
                assert np.array_equal(y, first[i]), (call, i)
            else:
                first[i] = y
        w2 = quantize(orc, gp.Q4_0, (rng.standard_normal((n, k)) * 0.02).astype(np.float32))
        g.set(W, w2)
        g.set(X, xs[0])
        for _ in range(3):
            assert g.compute() == gp.STATUS_SUCCESS
            want = orc.mul_mat(gp.Q4_0, w2, n, k, orc.quantize_q8_0(xs[0], orc.Q8_X86), 1) + r
            assert rel_l2(g.get(Y, np.float32, (1, n)), want) < 1e-3
    finally:
        g.free()


@pytest.mark.parametrize("extra_reads", [False, True])
def test_node_groups_and_their_guards(plugin, orc, extra_reads):
    """The q/k/v (+ ROPE + SET_ROWS) and gate/up (+ SWIGLU) node groups run as one launch each, and only when nothing
    else reads their intermediate values: with a later MUL reading the un-rotated q and another reading the raw gate,
    the plugin runs the nodes one by one. Both graphs match the oracle's chain."""
    rng = np.random.default_rng(99)
    H, NH, NKV, D, FF, CTX, pos_t = 4096, 4, 2, 128, 1024, 64, 37
    def wq4(n, k):
        return orc.quantize_q4_0((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    w = {"q": wq4(NH * D, H), "k": wq4(NKV * D, H), "v": wq4(NKV * D, H), "gate": wq4(FF, H), "up": wq4(FF, H),
         "down": wq4(H, FF)}
    x = rng.standard_normal((1, H)).astype(np.float32)
    e_q = rng.standard_normal((1, NH * D)).astype(np.float32)
    e_g = rng.standard_normal((1, FF)).astype(np.float32)
    kc = rng.standard_normal((CTX, NKV * D)).astype(np.float16)
    vc = rng.standard_normal((CTX, NKV * D)).astype(np.float16)
    g = gp.Graph(sum(a.nbytes for a in w.values()) + 8 * 4096, 16 << 20)
    try:
        T = {k_: g.tensor(gp.Q4_0, [a.shape[1] * 32 // 18, a.shape[0]], "w", k_) for k_, a in w.items()}
        for k_, a in w.items():
            g.set(T[k_], a)
        X = g.tensor(gp.F32, [H, 1], "c", "x")
        g.set(X, x)
        EQ, EG = g.tensor(gp.F32, [NH * D, 1], "c", "eq"), g.tensor(gp.F32, [FF, 1], "c", "eg")
        g.set(EQ, e_q)
        g.set(EG, e_g)
        POS, IDX = g.tensor(gp.I32, [1], "c", "pos"), g.tensor(gp.I64, [1], "c", "idx")
        g.set(POS, np.array([pos_t], np.int32))
        g.set(IDX, np.array([pos_t], np.int64))
        KC, VC = g.tensor(gp.F16, [NKV * D, CTX], "c", "kc"), g.tensor(gp.F16, [NKV * D, CTX], "c", "vc")
        g.set(KC, kc)
        g.set(VC, vc)
        q_raw = g.mul_mat(T["q"], X)
        q = g.rope(g.reshape_3d(q_raw, D, NH, 1), POS, D, 0, 500000.0)
        k = g.rope(g.reshape_3d(g.mul_mat(T["k"], X), D, NKV, 1), POS, D, 0, 500000.0)
        v = g.mul_mat(T["v"], X)
        g.set_rows(KC, g.view_nd(k, gp.OP_RESHAPE, [NKV * D, 1], [4, NKV * D * 4, NKV * D * 4, NKV * D * 4]), IDX)
        g.set_rows(VC, v, IDX)
        gate = g.mul_mat(T["gate"], X)
        ff = g.swiglu(gate, g.mul_mat(T["up"], X))
        y = g.mul_mat(T["down"], ff)
        if extra_reads:
            yq, yg = g.mul(q_raw, EQ), g.mul(gate, EG)
        plugin.ggml_backend_ameva_reset_counters()
        assert g.compute() == gp.STATUS_SUCCESS
        fused = gp.counter(plugin, "fused_pair_count")
        assert gp.counter(plugin, "f32_gpu_sgemm_dispatch_count") == 6
        if extra_reads:
            assert fused < 8
        else:
            assert fused == 8  # k, v, both ROPEs and both SET_ROWS in the q launch; up and SWIGLU in the gate launch

        q8 = lambda a: orc.quantize_q8_0(a, orc.Q8_X86)  # noqa: E731
        def mm(name, a):
            n_, kk_ = w[name].shape[0], w[name].shape[1] * 32 // 18
            return orc.mul_mat(gp.Q4_0, w[name], n_, kk_, q8(a), 1)
        qm, km, gm = mm("q", x), mm("k", x), mm("gate", x)
        qr = orc.rope(qm.reshape(1, NH, D), np.array([pos_t], np.int32), D, 0, 500000.0)
        kr = orc.rope(km.reshape(1, NKV, D), np.array([pos_t], np.int32), D, 0, 500000.0)
        assert rel_l2(g.get(q, np.float32, (1, NH, D)), qr) < 1e-3
        assert rel_l2(g.get(v, np.float32, (1, NKV * D)), mm("v", x)) < 1e-3
        kc_out = g.get(KC, np.float16, (CTX, NKV * D))
        assert np.array_equal(np.delete(kc_out, pos_t, axis=0).view(np.uint16), np.delete(kc, pos_t, axis=0).view(np.uint16))
        assert rel_l2(kc_out[pos_t], kr.reshape(-1).astype(np.float16)) < 1e-3
        assert rel_l2(g.get(VC, np.float16, (CTX, NKV * D))[pos_t], mm("v", x).reshape(-1).astype(np.float16)) < 1e-3
        h = orc.swiglu(gm, mm("up", x))
        assert rel_l2(g.get(ff, np.float32, (1, FF)), h) < 1e-3
        assert rel_l2(g.get(y, np.float32, (1, H)), mm("down", h)) < 2e-3
        if extra_reads:
            assert rel_l2(g.get(yq, np.float32, (1, NH * D)), qm * e_q) < 1e-3
            assert rel_l2(g.get(yg, np.float32, (1, FF)), gm * e_g) < 1e-3
    finally:
        g.free()


def test_qkv_group_declined_when_outputs_share_memory(plugin, orc):
    """ggml-alloc places a node's output in the memory of a tensor that is dead by then in the graph's node order. With
    the nodes ordered k MUL_MAT, k ROPE, k SET_ROWS, q MUL_MAT, q ROPE, v MUL_MAT, v SET_ROWS, the roped q may take the
    memory of the roped k, which SET_ROWS has consumed: correct node by node, but one launch writing q and k at once
    would lose one of them. The plugin then declines the q/k/v node group and runs the nodes one by one: the q values,
    both cache rows and v match the oracle."""
    rng = np.random.default_rng(123)
    H, NH, NKV, D, CTX, pos_t = 4096, 2, 2, 128, 48, 29
    def wq4(n, k):
        return orc.quantize_q4_0((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    w = {"q": wq4(NH * D, H), "k": wq4(NKV * D, H), "v": wq4(NKV * D, H)}
    x = rng.standard_normal((1, H)).astype(np.float32)
    kc = rng.standard_normal((CTX, NKV * D)).astype(np.float16)
    vc = rng.standard_normal((CTX, NKV * D)).astype(np.float16)
    g = gp.Graph(sum(a.nbytes for a in w.values()) + 4 * 4096, 8 << 20)
    try:
        T = {k_: g.tensor(gp.Q4_0, [H, a.shape[0]], "w", k_) for k_, a in w.items()}
        for k_, a in w.items():
            g.set(T[k_], a)
        X = g.tensor(gp.F32, [H, 1], "c", "x")
        g.set(X, x)
        POS, IDX = g.tensor(gp.I32, [1], "c", "pos"), g.tensor(gp.I64, [1], "c", "idx")
        g.set(POS, np.array([pos_t], np.int32))
        g.set(IDX, np.array([pos_t], np.int64))
        KC, VC = g.tensor(gp.F16, [NKV * D, CTX], "c", "kc"), g.tensor(gp.F16, [NKV * D, CTX], "c", "vc")
        g.set(KC, kc)
        g.set(VC, vc)
        k = g.rope(g.reshape_3d(g.mul_mat(T["k"], X), D, NKV, 1), POS, D, 0, 500000.0)
        g.set_rows(KC, g.view_nd(k, gp.OP_RESHAPE, [NKV * D, 1], [4, NKV * D * 4, NKV * D * 4, NKV * D * 4]), IDX)
        q = g.rope(g.reshape_3d(g.mul_mat(T["q"], X), D, NH, 1), POS, D, 0, 500000.0)
        q.data = k.data  # the roped k is dead after its SET_ROWS: gallocr may hand its memory to the roped q
        v = g.mul_mat(T["v"], X)
        g.set_rows(VC, v, IDX)
        plugin.ggml_backend_ameva_reset_counters()
        assert g.compute() == gp.STATUS_SUCCESS
        assert gp.counter(plugin, "fused_pair_count") == 0  # no group: q would overwrite k inside one launch
        assert gp.counter(plugin, "f32_gpu_sgemm_dispatch_count") == 3

        def mm(name):
            return orc.mul_mat(gp.Q4_0, w[name], w[name].shape[0], H, orc.quantize_q8_0(x, orc.Q8_X86), 1)
        p = np.array([pos_t], np.int32)
        qr = orc.rope(mm("q").reshape(1, NH, D), p, D, 0, 500000.0)
        kr = orc.rope(mm("k").reshape(1, NKV, D), p, D, 0, 500000.0)
        assert rel_l2(g.get(q, np.float32, (1, NH, D)), qr) < 1e-3
        assert rel_l2(g.get(v, np.float32, (1, NKV * D)), mm("v")) < 1e-3
        kc_out = g.get(KC, np.float16, (CTX, NKV * D))
        assert rel_l2(kc_out[pos_t], kr.reshape(-1).astype(np.float16)) < 1e-3
        assert np.array_equal(np.delete(kc_out, pos_t, axis=0).view(np.uint16),
                              np.delete(kc, pos_t, axis=0).view(np.uint16))
        assert rel_l2(g.get(VC, np.float16, (CTX, NKV * D))[pos_t], mm("v").reshape(-1).astype(np.float16)) < 1e-3
    finally:
        g.free()


@pytest.mark.parametrize("guard", ["none", "extra_read", "output_flag", "x_shared"])
def test_norm_fold_and_its_guards(plugin, orc, guard):
    """RMS_NORM + MUL before a Q4_0 q/k/v or gate/up node group at K = 4096 runs inside that group's launch, and only
    when its product is read by nothing else, is not a graph output and no output of the group shares the norm
    input's memory: a later MUL reading the normed row, the OUTPUT flag on it, or the SWIGLU output placed over the
    FFN input each make the plugin run the norm as a launch of its own. Every graph matches the oracle's chain."""
    rng = np.random.default_rng(321)
    H, NH, NKV, D, FF, CTX, pos_t = 4096, 4, 2, 128, 1024, 64, 41
    eps, base = 1e-5, 500000.0
    def wq4(n, k):
        return orc.quantize_q4_0((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    w = {"q": wq4(NH * D, H), "k": wq4(NKV * D, H), "v": wq4(NKV * D, H), "gate": wq4(FF, H), "up": wq4(FF, H),
         "down": wq4(H, FF)}
    x = rng.standard_normal((1, H)).astype(np.float32)
    x2 = rng.standard_normal((1, H)).astype(np.float32)
    an = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    fn = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    e = rng.standard_normal((1, H)).astype(np.float32)
    kc = rng.standard_normal((CTX, NKV * D)).astype(np.float16)
    vc = rng.standard_normal((CTX, NKV * D)).astype(np.float16)
    g = gp.Graph(sum(a.nbytes for a in w.values()) + 16 * 4096, 16 << 20)
    try:
        T = {k_: g.tensor(gp.Q4_0, [a.shape[1] * 32 // 18, a.shape[0]], "w", k_) for k_, a in w.items()}
        for k_, a in w.items():
            g.set(T[k_], a)
        AN, FN = g.tensor(gp.F32, [H], "w", "an"), g.tensor(gp.F32, [H], "w", "fn")
        g.set(AN, an)
        g.set(FN, fn)
        X, X2, E = g.tensor(gp.F32, [H, 1], "c", "x"), g.tensor(gp.F32, [H, 1], "c", "x2"), g.tensor(gp.F32, [H, 1], "c", "e")
        g.set(X, x)
        g.set(X2, x2)
        g.set(E, e)
        POS, IDX = g.tensor(gp.I32, [1], "c", "pos"), g.tensor(gp.I64, [1], "c", "idx")
        g.set(POS, np.array([pos_t], np.int32))
        g.set(IDX, np.array([pos_t], np.int64))
        KC, VC = g.tensor(gp.F16, [NKV * D, CTX], "c", "kc"), g.tensor(gp.F16, [NKV * D, CTX], "c", "vc")
        g.set(KC, kc)
        g.set(VC, vc)
        cur = g.mul(g.rms_norm(X, eps), AN)
        q = g.rope(g.reshape_3d(g.mul_mat(T["q"], cur), D, NH, 1), POS, D, 0, base)
        k = g.rope(g.reshape_3d(g.mul_mat(T["k"], cur), D, NKV, 1), POS, D, 0, base)
        v = g.mul_mat(T["v"], cur)
        g.set_rows(KC, g.view_nd(k, gp.OP_RESHAPE, [NKV * D, 1], [4, NKV * D * 4, NKV * D * 4, NKV * D * 4]), IDX)
        g.set_rows(VC, v, IDX)
        cur2 = g.mul(g.rms_norm(X2, eps), FN)
        ff = g.swiglu(g.mul_mat(T["gate"], cur2), g.mul_mat(T["up"], cur2))
        y = g.mul_mat(T["down"], ff)  # the one-row GEMV the gate/up group writes the activation row for
        if guard == "extra_read":
            ye = g.mul(cur, E)
        elif guard == "output_flag":
            cur2.flags = 2  # GGML_TENSOR_FLAG_OUTPUT
        elif guard == "x_shared":
            ff.data = X2.data  # the SWIGLU output over the FFN norm's input (dead after the norm in node order)
        plugin.ggml_backend_ameva_reset_counters()
        assert g.compute() == gp.STATUS_SUCCESS
        fused = gp.counter(plugin, "fused_pair_count")
        # folded: the norm, its MUL, k, v, both ROPEs and both SET_ROWS in the q launch (8); the norm, its MUL, up and
        # SWIGLU in the gate launch (4); a declined fold keeps the RMS_NORM + MUL pair (1) before its group
        assert fused == {"none": 12, "extra_read": 7 + 4, "output_flag": 8 + 3, "x_shared": 8 + 3}[guard]

        q8 = lambda a: orc.quantize_q8_0(a, orc.Q8_X86)  # noqa: E731
        def mm(name, a):
            return orc.mul_mat(gp.Q4_0, w[name], w[name].shape[0], H, q8(a), 1)
        _, c = orc.rms_norm(x, eps, an)
        _, c2 = orc.rms_norm(x2, eps, fn)
        p = np.array([pos_t], np.int32)
        qr = orc.rope(mm("q", c).reshape(1, NH, D), p, D, 0, base)
        kr = orc.rope(mm("k", c).reshape(1, NKV, D), p, D, 0, base)
        assert rel_l2(g.get(q, np.float32, (1, NH, D)), qr) < 1e-3
        assert rel_l2(g.get(KC, np.float16, (CTX, NKV * D))[pos_t], kr.reshape(-1).astype(np.float16)) < 1e-3
        assert rel_l2(g.get(VC, np.float16, (CTX, NKV * D))[pos_t], mm("v", c).reshape(-1).astype(np.float16)) < 1e-3
        h = orc.swiglu(mm("gate", c2), mm("up", c2))
        assert rel_l2(g.get(ff, np.float32, (1, FF)), h) < 1e-3
        assert rel_l2(g.get(y, np.float32, (1, H)), orc.mul_mat(gp.Q4_0, w["down"], H, FF, q8(h), 1)) < 2e-3
        if guard == "extra_read":
            assert rel_l2(g.get(ye, np.float32, (1, H)), c * e) < 1e-6
        if guard == "output_flag":
            assert rel_l2(g.get(cur2, np.float32, (1, H)), c2) < 1e-6
    finally:
        g.free()
