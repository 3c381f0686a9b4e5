"""The decode step of ameva_compute_amd.llama.LlamaLayer (stacked q/k/v and gate/up weights, fused norm+quant) against
the oracle's chain of the same ops at the Llama-3-8B shape, and its HIP-graph replay against eager execution."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def test_layer_decode_vs_oracle_and_graph_replay(dev, orc):
    from ameva_compute_amd import ops
    from ameva_compute_amd.llama import LlamaLayer
    rng = np.random.default_rng(77)
    H, NH, NKV, D, FF, CTX = 4096, 32, 8, 128, 14336, 4096
    eps, base = 1e-5, 500000.0
    def wq4(n, k):
        return orc.quantize_q4_0((rng.standard_normal((n, k)) * 0.02).astype(np.float32))
    w = {"q": wq4(NH * D, H), "k": wq4(NKV * D, H), "v": wq4(NKV * D, H), "o": wq4(H, H), "gate": wq4(FF, H),
         "up": wq4(FF, H), "down": wq4(H, FF)}
    an = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    fn = (1 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    g = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
    layer = LlamaLayer(ops.QWeight.from_ggml(ops.Q4_0, g(np.concatenate([w["q"], w["k"], w["v"]])), H + 2 * NKV * D, H),
                       ops.QWeight.from_ggml(ops.Q4_0, g(w["o"]), H, H),
                       ops.QWeight.from_ggml(ops.Q4_0, g(np.concatenate([w["gate"], w["up"]])), 2 * FF, H),
                       ops.QWeight.from_ggml(ops.Q4_0, g(w["down"]), H, FF), g(an), g(fn), ctx=CTX)
    kc = rng.standard_normal((CTX, NKV * D)).astype(np.float16)
    vc = rng.standard_normal((CTX, NKV * D)).astype(np.float16)
    layer.k_cache.copy_(g(kc))
    layer.v_cache.copy_(g(vc))
    pos = 3000
    layer.set_position(pos)
    x = rng.standard_normal(H).astype(np.float32)
    xg, out = g(x), torch.empty(H, dtype=torch.float32, device=dev)
    layer.decode(xg, out)
    torch.cuda.synchronize()
    y = out.cpu().numpy()
    # the fused launches (RoPE + KV store, GEMV epilogues) compute exactly what one launch per graph node computes
    out_u = torch.empty_like(out)
    layer.decode(xg, out_u, fused=False)
    torch.cuda.synchronize()
    assert torch.equal(out_u, out)

    q8 = lambda a: orc.quantize_q8_0(a.reshape(1, -1), orc.Q8_X86)  # noqa: E731
    def mm(name, a):
        n_, k_ = w[name].shape[0], w[name].shape[1] * 32 // 18
        return orc.mul_mat(orc.Q4_0, w[name], n_, k_, q8(a), 1).reshape(-1)
    cpu = lambda t: t.float().cpu().numpy().reshape(-1)  # noqa: E731
    p = np.array([pos], np.int32)

    # stage by stage: each kernel against the oracle fed the GPU's own input to that stage (the f32 / FA bars)
    _, c = orc.rms_norm(x.reshape(1, H), eps, an)
    assert rel_l2(cpu(layer.t_o), c) < 1e-6
    qkv_g = cpu(layer.qkv)
    q_in = np.concatenate([mm("q", cpu(layer.t_o)), mm("k", cpu(layer.t_o))])
    qk_ref = orc.rope(q_in.reshape(1, NH + NKV, D), p, D, 0, base).reshape(-1)
    assert rel_l2(qkv_g[: H + NKV * D], qk_ref) < 1e-3
    assert rel_l2(qkv_g[H + NKV * D:], mm("v", cpu(layer.t_o))) < 1e-3
    kc2, vc2 = kc.copy(), vc.copy()
    kc2[pos] = qkv_g[H:H + NKV * D].astype(np.float16)
    vc2[pos] = qkv_g[H + NKV * D:].astype(np.float16)
    assert np.array_equal(layer.k_cache[pos].cpu().numpy(), kc2[pos])
    assert np.array_equal(layer.v_cache[pos].cpu().numpy(), vc2[pos])
    assert np.array_equal(layer.k_cache[:pos].cpu().numpy().view(np.uint16), kc[:pos].view(np.uint16))
    kh = np.ascontiguousarray(kc2[: pos + 1].reshape(pos + 1, NKV, D).transpose(1, 0, 2))
    vh = np.ascontiguousarray(vc2[: pos + 1].reshape(pos + 1, NKV, D).transpose(1, 0, 2))
    att_ref = orc.flash_attn_decode(qkv_g[:H].reshape(NH, D), kh.view(np.uint16), vh.view(np.uint16),
                                    1.0 / np.sqrt(D)).reshape(-1)
    assert rel_l2(cpu(layer.att), att_ref) < 2e-3
    x1_ref = mm("o", cpu(layer.att)) + x
    assert rel_l2(cpu(layer.x1), x1_ref) < 1e-3
    _, c2 = orc.rms_norm(cpu(layer.x1).reshape(1, H), eps, fn)
    assert rel_l2(cpu(layer.t_o2), c2) < 1e-6
    gu_ref = np.concatenate([mm("gate", cpu(layer.t_o2)), mm("up", cpu(layer.t_o2))])
    assert rel_l2(cpu(layer.gu), gu_ref) < 1e-3
    h_ref = orc.swiglu(cpu(layer.gu)[:FF], cpu(layer.gu)[FF:])
    assert rel_l2(cpu(layer.h), h_ref) < 1e-6
    y_stage = mm("down", cpu(layer.h)) + cpu(layer.x1)
    assert rel_l2(y, y_stage) < 1e-3

    # end to end against the oracle's own chain: the requantizations between the stages (three Q8_0 and one f16
    # rounding of inputs that already differ by f32 rounding) let the two chains drift apart beyond a single op's bar
    _, c = orc.rms_norm(x.reshape(1, H), eps, an)
    qr = orc.rope(mm("q", c).reshape(1, NH, D), p, D, 0, base).reshape(NH, D)
    kr = orc.rope(mm("k", c).reshape(1, NKV, D), p, D, 0, base).reshape(-1)
    ko, vo = kc.copy(), vc.copy()
    ko[pos], vo[pos] = kr.astype(np.float16), mm("v", c).astype(np.float16)
    kh = np.ascontiguousarray(ko[: pos + 1].reshape(pos + 1, NKV, D).transpose(1, 0, 2))
    vh = np.ascontiguousarray(vo[: pos + 1].reshape(pos + 1, NKV, D).transpose(1, 0, 2))
    att = orc.flash_attn_decode(qr, kh.view(np.uint16), vh.view(np.uint16), 1.0 / np.sqrt(D)).reshape(-1)
    x1 = mm("o", att) + x
    _, c2 = orc.rms_norm(x1.reshape(1, H), eps, fn)
    y_ref = mm("down", orc.swiglu(mm("gate", c2), mm("up", c2))) + x1
    err = rel_l2(y, y_ref)
    print(f"layer end-to-end rel L2 {err:.2e}; att {rel_l2(cpu(layer.att), att):.2e}; x1 {rel_l2(cpu(layer.x1), x1):.2e}")
    assert err < 1e-2, err

    # the same step captured in a HIP graph and replayed matches the eager result on every replay
    gr = torch.cuda.CUDAGraph()
    out2 = torch.empty_like(out)
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        layer.decode(xg, out2)  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    with torch.cuda.graph(gr):
        layer.decode(xg, out2)
    for _ in range(3):
        out2.zero_()
        torch.cuda.synchronize()
        gr.replay()
        torch.cuda.synchronize()
        assert torch.equal(out2, out)


@pytest.mark.parametrize("n_tok,pos0", [(8, 1000), (512, 0), (77, 300)])
def test_layer_prefill_matches_decode_steps(dev, n_tok, pos0):
    """A prompt chunk through LlamaLayer.prefill (int8-MFMA MUL_MATs, f16-MFMA causal attention, fused SWIGLU+Q8_0)
    against the same tokens decoded one by one (the path checked against the oracle above): each token's output and
    the K/V rows written agree within the chain bar (the two paths round and sum in different orders: MFMA vs GEMV
    accumulation, f16 vs f32 probabilities)."""
    from ameva_compute_amd.llama import random_layer
    layer = random_layer(dev, seed=11, ctx=1024)
    g = torch.Generator(device=dev)
    g.manual_seed(3)
    layer.k_cache.copy_(torch.randn(layer.k_cache.shape, generator=g, device=dev).half())
    layer.v_cache.copy_(torch.randn(layer.v_cache.shape, generator=g, device=dev).half())
    k0, v0 = layer.k_cache.clone(), layer.v_cache.clone()
    x = torch.randn((n_tok, layer.H), generator=g, device=dev)
    out_p = torch.empty_like(x)
    layer.set_prefill_position(pos0, n_tok)
    layer.prefill(x, out_p)
    torch.cuda.synchronize()
    kp, vp = layer.k_cache.clone(), layer.v_cache.clone()
    layer.k_cache.copy_(k0)
    layer.v_cache.copy_(v0)
    out_d = torch.empty_like(x)
    for t in range(n_tok):
        layer.set_position(pos0 + t)
        layer.decode(x[t].contiguous(), out_d[t])
    torch.cuda.synchronize()
    e = rel_l2(out_p.cpu().numpy(), out_d.cpu().numpy())
    worst = max(rel_l2(out_p[t].cpu().numpy(), out_d[t].cpu().numpy()) for t in range(n_tok))
    print(f"prefill vs decode: rel L2 {e:.2e}, worst token {worst:.2e}")
    assert e < 1e-2 and worst < 2e-2
    rows = slice(pos0, pos0 + n_tok)
    assert rel_l2(kp[rows].float().cpu().numpy(), layer.k_cache[rows].float().cpu().numpy()) < 1e-2
    assert rel_l2(vp[rows].float().cpu().numpy(), layer.v_cache[rows].float().cpu().numpy()) < 1e-2
    assert torch.equal(kp[:pos0], k0[:pos0]) and torch.equal(kp[pos0 + n_tok:], k0[pos0 + n_tok:])


def _fill_caches(layer, dev, seed):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    layer.k_cache.copy_(torch.randn(layer.k_cache.shape, generator=g, device=dev).half())
    layer.v_cache.copy_(torch.randn(layer.v_cache.shape, generator=g, device=dev).half())
    return g


@pytest.mark.parametrize("wtype", [2, 12])
def test_fused_chain_matches_unfused(dev, wtype):
    """Two chained layers, fused (Q4_0: 6 launches per layer, each RMS_NORM folded into the GEMV after it; Q4_K: 8,
    the first layer's step ending with the second layer's attention norm and its activation row) against one launch
    per node: identical outputs, K/V rows and activation rows, for Q4_0 (Q8_0 activations) and Q4_K (Q8_K
    activations) weights."""
    from ameva_compute_amd.llama import random_layer
    layers = [random_layer(dev, seed=21 + i, ctx=512, wtype=wtype) for i in range(2)]
    for i, lay in enumerate(layers):
        _fill_caches(lay, dev, 40 + i)
        lay.set_position(300)
    k0 = [lay.k_cache.clone() for lay in layers]
    v0 = [lay.v_cache.clone() for lay in layers]
    g = torch.Generator(device=dev)
    g.manual_seed(9)
    x = torch.randn(layers[0].H, generator=g, device=dev)
    mid, out = torch.empty_like(x), torch.empty_like(x)
    layers[0].decode(x, mid, fused=False)
    layers[1].decode(mid, out, fused=False)
    torch.cuda.synchronize()
    ref = (mid.clone(), out.clone(), [lay.k_cache.clone() for lay in layers], [lay.v_cache.clone() for lay in layers],
           [lay.act_ff.clone() for lay in layers], layers[1].act_h.clone())
    for i, lay in enumerate(layers):
        lay.k_cache.copy_(k0[i])
        lay.v_cache.copy_(v0[i])
    layers[0].decode(x, mid, fused=True, next_layer=layers[1])
    layers[1].decode(mid, out, fused=True, act_ready=True)
    torch.cuda.synchronize()
    assert torch.equal(mid, ref[0]) and torch.equal(out, ref[1])
    for i, lay in enumerate(layers):
        assert torch.equal(lay.k_cache, ref[2][i]) and torch.equal(lay.v_cache, ref[3][i])
        assert torch.equal(lay.act_ff, ref[4][i])
    if not layers[1].fold_attn:  # a folded norm keeps its activation row in LDS
        assert torch.equal(layers[1].act_h, ref[5])


def test_decode_graph_replays_at_growing_positions(dev):
    """One fused decode step captured once and replayed at positions p .. p + 5 (position, cache row and key count
    live in device memory): every replay equals the eager step at that position, K/V rows included."""
    from ameva_compute_amd.llama import random_layer
    layer = random_layer(dev, seed=5, ctx=1024)
    g = _fill_caches(layer, dev, 8)
    k0, v0 = layer.k_cache.clone(), layer.v_cache.clone()
    xs = [torch.randn(layer.H, generator=g, device=dev) for _ in range(6)]
    x, out = torch.empty(layer.H, device=dev), torch.empty(layer.H, device=dev)
    p0 = 700
    eager = []
    for i in range(6):
        layer.set_position(p0 + i)
        x.copy_(xs[i])
        layer.decode(x, out)
        eager.append(out.clone())
    torch.cuda.synchronize()
    k_e, v_e = layer.k_cache.clone(), layer.v_cache.clone()
    layer.k_cache.copy_(k0)
    layer.v_cache.copy_(v0)
    layer.set_position(p0)
    x.copy_(xs[0])
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        layer.decode(x, out)  # warm-up on the capture stream (rewrites row p0 with the same values)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        layer.decode(x, out)
    for i in range(6):
        layer.set_position(p0 + i)
        x.copy_(xs[i])
        out.zero_()
        torch.cuda.synchronize()
        gr.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager[i]), i
    assert torch.equal(layer.k_cache, k_e) and torch.equal(layer.v_cache, v_e)
