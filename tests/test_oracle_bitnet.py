"""Pins the oracle's restatement of the BitNet b1.58 CPU token step (llama_bitnet_core.cpp:886-1300) before the GPU
engine is compared with it: rms_norm, the f16 GEMV and the attention against float64 closed forms; the token step
through structural facts a mistake would break: a model of zero projections leaves the residual stream unchanged and
its logits are the closed-form LM head of the normalized input; at position 0 the attention returns V exactly (one
key, weight 1), so with an identity output projection the residual gains exactly the int8 V; a later position reads
the cache rows written before it (the float64 attention over the oracle's own cache)."""
import numpy as np
import pytest


def rel(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def i2s_pack(codes):
    """codes [rows, k] in 0..3 -> BitNet I2_S bytes (byte i of a 128-block: weights i, 32+i, 64+i, 96+i)."""
    rows, k = codes.shape
    blk = codes.reshape(rows, k // 128, 4, 32).astype(np.uint8)
    return ((blk[:, :, 0] << 6) | (blk[:, :, 1] << 4) | (blk[:, :, 2] << 2) | blk[:, :, 3]).reshape(rows, k // 4)


def test_rms_norm_gemv_f16_attention_closed_forms(orc):
    rng = np.random.default_rng(1)
    x = rng.standard_normal(2560).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(2560)).astype(np.float32)
    want = x.astype(np.float64) / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-5) * w
    assert rel(orc.bitnet_rms_norm(x, w, 1e-5), want) < 1e-5
    assert rel(orc.bitnet_rms_norm(x, None, 1e-5), want / w) < 1e-5
    W = rng.standard_normal((300, 2560)).astype(np.float16)
    assert rel(orc.bitnet_gemv_f16(W.view(np.uint16), x), W.astype(np.float64) @ x) < 1e-5
    H, KVH, hd, pos = 8, 2, 128, 40
    q = rng.standard_normal((H, hd)).astype(np.float32)
    kc = rng.standard_normal((64, KVH * hd)).astype(np.float32)
    vc = rng.standard_normal((64, KVH * hd)).astype(np.float32)
    out = orc.bitnet_attention(q, kc, vc, pos, KVH)
    ref = np.empty((H, hd))
    for h in range(H):
        kh = kc[: pos + 1].reshape(pos + 1, KVH, hd)[:, h // (H // KVH)].astype(np.float64)
        vh = vc[: pos + 1].reshape(pos + 1, KVH, hd)[:, h // (H // KVH)].astype(np.float64)
        s = kh @ q[h] / np.sqrt(hd)
        p = np.exp(s - s.max())
        ref[h] = p @ vh / p.sum()
    assert rel(out, ref) < 1e-5


def small_cfg(relu2=True):
    return dict(n_embd=256, n_ffn=512, n_heads=2, n_kv_heads=1, head_dim=128, n_ctx=16, norm_eps=1e-5,
                rope_theta=10000.0, relu2=relu2)


def zero_layer(cfg):
    E, F, kv = cfg["n_embd"], cfg["n_ffn"], cfg["n_kv_heads"] * cfg["head_dim"]
    z = lambda r, k: i2s_pack(np.ones((r, k), np.uint8))  # noqa: E731  code 1 = weight 0
    return dict(attn_norm=np.ones(E, np.float32), ffn_norm=np.ones(E, np.float32),
                ffn_sub_norm=np.ones(F, np.float32) if cfg["relu2"] else None,
                wq=z(E, E), wk=z(kv, E), wv=z(kv, E), wo=z(E, E), w_gate=z(F, E), w_up=z(F, E), w_down=z(E, F))


def test_token_of_zero_projections(orc):
    cfg = small_cfg()
    rng = np.random.default_rng(2)
    E = cfg["n_embd"]
    out_norm = (1 + 0.1 * rng.standard_normal(E)).astype(np.float32)
    head = (rng.standard_normal((50, E)) * 0.1).astype(np.float16)
    m = orc.BitnetModel(cfg, [zero_layer(cfg), zero_layer(cfg)], out_norm, head.view(np.uint16))
    x = rng.standard_normal(E).astype(np.float32)
    y, logits = m.token(3, x)
    assert np.array_equal(y, x)
    xn = x.astype(np.float64) / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-5) * out_norm
    assert rel(logits, head.astype(np.float64) @ xn) < 1e-5
    assert not m.kc.any() and not m.vc.any()


def test_token_attention_of_one_key_is_v(orc):
    """Layer: random wv, identity wo (code 2 on the diagonal), zero elsewhere, no attention sub norm: at position 0
    x_out = x + q8(v) * dequant exactly, with v = the V projection of the int8 normalized input."""
    cfg = small_cfg(relu2=False)
    E, kv = cfg["n_embd"], cfg["n_kv_heads"] * cfg["head_dim"]
    rng = np.random.default_rng(3)
    L = zero_layer(cfg)
    codes_v = rng.integers(0, 3, (kv, E)).astype(np.uint8)
    L["wv"] = i2s_pack(codes_v)
    eye = np.ones((E, E), np.uint8)
    np.fill_diagonal(eye, 2)
    L["wo"] = i2s_pack(eye)
    L["scale_wv"] = 0.75
    m = orc.BitnetModel(cfg, [L], np.ones(E, np.float32), np.zeros((1, E), np.uint16))
    x = rng.standard_normal(E).astype(np.float32)
    y, _ = m.token(0, x, logits=False)
    xn = orc.bitnet_rms_norm(x, L["attn_norm"], 1e-5)
    q8 = np.empty(E, np.int8)
    dq = orc.lib().orc_i2s_quantize_act(xn.ctypes.data, q8.ctypes.data, E)
    v = ((codes_v.astype(np.int64) - 1) @ q8.astype(np.int64)).astype(np.float32) * np.float32(dq * np.float32(0.75))
    att = np.ascontiguousarray(np.tile(v, cfg["n_heads"] // cfg["n_kv_heads"]), np.float32)  # G heads, one KV head
    qa = np.empty(E, np.int8)
    da = orc.lib().orc_i2s_quantize_act(att.ctypes.data, qa.ctypes.data, E)
    assert np.array_equal(m.vc[0, 0], v)
    assert np.array_equal(y, x + qa.astype(np.float32) * np.float32(da))


def test_token_reads_earlier_cache_rows(orc):
    cfg = small_cfg()
    E, F, kv, hd = cfg["n_embd"], cfg["n_ffn"], cfg["n_kv_heads"] * cfg["head_dim"], cfg["head_dim"]
    rng = np.random.default_rng(4)
    r = lambda a, b: i2s_pack(rng.integers(0, 3, (a, b)).astype(np.uint8))  # noqa: E731
    L = dict(attn_norm=np.ones(E, np.float32), attn_sub_norm=np.ones(E, np.float32), ffn_norm=np.ones(E, np.float32),
             ffn_sub_norm=np.ones(F, np.float32), wq=r(E, E), wk=r(kv, E), wv=r(kv, E), wo=r(E, E),
             w_gate=r(F, E), w_up=r(F, E), w_down=r(E, F))
    m = orc.BitnetModel(cfg, [L], np.ones(E, np.float32), np.zeros((1, E), np.uint16))
    for p in range(4):
        m.token(p, rng.standard_normal(E).astype(np.float32), logits=False)
    assert np.count_nonzero(m.kc[0, :4].any(axis=1)) == 4 and not m.kc[0, 4:].any()
    # the attention the oracle computes at position 3 over its own cache equals the float64 closed form
    q = rng.standard_normal((cfg["n_heads"], hd)).astype(np.float32)
    got = orc.bitnet_attention(q, m.kc[0], m.vc[0], 3, cfg["n_kv_heads"])
    s = m.kc[0, :4].astype(np.float64) @ q.astype(np.float64).T / np.sqrt(hd)   # [4, H] (one KV head)
    p = np.exp(s - s.max(axis=0))
    ref = (p / p.sum(axis=0)).T @ m.vc[0, :4].astype(np.float64)
    assert rel(got, ref) < 1e-5
