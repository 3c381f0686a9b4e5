"""Quantized KV cache on the GPU (the reference's ameva_set_rows_q.comp and the Q8_0 / Q4_0 paths of
ameva_flash_attn.comp:104-136): SET_ROWS f32 -> Q8_0 (three rounding rules) / Q4_0 bit for bit against the oracle's
quantizers, with index scatter, row strides and out-of-range indices; FLASH_ATTN_EXT decode over Q8_0 / Q4_0 caches
against the oracle's restatement of ggml's CPU kernel (q quantized to Q8_0, integer block dots, V dequantized) within
1e-4 relative L2 (f32 arithmetic throughout; the BASELINE attention bar is 2e-3), for every GQA group, with masks,
cache layouts of llama.cpp (token-major rows of all KV heads) and head-major, the key count from device memory, and
the one-launch merge equal to the two-launch one."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

Q8_0, Q4_0, F16 = 8, 2, 1


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


def quant(orc, t, x, rule=0):
    return orc.quantize_q8_0(x, rule) if t == Q8_0 else orc.quantize_q4_0(x)


@pytest.mark.parametrize("t,rule", [(Q8_0, 0), (Q8_0, 1), (Q8_0, 2), (Q4_0, 0)])
def test_set_rows_quantized(dev, ops, orc, t, rule):
    rng = np.random.default_rng(10 + t + rule)
    n, rows, dst_rows = 1024, 7, 20
    x = rng.standard_normal((rows, n)).astype(np.float32)
    x[1] = 0.0                                   # an all-zero row
    x[2, :32] = np.linspace(-2, 2, 32)           # exact halves: rounding ties
    x[3] *= 1e-6
    rb = n // 32 * (34 if t == Q8_0 else 18)
    pitch = rb + 6                               # a padded row pitch (even)
    dst = torch.full((dst_rows, pitch), 0xAB, dtype=torch.uint8, device=dev)
    idx = torch.tensor([5, 0, 19, 7, 3, 11, 2], dtype=torch.int64, device=dev)
    ops.set_rows_q(dst, torch.from_numpy(x).to(dev), t, idx, rule)
    got = dst.cpu().numpy()
    want = quant(orc, t, x, rule)
    for r, d in enumerate(idx.tolist()):
        assert np.array_equal(got[d, :rb], want[r]), (r, d)
    untouched = [i for i in range(dst_rows) if i not in idx.tolist()]
    assert np.all(got[untouched] == 0xAB) and np.all(got[:, rb:] == 0xAB)
    # i32 indices, no index (CPY), and the fail-fast path for an index out of range
    dst2 = torch.zeros((rows, rb), dtype=torch.uint8, device=dev)
    ops.set_rows_q(dst2, torch.from_numpy(x).to(dev), t, None, rule)
    assert np.array_equal(dst2.cpu().numpy(), want)
    with pytest.raises(IndexError):
        ops.set_rows_q(dst, torch.from_numpy(x[:2]).to(dev), t, torch.tensor([3, 20], dtype=torch.int32, device=dev),
                       rule)


def make_cache(orc, rng, t, n_head_kv, n_kv, D, token_major):
    """f32 values, their ggml blocks, and a cache view [n_head_kv, n_kv, row bytes] in llama.cpp's token-major layout
    (row j holds all KV heads) or head-major."""
    xf = rng.standard_normal((n_head_kv, n_kv, D)).astype(np.float32)
    blocks = quant(orc, t, xf.reshape(-1, D)).reshape(n_head_kv, n_kv, -1)
    if token_major:
        store = np.ascontiguousarray(blocks.transpose(1, 0, 2))      # [n_kv, n_head_kv, rb]
        return blocks, store, lambda d: d.permute(1, 0, 2)
    return blocks, np.ascontiguousarray(blocks), lambda d: d


@pytest.mark.parametrize("t", [Q8_0, Q4_0])
@pytest.mark.parametrize("G,n_kv,token_major,masked", [(4, 4096, True, False), (1, 17, False, True),
                                                      (2, 300, True, True), (8, 1, False, False),
                                                      (4, 1000, False, True)])
def test_flash_attn_decode_quantized(dev, ops, orc, t, G, n_kv, token_major, masked):
    rng = np.random.default_rng(n_kv + G + t)
    n_head_kv, D = 8 if G < 8 else 4, 128
    n_head = n_head_kv * G
    scale = 1.0 / np.sqrt(D)
    q = rng.standard_normal((n_head, D)).astype(np.float32)
    kb, ks, kview = make_cache(orc, rng, t, n_head_kv, n_kv, D, token_major)
    vb, vs, vview = make_cache(orc, rng, t, n_head_kv, n_kv, D, token_major)
    mask = None
    if masked:
        mask = np.zeros(n_kv, np.float16)
        mask[n_kv * 2 // 3:] = -np.inf
        mask[::5] = -1.5
    want = orc.flash_attn_decode_q(t, q, kb, vb, scale, None if mask is None else mask.view(np.uint16))
    qd = torch.from_numpy(q).to(dev)
    kd, vd = kview(torch.from_numpy(ks).to(dev)), vview(torch.from_numpy(vs).to(dev))
    md = None if mask is None else torch.from_numpy(mask.view(np.uint16)).to(dev)
    out = ops.flash_attn_decode_kv(qd, kd, vd, t, scale, mask=md)
    got = out.cpu().numpy()
    assert rel_l2(got, want) < 1e-4
    assert rel_l2(got, want) < 2e-3  # the BASELINE attention bar
    # key count from device memory, one-launch merge: identical to the plain call
    nkv = torch.tensor([n_kv], dtype=torch.int32, device=dev)
    a = ops.flash_attn_decode_kv(qd, kd, vd, t, scale, n_kv_max=n_kv, n_kv_dev=nkv, mask=md)
    b = ops.flash_attn_decode_kv(qd, kd, vd, t, scale, n_kv_max=n_kv, n_kv_dev=nkv, mask=md, one_launch=True)
    assert torch.equal(a, out) and torch.equal(b, out)


@pytest.mark.parametrize("t", [Q8_0, Q4_0])
def test_quantized_cache_exact_regime_matches_f16_path(dev, ops, orc, t):
    """Cache values exact in f16 and q whose Q8_0 is exact: the quantized-cache kernel and the f16-cache kernel see the
    same numbers, and their outputs agree to f32 rounding."""
    from test_oracle import exact_cache
    rng = np.random.default_rng(60 + t)
    n_head, n_head_kv, n_kv, D = 32, 8, 700, 128
    n = rng.integers(-127, 128, (n_head, D))
    n[:, ::32] = 127
    q = (n * 2.0 ** -6).astype(np.float32)
    kx = exact_cache(rng, t, n_head_kv * n_kv, D)
    vx = exact_cache(rng, t, n_head_kv * n_kv, D)
    k16 = orc.dequantize(t, kx, D).reshape(n_head_kv, n_kv, D).astype(np.float16)
    v16 = orc.dequantize(t, vx, D).reshape(n_head_kv, n_kv, D).astype(np.float16)
    qd = torch.from_numpy(q).to(dev)
    a = ops.flash_attn_decode_kv(qd, torch.from_numpy(kx.reshape(n_head_kv, n_kv, -1)).to(dev),
                                 torch.from_numpy(vx.reshape(n_head_kv, n_kv, -1)).to(dev), t, 0.0884)
    b = ops.flash_attn_decode_kv(qd, torch.from_numpy(k16).to(dev), torch.from_numpy(v16).to(dev), F16, 0.0884)
    assert rel_l2(a.cpu().numpy(), b.cpu().numpy()) < 1e-6


def test_quantized_cache_rejects_bad_layouts(dev, ops):
    q = torch.zeros((8, 128), dtype=torch.float32, device=dev)
    k = torch.zeros((2, 16, 136), dtype=torch.uint8, device=dev)
    short = torch.zeros((2, 16, 100), dtype=torch.uint8, device=dev)
    with pytest.raises(RuntimeError):  # a Q8_0 row of 128 elements is 136 bytes: a 100-byte pitch is too short
        ops.flash_attn_decode_kv(q, short, short, Q8_0, 0.1)
    ops.flash_attn_decode_kv(q, short, short, Q4_0, 0.1)  # 72-byte Q4_0 rows fit
    with pytest.raises(RuntimeError):
        ops.flash_attn_decode_kv(q, k, k, 3, 0.1)  # not a cache type
