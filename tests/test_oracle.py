"""Pins the CPU oracle (oracle/ameva_oracle.c) before anything is compared with it.

Each check comes from outside the oracle's own formula: a library routine (numpy's IEEE float16), the reference's own
golden fixtures (tests/golden/, from /root/reference/tests/fixtures), the reference's own compiled I2_S kernel
(oracle/_ref), hand-computed known answers, closed forms evaluated in float64 from dequantized values, and
invariants a plausible mistake (swapped nibble, wrong index, dropped term, wrong sign) would break.
"""
import hashlib
import json
import os

import numpy as np
import pytest

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def rel_l2(a, b):
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


# ---------------------------------------------------------------------------------------------------------- fp16
def test_fp16_to_fp32_all_65536(orc):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = orc.fp16_to_fp32(h)
    want = h.view(np.float16).astype(np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_fp32_to_fp16_matches_ieee_rne(orc):
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 2**32, size=2_000_000, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    special = np.array([0.0, -0.0, 65504.0, 65519.99, 65520.0, 65536.0, 2.0**-24, 2.0**-25, 2.0**-25 * 1.0000001,
                        2.0**-14, 2.0**-14 * (1 - 2**-11), 3 * 2.0**-26, np.inf, -np.inf, 1.0 + 2**-11,
                        1.0 + 3 * 2**-11, 0.1, -7.3e-6], dtype=np.float32)
    # also every f32 that lies exactly halfway between two adjacent halves, and its neighbours
    h = np.arange(0, 0x7BFF, 7, dtype=np.uint16)
    lo = h.view(np.float16).astype(np.float64)
    hi = (h + 1).view(np.float16).astype(np.float64)
    mid = ((lo + hi) / 2).astype(np.float32)
    x = np.concatenate([x, special, mid, np.nextafter(mid, np.float32(np.inf)), np.nextafter(mid, np.float32(0))])
    x = x[~np.isnan(x)]
    got = orc.fp32_to_fp16(x)
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    assert orc.fp32_to_fp16(np.array([np.nan], np.float32))[0] & 0x7FFF == 0x7E00


# ---------------------------------------------------------------------------------------------------------- Q4_0
def test_q4_0_known_answer(orc):
    # block: max magnitude element -8 at index 3 -> d = 1, id = 1, nibble = min(15, trunc(x + 8.5))
    x = np.zeros(32, np.float32)
    x[3] = -8.0
    x[0] = 1.0       # 9.5 -> 9
    x[1] = 0.5       # 9.0 -> 9
    x[2] = -0.5      # 8.0 -> 8
    x[16] = 7.9      # 16.4 -> 16 -> clamp 15
    x[17] = -7.6     # 0.9 -> 0
    x[31] = 2.49     # 10.99 -> 10
    y = orc.quantize_q4_0(x)[0]
    assert y.size == 18
    assert (int(y[0]) | (int(y[1]) << 8)) == 0x3C00  # fp16(1.0)
    qs = y[2:]
    lo = qs & 0xF
    hi = qs >> 4
    assert lo[0] == 9 and lo[1] == 9 and lo[2] == 8 and lo[3] == 0 and lo[4] == 8
    assert hi[0] == 15 and hi[1] == 0 and hi[15] == 10 and hi[2] == 8
    deq = orc.dequantize(orc.Q4_0, y, 32)[0]
    assert deq[0] == 1.0 and deq[3] == -8.0 and deq[16] == 7.0 and deq[17] == -8.0 and deq[31] == 2.0


def test_q4_0_invariants_and_idempotence(orc):
    rng = np.random.default_rng(2)
    x = (rng.standard_normal((64, 256)) * 0.02).astype(np.float32)
    x[5, 33] = -0.1  # tie in magnitude: the first one (index 33, -0.1) is the max
    x[5, 40] = 0.1
    y = orc.quantize_q4_0(x)
    deq = orc.dequantize(orc.Q4_0, y, 256)
    blocks = y.reshape(-1, 18)
    d16 = orc.fp16_to_fp32(blocks[:, 0].astype(np.uint16) | (blocks[:, 1].astype(np.uint16) << 8))
    xb = x.reshape(-1, 32)
    err = np.abs(deq.reshape(-1, 32) - xb)
    assert np.all(err <= np.abs(d16)[:, None] * 1.01 + 1e-12)
    # the element of largest magnitude maps to nibble 0 (x * id = -8)
    amax_idx = np.argmax(np.abs(xb), axis=1)
    nib = np.concatenate([blocks[:, 2:] & 0xF, blocks[:, 2:] >> 4], axis=1)
    assert np.all(nib[np.arange(len(nib)), amax_idx] == 0)
    # tie: block 5*8+1 holds indices 32..63 of row 5; element 33 (first) is the max -> d > 0 (max negative)
    assert d16[5 * 8 + 1] > 0
    # quantize(dequantize(q)) == q
    assert np.array_equal(orc.quantize_q4_0(deq), y)


# ---------------------------------------------------------------------------------------------------------- Q8_0
def test_q8_0_rules_known_answers(orc):
    # amax = 127 -> d = 1, id = 1 under all rules; 2.5 and -3.5 are ties
    x = np.zeros(32, np.float32)
    x[0] = 127.0
    x[1] = 2.5
    x[2] = -3.5
    x[3] = 2.4999
    x[4] = -127.0
    for rule, want in ((orc.Q8_X86, (2, -4)), (orc.Q8_ARM, (2, -4)), (orc.Q8_REF, (3, -4))):
        y = orc.quantize_q8_0(x, rule)[0]
        q = y[2:].view(np.int8)
        assert (int(y[0]) | (int(y[1]) << 8)) == 0x3C00
        assert q[0] == 127 and q[4] == -127 and q[3] == 2
        assert (q[1], q[2]) == want, rule


def test_q8_0_x86_and_arm_rules_differ(orc):
    """Blocks where 127/amax and 1/(amax/127) are different f32 values and one element lands on opposite sides of
    a rounding boundary: rule 0 must give the x86 result (x * (127/amax)), rule 1 the ARM one (x * (1/d)). The
    expected integers are fixed constants, and numpy's IEEE single-precision arithmetic recomputes both rules."""
    f = np.float32
    cases = [  # (amax bits, x bits, q under x86, q under ARM)
        (1081376603, 1064977893, 32, 33),
        (1073587831, 1058916430, 40, 39),
        (1074107746, 1073866479, 123, 124),
        (1072994361, 1049022689, 18, 17),
        (1067132384, 1058743776, 63, 64),  # x = amax / 2 exactly: a real tie at 63.5
    ]
    x = np.zeros((len(cases), 32), np.float32)
    for i, (ab, xb, _, _) in enumerate(cases):
        x[i, 0] = np.array(ab, np.uint32).view(np.float32)
        x[i, 7] = np.array(xb, np.uint32).view(np.float32)
    y86 = orc.quantize_q8_0(x, orc.Q8_X86).reshape(len(cases), 34)
    yarm = orc.quantize_q8_0(x, orc.Q8_ARM).reshape(len(cases), 34)
    for i, (_, _, q86, qarm) in enumerate(cases):
        amax, xv = x[i, 0], x[i, 7]
        id86, idarm = f(127) / amax, f(1) / (amax / f(127))
        assert id86 != idarm
        assert np.rint(xv * id86) == q86 and np.rint(xv * idarm) == qarm
        assert int(y86[i, 2 + 7].view(np.int8)) == q86, i
        assert int(yarm[i, 2 + 7].view(np.int8)) == qarm, i
        assert int(y86[i, 2].view(np.int8)) == 127 and int(yarm[i, 2].view(np.int8)) == 127


def test_q8_0_invariants(orc):
    rng = np.random.default_rng(3)
    x = rng.standard_normal((16, 4096)).astype(np.float32)
    for rule in (orc.Q8_X86, orc.Q8_ARM, orc.Q8_REF):
        y = orc.quantize_q8_0(x, rule).reshape(-1, 34)
        q = y[:, 2:].view(np.int8).astype(np.int32)
        xb = x.reshape(-1, 32)
        amax = np.abs(xb).max(axis=1)
        # d is amax/127 rounded to fp16
        d16 = orc.fp16_to_fp32(y[:, 0].astype(np.uint16) | (y[:, 1].astype(np.uint16) << 8))
        assert np.array_equal(d16.view(np.uint32),
                              (amax / np.float32(127)).astype(np.float16).astype(np.float32).view(np.uint32))
        assert np.all(np.abs(q) <= 127)
        i = np.argmax(np.abs(xb), axis=1)
        assert np.all(np.abs(q[np.arange(len(q)), i]) == 127)
        # |x * 127/amax - q| <= 0.5 (+ tiny f32 slack)
        t = xb.astype(np.float64) * 127.0 / amax[:, None]
        assert np.all(np.abs(t - q) <= 0.5 + 1e-4)
    a = orc.quantize_q8_0(x, orc.Q8_X86)
    b = orc.quantize_q8_0(x, orc.Q8_ARM)
    c = orc.quantize_q8_0(x, orc.Q8_REF)
    # the rules differ only on (near) ties: agreement is high but the x86 rule is the chosen one
    assert (a == b).mean() > 0.999 and (a == c).mean() > 0.999


# ---------------------------------------------------------------------------------------------------------- Q8_K
def test_q8_K_invariants(orc):
    rng = np.random.default_rng(4)
    x = rng.standard_normal((4, 1024)).astype(np.float32)
    y = orc.quantize_q8_K(x).reshape(-1, 292)
    d = y[:, :4].copy().view(np.float32)[:, 0]
    q = y[:, 4:260].view(np.int8).astype(np.int32)
    bs = y[:, 260:].copy().view(np.int16).astype(np.int32)
    assert np.array_equal(bs, q.reshape(-1, 16, 16).sum(axis=2))
    xb = x.reshape(-1, 256)
    i = np.argmax(np.abs(xb), axis=1)
    assert np.all(q[np.arange(len(q)), i] == -127)  # iscale = -127/max maps max to -127
    assert np.all(np.abs(d[:, None] * q - xb) <= np.abs(d)[:, None] * 0.5001)
    z = orc.quantize_q8_K(np.zeros((1, 256), np.float32))
    assert not z.any()


def test_q8_K_ties_round_half_even(orc):
    """Known answers at exact ties: a block whose largest element is -127 (or +127) has iscale = -127/max = +1 (-1)
    exactly, so half-integer inputs land on ties, which ggml's nearest_int (the 1.5 * 2^23 addition in the default
    rounding mode) resolves to the even neighbour, as numpy's rint does; d = 1 / iscale."""
    ties = np.array([2.5, 3.5, -2.5, -3.5, 0.5, 1.5, -0.5, 126.5, -126.5, 64.5], np.float32)
    for lead, sign in ((-127.0, 1.0), (127.0, -1.0)):
        x = np.zeros((1, 256), np.float32)
        x[0, 0] = lead
        x[0, 1:1 + ties.size] = ties
        x[0, 100] = 3.25  # not a tie: nearest
        y = orc.quantize_q8_K(x).reshape(292)
        assert y[:4].copy().view(np.float32)[0] == sign
        q = y[4:260].view(np.int8).astype(np.int32)
        want = np.zeros(256, np.int32)
        want[0] = -127
        want[1:1 + ties.size] = (sign * np.array([2, 4, -2, -4, 0, 2, 0, 126, -126, 64])).astype(np.int32)
        want[100] = int(sign * 3)
        assert np.array_equal(q, want)
        assert np.array_equal(np.rint(sign * x[0]).astype(np.int32), want)


# ------------------------------------------------------------------------------------------- K-quant layouts
def _pack_k4_scales(sc, mn):
    """ggml's documented 12-byte packing of 8 six-bit scales and mins (the inverse of get_scale_min_k4)."""
    out = np.zeros(12, np.uint8)
    for j in range(4):
        out[j] = (sc[j] & 63) | ((sc[j + 4] >> 4) << 6)
        out[j + 4] = (mn[j] & 63) | ((mn[j + 4] >> 4) << 6)
        out[j + 8] = (sc[j + 4] & 0xF) | ((mn[j + 4] & 0xF) << 4)
    return out


def test_q4_K_dequant_known_answer(orc):
    sc = np.array([1, 2, 3, 63, 17, 33, 48, 62], np.int64)
    mn = np.array([0, 5, 9, 40, 16, 31, 63, 1], np.int64)
    blk = np.zeros(144, np.uint8)
    blk[0:2] = np.frombuffer(np.float16(0.5).tobytes(), np.uint8)
    blk[2:4] = np.frombuffer(np.float16(0.25).tobytes(), np.uint8)
    blk[4:16] = _pack_k4_scales(sc, mn)
    vals = np.arange(256) % 16  # 4-bit value of weight i
    qs = np.zeros(128, np.uint8)
    for c in range(4):
        for l in range(32):
            qs[32 * c + l] = vals[64 * c + l] | (vals[64 * c + 32 + l] << 4)
    blk[16:] = qs
    got = orc.dequantize(orc.Q4_K, blk, 256)[0]
    unit = np.arange(256) // 32
    want = 0.5 * sc[unit] * vals - 0.25 * mn[unit]
    assert np.array_equal(got, want.astype(np.float32))


def test_q6_K_dequant_known_answer(orc):
    rng = np.random.default_rng(5)
    v = rng.integers(0, 64, 256)  # 6-bit value of weight i
    sc = rng.integers(-128, 128, 16).astype(np.int8)
    blk = np.zeros(210, np.uint8)
    # ggml's layout: per half of 128 weights, ql[64] and qh[32]; weight l+32s of the half (s = 0..3) has its low
    # nibble in ql[l + 32*(s&1)] (low nibble for s < 2, high for s >= 2) and its top bits at qh[l] bits 2s..2s+1
    for h in range(2):
        for s in range(4):
            for l in range(32):
                val = int(v[128 * h + 32 * s + l])
                qi = 64 * h + l + 32 * (s & 1)
                blk[qi] |= (val & 0xF) << (4 * (s >> 1))
                blk[128 + 32 * h + l] |= (val >> 4) << (2 * s)
    blk[192:208] = sc.view(np.uint8)
    blk[208:210] = np.frombuffer(np.float16(0.125).tobytes(), np.uint8)
    got = orc.dequantize(orc.Q6_K, blk, 256)[0]
    want = 0.125 * sc[np.arange(256) // 16].astype(np.float64) * (v - 32)
    assert np.array_equal(got, want.astype(np.float32))


# ------------------------------------------------------------------------------------------------ dot products
def _random_blocks(rng, t, rows, k):
    """Random bytes are valid ggml blocks once the fp16 scale fields hold small finite values."""
    be, bb = {2: (32, 18), 8: (32, 34), 12: (256, 144), 14: (256, 210)}[t]
    y = rng.integers(0, 256, (rows, k // be, bb), dtype=np.uint8)
    def put(off, lo, hi):
        v = rng.uniform(lo, hi, (rows, k // be)).astype(np.float16)
        y[:, :, off:off + 2] = v.view(np.uint8).reshape(rows, k // be, 2)
    if t in (2, 8):
        put(0, -0.01, 0.01)
    elif t == 12:
        put(0, 0.0, 0.002)
        put(2, 0.0, 0.002)
    else:
        put(208, 0.0, 0.002)
    return y.reshape(rows, -1)


@pytest.mark.parametrize("wtype", [2, 8, 12, 14])
def test_mul_mat_vs_dequantized_float64(orc, wtype):
    rng = np.random.default_rng(10 + wtype)
    n, k, m = 48, 1024, 3
    w = _random_blocks(rng, wtype, n, k)
    x = rng.standard_normal((m, k)).astype(np.float32)
    aq = orc.quantize_q8_K(x) if wtype in (12, 14) else orc.quantize_q8_0(x, orc.Q8_X86)
    dst, blk = orc.mul_mat(wtype, w, n, k, aq, m, with_blocks=True)
    wd = orc.dequantize(wtype, w, k).astype(np.float64)
    ad = orc.dequantize(8, aq, k) if wtype in (2, 8) else None
    if ad is None:  # Q8_K: d f32 at 0, int8 qs at 4
        ab = aq.reshape(m, -1, 292)
        d = ab[:, :, :4].copy().view(np.float32)
        ad = (ab[:, :, 4:260].view(np.int8).astype(np.float64) * d).reshape(m, k)
    want = ad.astype(np.float64) @ wd.T
    assert rel_l2(dst, want) < 1e-5
    # the exact integer block sums, by brute force from unpacked integer values
    if wtype in (2, 8):
        bb = 18 if wtype == 2 else 34
        wb = w.reshape(n, -1, bb)
        if wtype == 2:
            nib = np.concatenate([wb[:, :, 2:] & 0xF, wb[:, :, 2:] >> 4], axis=2).astype(np.int64) - 8
        else:
            nib = wb[:, :, 2:].view(np.int8).astype(np.int64)
        qa = aq.reshape(m, -1, 34)[:, :, 2:].view(np.int8).astype(np.int64)
        sums = np.einsum("nbj,mbj->mnb", nib, qa)
        assert np.array_equal(blk, sums)


# ---------------------------------------------------------------------------------------------------- RMSNorm
def test_rms_norm_closed_form(orc):
    rng = np.random.default_rng(20)
    x = rng.standard_normal((5, 4096)).astype(np.float32) * 3
    w = rng.standard_normal(4096).astype(np.float32)
    y, o = orc.rms_norm(x, 1e-5, w)
    x64 = x.astype(np.float64)
    want = x64 / np.sqrt((x64 ** 2).mean(axis=1, keepdims=True) + 1e-5)
    assert rel_l2(y, want) < 1e-6
    assert rel_l2(o, want * w) < 1e-6
    assert np.allclose((y.astype(np.float64) ** 2).mean(axis=1), 1.0, rtol=1e-5)


# ------------------------------------------------------------------------------------------------------- RoPE
@pytest.mark.parametrize("mode", [0, 2])
def test_rope_closed_form(orc, mode):
    rng = np.random.default_rng(21)
    n_tok, n_head, D = 6, 4, 128
    x = rng.standard_normal((n_tok, n_head, D)).astype(np.float32)
    pos = np.array([0, 1, 7, 100, 4095, 4096], np.int32)
    y = orc.rope(x, pos, D, mode, 500000.0)
    assert np.array_equal(y[0], x[0])  # position 0 is the identity
    j = np.arange(D // 2)
    theta = pos[:, None].astype(np.float64) * 500000.0 ** (-2.0 * j / D)
    c, s = np.cos(theta)[:, None, :], np.sin(theta)[:, None, :]
    x64 = x.astype(np.float64)
    if mode == 0:
        x0, x1 = x64[..., 0::2], x64[..., 1::2]
        want = np.empty_like(x64)
        want[..., 0::2] = x0 * c - x1 * s
        want[..., 1::2] = x0 * s + x1 * c
    else:
        x0, x1 = x64[..., :D // 2], x64[..., D // 2:]
        want = np.concatenate([x0 * c - x1 * s, x0 * s + x1 * c], axis=-1)
    # the f32 angle built by repeated multiplication drifts by a few ulp of p: 1e-4 relative at p = 4096
    assert rel_l2(y, want) < 1e-4
    assert np.allclose(np.linalg.norm(y, axis=-1), np.linalg.norm(x, axis=-1), rtol=1e-5)


# ------------------------------------------------------------------------------------------------ FA decode
def test_flash_attn_decode_closed_form(orc):
    rng = np.random.default_rng(22)
    n_head, n_head_kv, n_kv, D = 8, 2, 300, 64
    q = rng.standard_normal((n_head, D)).astype(np.float32)
    k = rng.standard_normal((n_head_kv, n_kv, D)).astype(np.float16)
    v = rng.standard_normal((n_head_kv, n_kv, D)).astype(np.float16)
    mask = np.zeros(n_kv, np.float16)
    mask[250:] = -np.inf
    scale = 1.0 / np.sqrt(D)
    out = orc.flash_attn_decode(q, k.view(np.uint16), v.view(np.uint16), scale, mask.view(np.uint16))
    qh = q.astype(np.float16).astype(np.float64)
    want = np.empty((n_head, D))
    for h in range(n_head):
        kk = k[h // (n_head // n_head_kv), :250].astype(np.float64)
        vv = v[h // (n_head // n_head_kv), :250].astype(np.float64)
        s = kk @ qh[h] * scale
        p = np.exp(s - s.max())
        want[h] = p @ vv / p.sum()
    assert rel_l2(out, want) < 1e-6


def exact_cache(rng, kv, n_rows, D):
    """Q8_0 / Q4_0 rows of D with d a power of two (2^-7, 2^-4): every dequantized value is exact in f16."""
    nb = D // 32
    if kv == 8:
        blk = np.zeros((n_rows, nb, 34), np.uint8)
        blk[:, :, 0:2] = np.array([2.0 ** -7], np.float16).view(np.uint8)
        blk[:, :, 2:] = rng.integers(-127, 128, (n_rows, nb, 32)).astype(np.int8).view(np.uint8)
    else:
        blk = np.zeros((n_rows, nb, 18), np.uint8)
        blk[:, :, 0:2] = np.array([2.0 ** -4], np.float16).view(np.uint8)
        blk[:, :, 2:] = rng.integers(0, 256, (n_rows, nb, 16)).astype(np.uint8)
    return blk.reshape(n_rows, -1)


@pytest.mark.parametrize("kv", [8, 2])
def test_flash_attn_decode_quantized_cache(orc, kv):
    """The quantized-cache oracle against (a) float64 from the pinned dequantizer and the pinned Q8_0 of q (the scores
    are exact integers times d_k d_q) and (b) the f16-cache oracle where Q8_0 of q is exact and the cache values are
    exact in f16: a swapped nibble, a wrong block or head index or a dropped d breaks one of them."""
    rng = np.random.default_rng(40 + kv)
    n_head, n_head_kv, n_kv, D = 8, 2, 300, 128
    scale = 1.0 / np.sqrt(D)
    mask = np.zeros(n_kv, np.float16)
    mask[250:] = -np.inf
    quant = (lambda x: orc.quantize_q8_0(x, orc.Q8_X86)) if kv == 8 else orc.quantize_q4_0
    q = rng.standard_normal((n_head, D)).astype(np.float32)
    kq = quant(rng.standard_normal((n_head_kv * n_kv, D)).astype(np.float32)).reshape(n_head_kv, n_kv, -1)
    vq = quant(rng.standard_normal((n_head_kv * n_kv, D)).astype(np.float32)).reshape(n_head_kv, n_kv, -1)
    out = orc.flash_attn_decode_q(kv, q, kq, vq, scale, mask.view(np.uint16))
    kd = orc.dequantize(kv, kq, D).reshape(n_head_kv, n_kv, D).astype(np.float64)
    vd = orc.dequantize(kv, vq, D).reshape(n_head_kv, n_kv, D).astype(np.float64)
    qd = orc.dequantize(8, orc.quantize_q8_0(q, orc.Q8_X86), D).astype(np.float64)
    want = np.empty((n_head, D))
    G = n_head // n_head_kv
    for h in range(n_head):
        sc = kd[h // G, :250] @ qd[h] * scale
        p = np.exp(sc - sc.max())
        want[h] = p @ vd[h // G, :250] / p.sum()
    assert rel_l2(out, want) < 1e-5
    # exact regime: q = n 2^-6 with a +-127 in every block (Q8_0 of q is exact), cache values exact in f16
    n = rng.integers(-127, 128, (n_head, D))
    n[:, ::32] = 127 * rng.choice([-1, 1], (n_head, D // 32))
    qx = (n * 2.0 ** -6).astype(np.float32)
    kx = exact_cache(rng, kv, n_head_kv * n_kv, D).reshape(n_head_kv, n_kv, -1)
    vx = exact_cache(rng, kv, n_head_kv * n_kv, D).reshape(n_head_kv, n_kv, -1)
    k16 = orc.dequantize(kv, kx, D).reshape(n_head_kv, n_kv, D).astype(np.float16)
    v16 = orc.dequantize(kv, vx, D).reshape(n_head_kv, n_kv, D).astype(np.float16)
    a = orc.flash_attn_decode_q(kv, qx, kx, vx, scale, mask.view(np.uint16))
    b = orc.flash_attn_decode(qx, k16.view(np.uint16), v16.view(np.uint16), scale, mask.view(np.uint16))
    assert rel_l2(a, b) < 1e-6


# ------------------------------------------------------------------------------------------------------ SwiGLU
def test_swiglu_closed_form(orc):
    rng = np.random.default_rng(23)
    g = rng.standard_normal(14336).astype(np.float32) * 4
    u = rng.standard_normal(14336).astype(np.float32)
    y = orc.swiglu(g, u)
    g64 = g.astype(np.float64)
    assert rel_l2(y, g64 / (1 + np.exp(-g64)) * u) < 1e-6


# -------------------------------------------------------------------------------------------------------- I2_S
def _sha(path):
    with open(path, "rb") as f:
        return hashlib.sha256(f.read()).hexdigest()


def test_i2s_golden_fixtures(orc):
    man = json.load(open(os.path.join(GOLD, "fixture_manifest.json")))["fixtures"]
    fx = os.path.join(GOLD, "fixture_i2s_upstream.bin")
    ex = os.path.join(GOLD, "expected_i2s_upstream_f32.bin")
    sl = os.path.join(GOLD, "gguf_slice_blk0_v.bin")
    assert _sha(fx) == man["fixture_i2s_upstream.bin"]["packed_fixture_sha256"]
    assert _sha(ex) == man["expected_i2s_upstream_f32.bin"]["expected_f32_sha256"]
    assert _sha(sl) == man["gguf_slice_blk0_v.bin"]["packed_fixture_sha256"]
    data = np.fromfile(fx, np.uint8)
    # 256 weights = 2 rows x 128; the trailer scale sits right after the 64-byte payload
    scale = orc.i2s_trailer_scale(data, 2, 128)
    assert scale == 1.625
    got = orc.i2s_dequantize(data[:64], scale, 256)
    want = np.fromfile(ex, np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert ((got < 0).sum(), (got == 0).sum(), (got > 0).sum()) == (86, 85, 85)
    s2 = np.fromfile(sl, np.uint8)
    sc2 = orc.i2s_trailer_scale(s2, 1, 128)
    assert abs(sc2 - 2.2931101322) < 1e-6
    w2 = orc.i2s_dequantize(s2[:32], sc2, 128)
    assert ((w2 < 0).sum(), (w2 == 0).sum(), (w2 > 0).sum()) == (48, 38, 42)


def test_i2s_quantize_act_rule(orc):
    x = np.zeros(8, np.float32)
    x[0] = 127.0        # scale = 1
    x[1] = 2.5          # half away from zero: 3
    x[2] = -2.5         # -3
    x[3] = 0.49
    q, deq = orc.i2s_quantize_act(x)
    assert deq[0] == 1.0
    assert list(q[0, :4]) == [127, 3, -3, 0]
    q0, d0 = orc.i2s_quantize_act(np.zeros((1, 16), np.float32))
    assert not q0.any() and d0[0] == np.float32(1e-7) / np.float32(127.0) or abs(d0[0] - 1e-7 / 127) < 1e-12


def test_i2s_gemv_vs_reference_kernel_and_brute_force(orc):
    rng = np.random.default_rng(30)
    n, k = 37, 2560
    codes = rng.integers(0, 3, (n, k))  # ternary codes 0,1,2 -> -1,0,+1
    w = np.zeros((n, k // 4), np.uint8)
    for b in range(k // 128):
        for g in range(4):
            w[:, 32 * b: 32 * b + 32] |= (codes[:, 128 * b + 32 * g: 128 * b + 32 * g + 32] << (6 - 2 * g)).astype(np.uint8)
    x = rng.standard_normal((2, k)).astype(np.float32)
    q, deq = orc.i2s_quantize_act(x)
    out, sums = orc.i2s_gemv(w, n, k, q, deq, 1.7)
    brute = q.astype(np.int64) @ (codes - 1).T.astype(np.int64)
    assert np.array_equal(sums, brute)
    assert np.array_equal(out, (brute.astype(np.float32) * (deq[:, None] * np.float32(1.7))).astype(np.float32))
    if orc.RefI2S.available():
        ref = orc.RefI2S()
        for c in range(2):
            s = ref.gemv_sums(w, n, k, q[c])
            assert np.array_equal(s, sums[c].astype(np.float32))
    else:
        pytest.skip("oracle/_ref not built (reference source absent)")


def test_flash_attn_prefill_oracle_is_masked_decode(orc):
    """The prefill restatement: query t equals the decode over the keys it sees; the built-in causal limit and an
    explicit ggml KQ mask (-inf above the diagonal, f16) give the same rows; the first query sees key 0 only, so its
    output is V row 0 of its KV head (softmax of one score)."""
    rng = np.random.default_rng(21)
    n_tok, n_head, n_head_kv, D, pos0 = 9, 4, 2, 128, 3
    n_kv = pos0 + n_tok
    q = rng.standard_normal((n_tok, n_head, D)).astype(np.float32)
    k = orc.fp32_to_fp16(rng.standard_normal((n_head_kv, n_kv, D)))
    v = orc.fp32_to_fp16(rng.standard_normal((n_head_kv, n_kv, D)))
    a = orc.flash_attn_prefill(q, k, v, 0.0884, causal_pos0=pos0)
    neg = np.uint16(0xFC00)  # f16 -inf
    mask = np.zeros((n_tok, n_kv), np.uint16)
    for t in range(n_tok):
        mask[t, pos0 + t + 1:] = neg
    b = orc.flash_attn_prefill(q, k, v, 0.0884, mask=mask)
    np.testing.assert_allclose(a, b, rtol=0, atol=0)
    for t in (0, 5):
        d = orc.flash_attn_decode(q[t], np.ascontiguousarray(k[:, :pos0 + t + 1]), np.ascontiguousarray(v[:, :pos0 + t + 1]),
                                  0.0884)
        np.testing.assert_array_equal(a[t], d)
    one = orc.flash_attn_prefill(q[:1], k[:, :1], v[:, :1], 0.0884, causal_pos0=0)
    vf = orc.fp16_to_fp32(v[:, 0])
    np.testing.assert_allclose(one[0], vf[np.arange(n_head) // (n_head // n_head_kv)], rtol=1e-6)
