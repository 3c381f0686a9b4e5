"""The CPU baseline kernels bench.py times (oracle/cpu_simd.c: ggml's AVX2 vec_dot_q4_0_q8_0 algorithm and an f16-KV
decode attention) compute what the oracle computes: the same per-block integers, so MUL_MAT agrees to float
accumulation order; the attention to the oracle's f16 V accumulation."""
import numpy as np
import pytest

import oracle

pytestmark = pytest.mark.skipif(oracle.cpu_simd() is None, reason="host CPU lacks AVX2 / FMA / F16C")


@pytest.mark.parametrize("n,k,m", [(1, 32, 1), (64, 256, 3), (130, 4096, 2), (33, 14336, 40)])
def test_simd_mul_mat_q4_0(n, k, m):
    rng = np.random.default_rng(n * 7 + m)
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float32)
    wq = oracle.quantize_q4_0(w)
    aq = oracle.quantize_q8_0(x, oracle.Q8_X86)
    ref = oracle.mul_mat(oracle.Q4_0, wq, n, k, aq, m)
    ref = ref[0] if isinstance(ref, tuple) else ref
    got = oracle.simd_mul_mat_q4_0(wq, n, k, aq, m)
    assert got.shape == (m, n)
    np.testing.assert_allclose(got, ref, rtol=2e-5, atol=2e-5 * np.abs(ref).max())


@pytest.mark.parametrize("n_kv,n_head,n_head_kv", [(1, 4, 4), (300, 32, 8), (1025, 8, 1)])
def test_simd_flash_attn_decode(n_kv, n_head, n_head_kv):
    rng = np.random.default_rng(n_kv)
    D = 128
    q = rng.standard_normal((n_head, D)).astype(np.float32)
    k = rng.standard_normal((n_kv, n_head_kv, D)).astype(np.float16)
    v = rng.standard_normal((n_kv, n_head_kv, D)).astype(np.float16)
    ref = oracle.flash_attn_decode(q, np.ascontiguousarray(k.transpose(1, 0, 2)).view(np.uint16),
                                   np.ascontiguousarray(v.transpose(1, 0, 2)).view(np.uint16), 0.0884)
    got = oracle.simd_flash_attn_decode(q, k, v, 0.0884)
    rel = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    assert rel < 2e-3, rel
