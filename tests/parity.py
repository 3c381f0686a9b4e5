"""The reference's per-output parity gate for MUL_MAT results (tests/ameva_qmm_check.cpp:201-216): every output must
satisfy |got - ref| <= tol * sum_k |w_k a_k|, where ref = sum_k w_k a_k is the float64 dot product of the dequantized
weight row and the dequantized (quantized) activation row, and tol is 1e-5. A single wrong block in one row of
14336 moves a global relative L2 by ~1e-4 and passes a 1e-3 global bar; it fails this gate by orders of magnitude.

The reference subtracts an allowance for its activation quantization because it compares against f32 activations;
here got and ref read the same quantized activation bytes, so the allowance is zero. Forms whose operands are rounded
to f16 on purpose (the scaled batched form) are held to the rounding bound of that: 2^-10 (each operand rounded once
to f16, 2^-11 relative each) with 10 % headroom.
"""
from __future__ import annotations

import numpy as np

TOL_EXACT = 1e-5
TOL_F16_OPERANDS = 1.1 * 2.0 ** -10

Q4_0, Q8_0, Q4_K, Q6_K, Q8_K = 2, 8, 12, 14, 15


def dequant_act(blocks: np.ndarray, atype: int, k: int) -> np.ndarray:
    """float64 [m, k] of ggml activation blocks: block_q8_0 (f16 d, int8 qs[32]) or block_q8_K (f32 d, int8 qs[256],
    int16 bsums[16]); each value q * d exactly."""
    b = np.ascontiguousarray(blocks, dtype=np.uint8).reshape(-1)
    if atype == Q8_0:
        r = b.reshape(-1, 34)
        d = r[:, :2].copy().view(np.float16).astype(np.float64)
        q = r[:, 2:].view(np.int8).astype(np.float64)
        return (q * d).reshape(-1, k)
    r = b.reshape(-1, 292)
    d = r[:, :4].copy().view(np.float32).astype(np.float64)
    q = r[:, 4:260].view(np.int8).astype(np.float64)
    return (q * d).reshape(-1, k)


def act_type_of(wtype: int) -> int:
    return Q8_K if wtype in (Q4_K, Q6_K) else Q8_0


def per_output_gate(got, w_deq, a_deq, tol: float = TOL_EXACT, what: str = "") -> float:
    """Asserts the gate for got [m, n] (or [n] for one activation row) against the dequantized operands w_deq
    [n, k] and a_deq [m, k]; returns the worst |got - ref| / sum |w a| for the log."""
    w = np.asarray(w_deq, np.float64)
    a = np.asarray(a_deq, np.float64).reshape(-1, w.shape[1])
    g = np.asarray(got, np.float64).reshape(a.shape[0], w.shape[0])
    ref = a @ w.T
    mag = np.abs(a) @ np.abs(w).T
    ratio = np.abs(g - ref) / np.maximum(mag, 1e-300)
    ratio[(mag == 0) & (g == 0)] = 0.0
    worst = float(ratio.max()) if ratio.size else 0.0
    assert np.isfinite(g).all(), f"{what}: non-finite output"
    if worst > tol:
        i = np.unravel_index(int(ratio.argmax()), ratio.shape)
        raise AssertionError(f"{what}: per-output error {worst:.3g} > {tol:.3g} at (token, row) {tuple(map(int, i))}: "
                             f"got {g[i]:.9g}, ref {ref[i]:.9g}, sum|w a| {mag[i]:.6g}")
    return worst
