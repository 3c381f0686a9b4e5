"""ctypes binding of the CPU parity checker (libameva_oracle.so, built from ameva_oracle.c).

TEST INFRASTRUCTURE ONLY: tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use this module as the
checker. The product package (ameva_compute_amd) never imports it.

Every function restates a ggml CPU rule; ameva_oracle.c names the reference file:line each one follows. Arrays are
numpy; quantized data are uint8 arrays holding ggml blocks in ggml's own byte layout.
"""
from __future__ import annotations

import ctypes
import os
import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libameva_oracle.so")
REF_I2S_PATH = os.path.join(HERE, "_ref", "libbitnet_mad_ref.so")
SIMD_PATH = os.path.join(HERE, "libameva_cpu_simd.so")

# ggml_type values (include/ggml/ggml.h:394-437)
Q4_0, Q8_0, Q4_K, Q6_K, Q8_K, I2_S = 2, 8, 12, 14, 15, 36
BLOCK = {Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210), Q8_K: (256, 292)}
# Q8_0 quantization rules (ameva_oracle.c orc_quantize_q8_0)
Q8_X86, Q8_ARM, Q8_REF = 0, 1, 2

_lib = None


def build() -> None:
    import subprocess
    subprocess.run(["make", "-s", "-C", HERE, "all"], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        _lib = ctypes.CDLL(LIB_PATH)
        P, I64, F = ctypes.c_void_p, ctypes.c_int64, ctypes.c_float
        sig = {
            "orc_fp32_to_fp16_n": (None, [P, P, I64]),
            "orc_fp16_to_fp32_n": (None, [P, P, I64]),
            "orc_quantize_q4_0": (None, [P, P, I64, I64]),
            "orc_quantize_q8_0": (None, [P, P, I64, I64, ctypes.c_int]),
            "orc_quantize_q8_K": (None, [P, P, I64, I64]),
            "orc_dequantize": (ctypes.c_int, [ctypes.c_int, P, P, I64]),
            "orc_mul_mat": (ctypes.c_int, [ctypes.c_int, P, I64, I64, P, I64, P, P]),
            "orc_num_threads": (ctypes.c_int, []),
            "orc_rms_norm": (None, [P, P, P, P, I64, I64, F]),
            "orc_rope": (None, [P, P, P, I64, I64, I64, ctypes.c_int, ctypes.c_int, F, F, F]),
            "orc_swiglu": (None, [P, P, P, I64]),
            "orc_flash_attn_decode": (None, [P, P, P, P, P, I64, I64, I64, I64, F]),
            "orc_flash_attn_decode_q": (ctypes.c_int, [ctypes.c_int, P, P, P, P, P, I64, I64, I64, I64, F,
                                                       ctypes.c_int]),
            "orc_i2s_quantize_act": (F, [P, P, I64]),
            "orc_bitnet_rms_norm": (None, [P, P, P, I64, F]),
            "orc_bitnet_gemv_f16": (None, [P, P, P, I64, I64]),
            "orc_bitnet_attention": (None, [P, P, P, P, I64, I64, I64, I64]),
            "orc_bitnet_token": (None, [P, I64, I64, I64, I64, I64, I64, I64, F, F, ctypes.c_int, P, P, I64, P, P,
                                        P, I64, P]),
            "orc_i2s_dot_row": (I64, [I64, P, P, P]),
            "orc_i2s_gemv": (None, [P, I64, I64, P, P, I64, F, P, P]),
            "orc_i2s_dequantize": (None, [P, F, I64, P]),
            "orc_i2s_trailer_scale": (F, [P, I64, I64]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(_lib, name)
            fn.restype = res
            fn.argtypes = args
    return _lib


_simd = None


def cpu_simd():
    """The CPU baseline kernels (cpu_simd.c, AVX2 / FMA / F16C), or None when this CPU lacks those extensions. Used by
    bench.py's cpu_baseline leg only; the parity checker is lib()."""
    global _simd
    if _simd is None:
        try:
            with open("/proc/cpuinfo") as f:
                flags = next((ln.split(":", 1)[1].split() for ln in f if ln.startswith("flags")), [])
        except OSError:
            flags = []
        if not all(x in flags for x in ("avx2", "fma", "f16c")):
            return None
        if not os.path.exists(SIMD_PATH):
            build()
        _simd = ctypes.CDLL(SIMD_PATH)
        P, I64, F = ctypes.c_void_p, ctypes.c_int64, ctypes.c_float
        _simd.cpu_mul_mat_q4_0.restype = None
        _simd.cpu_mul_mat_q4_0.argtypes = [P, I64, I64, P, I64, P]
        _simd.cpu_flash_attn_decode_f16.restype = None
        _simd.cpu_flash_attn_decode_f16.argtypes = [P, P, P, P, I64, I64, I64, I64, F]
        _simd.cpu_num_threads.restype = ctypes.c_int
        _simd.cpu_num_threads.argtypes = []
    return _simd


def simd_mul_mat_q4_0(w: np.ndarray, n_rows: int, k: int, a_q: np.ndarray, m: int, out: np.ndarray | None = None):
    """CPU baseline Q4_0 x Q8_0 MUL_MAT (ggml's AVX2 vec_dot algorithm): [m][n_rows] f32."""
    if out is None:
        out = np.empty((m, n_rows), np.float32)
    cpu_simd().cpu_mul_mat_q4_0(_p(w), n_rows, k, _p(a_q), m, _p(out))
    return out


def simd_flash_attn_decode(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float) -> np.ndarray:
    """CPU baseline decode attention: q f32 [n_head][D], k / v f16 [n_kv][n_head_kv][D] -> [n_head][D]."""
    n_head, D = q.shape
    n_kv, n_head_kv, _ = k.shape
    assert D % 8 == 0 and D <= 256 and n_head % n_head_kv == 0
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.float16)
    v = np.ascontiguousarray(v, np.float16)
    out = np.empty((n_head, D), np.float32)
    cpu_simd().cpu_flash_attn_decode_f16(_p(q), _p(k), _p(v), _p(out), n_head, n_head_kv, n_kv, D, scale)
    return out


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(ctypes.c_void_p)


def row_bytes(t: int, k: int) -> int:
    be, bb = BLOCK[t]
    assert k % be == 0
    return k // be * bb


def fp32_to_fp16(x) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.empty(x.shape, dtype=np.uint16)
    lib().orc_fp32_to_fp16_n(_p(x), _p(y), x.size)
    return y


def fp16_to_fp32(h) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    y = np.empty(h.shape, dtype=np.float32)
    lib().orc_fp16_to_fp32_n(_p(h), _p(y), h.size)
    return y


def quantize_q4_0(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, k = x.reshape(-1, x.shape[-1]).shape
    y = np.empty((rows, row_bytes(Q4_0, k)), dtype=np.uint8)
    lib().orc_quantize_q4_0(_p(x), _p(y), rows, k)
    return y


def quantize_q8_0(x: np.ndarray, rule: int = Q8_X86) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, k = x.reshape(-1, x.shape[-1]).shape
    y = np.empty((rows, row_bytes(Q8_0, k)), dtype=np.uint8)
    lib().orc_quantize_q8_0(_p(x), _p(y), rows, k, rule)
    return y


def quantize_q8_K(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, k = x.reshape(-1, x.shape[-1]).shape
    y = np.empty((rows, row_bytes(Q8_K, k)), dtype=np.uint8)
    lib().orc_quantize_q8_K(_p(x), _p(y), rows, k)
    return y


def dequantize(t: int, blocks: np.ndarray, k: int) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, dtype=np.uint8)
    rows = blocks.size // row_bytes(t, k)
    y = np.empty((rows, k), dtype=np.float32)
    rc = lib().orc_dequantize(t, _p(blocks), _p(y), rows * k)
    assert rc == 0
    return y


def act_type(wtype: int) -> int:
    return Q8_K if wtype in (Q4_K, Q6_K) else Q8_0


def mul_mat(wtype: int, w: np.ndarray, n_rows: int, k: int, a_q: np.ndarray, m: int, with_blocks: bool = False):
    """dst [m, n_rows] f32 = W (ggml blocks, [n_rows, k]) . quantized activations [m, k]. With with_blocks also the
    per-block integer sums [m, n_rows, nblk(*2 for Q4_K)] int32."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    a_q = np.ascontiguousarray(a_q, dtype=np.uint8)
    assert w.size == n_rows * row_bytes(wtype, k)
    assert a_q.size == m * row_bytes(act_type(wtype), k)
    dst = np.empty((m, n_rows), dtype=np.float32)
    blk = None
    if with_blocks:
        be = BLOCK[wtype][0]
        per = 2 if wtype == Q4_K else 1
        blk = np.empty((m, n_rows, k // be * per), dtype=np.int32)
    rc = lib().orc_mul_mat(wtype, _p(w), n_rows, k, _p(a_q), m, _p(dst), _p(blk) if blk is not None else None)
    assert rc == 0
    return (dst, blk) if with_blocks else dst


def num_threads() -> int:
    return lib().orc_num_threads()


def rms_norm(x: np.ndarray, eps: float, w: np.ndarray | None = None):
    x = np.ascontiguousarray(x, dtype=np.float32)
    n = x.shape[-1]
    rows = x.size // n
    y = np.empty_like(x)
    if w is None:
        lib().orc_rms_norm(_p(x), _p(y), None, None, rows, n, eps)
        return y
    w = np.ascontiguousarray(w, dtype=np.float32)
    o = np.empty_like(x)
    lib().orc_rms_norm(_p(x), _p(y), _p(w), _p(o), rows, n, eps)
    return y, o


def rope(x: np.ndarray, pos: np.ndarray, n_dims: int, mode: int = 0, freq_base: float = 10000.0,
         freq_scale: float = 1.0, attn_factor: float = 1.0) -> np.ndarray:
    """x [n_tok, n_head, ne0] f32, pos [n_tok] int32."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    pos = np.ascontiguousarray(pos, dtype=np.int32)
    n_tok, n_head, ne0 = x.shape
    y = np.empty_like(x)
    lib().orc_rope(_p(x), _p(y), _p(pos), n_tok, n_head, ne0, n_dims, mode, freq_base, freq_scale, attn_factor)
    return y


def swiglu(g: np.ndarray, u: np.ndarray) -> np.ndarray:
    g = np.ascontiguousarray(g, dtype=np.float32)
    u = np.ascontiguousarray(u, dtype=np.float32)
    y = np.empty_like(g)
    lib().orc_swiglu(_p(g), _p(u), _p(y), g.size)
    return y


def flash_attn_decode(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float, mask: np.ndarray | None = None):
    """q f32 [n_head, D]; k, v f16 bits (uint16) [n_head_kv, n_kv, D]; mask f16 bits [n_kv] or None."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.uint16)
    v = np.ascontiguousarray(v, dtype=np.uint16)
    n_head, D = q.shape
    n_head_kv, n_kv, _ = k.shape
    out = np.empty((n_head, D), dtype=np.float32)
    mp = None
    if mask is not None:
        mask = np.ascontiguousarray(mask, dtype=np.uint16)
        mp = _p(mask)
    lib().orc_flash_attn_decode(_p(q), _p(k), _p(v), mp, _p(out), n_head, n_head_kv, n_kv, D, scale)
    return out


def flash_attn_decode_q(kv_type: int, q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float,
                        mask: np.ndarray | None = None, rule: int = Q8_X86):
    """q f32 [n_head, D]; k, v uint8 [n_head_kv, n_kv, row bytes] of Q8_0 (kv_type 8) or Q4_0 (2) blocks; mask f16
    bits [n_kv] or None."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.uint8)
    v = np.ascontiguousarray(v, dtype=np.uint8)
    n_head, D = q.shape
    n_head_kv, n_kv, _ = k.shape
    out = np.empty((n_head, D), dtype=np.float32)
    mp = None
    if mask is not None:
        mask = np.ascontiguousarray(mask, dtype=np.uint16)
        mp = _p(mask)
    rc = lib().orc_flash_attn_decode_q(kv_type, _p(q), _p(k), _p(v), mp, _p(out), n_head, n_head_kv, n_kv, D,
                                       scale, rule)
    assert rc == 0
    return out


def flash_attn_prefill(q: np.ndarray, k: np.ndarray, v: np.ndarray, scale: float, causal_pos0: int = -1,
                       mask: np.ndarray | None = None):
    """q f32 [n_tok, n_head, D]; k, v f16 bits [n_head_kv, n_kv, D]; mask f16 bits [n_tok, n_kv] or None.
    Query t is the decode of flash_attn_decode over the keys it may see: all n_kv, or with causal_pos0 >= 0 the
    first causal_pos0 + t + 1 (ggml's causal KQ mask hides the later ones), plus its mask row."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    n_tok, n_head, D = q.shape
    n_kv = k.shape[1]
    out = np.zeros((n_tok, n_head, D), dtype=np.float32)
    for t in range(n_tok):
        nk = n_kv if causal_pos0 < 0 else min(n_kv, causal_pos0 + t + 1)
        if nk <= 0:
            continue
        mrow = None if mask is None else np.ascontiguousarray(mask[t, :nk])
        out[t] = flash_attn_decode(q[t], np.ascontiguousarray(k[:, :nk]), np.ascontiguousarray(v[:, :nk]), scale,
                                   mrow)
    return out


def i2s_quantize_act(x: np.ndarray):
    """Per-row absmax int8 quantization; returns (q int8 [rows, n], dequant f32 [rows])."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    x2 = x.reshape(-1, x.shape[-1])
    q = np.empty(x2.shape, dtype=np.int8)
    deq = np.empty(x2.shape[0], dtype=np.float32)
    for r in range(x2.shape[0]):
        deq[r] = lib().orc_i2s_quantize_act(_p(x2[r]), _p(q[r]), x2.shape[1])
    return q, deq


def i2s_gemv(w: np.ndarray, n_rows: int, k: int, q: np.ndarray, deq: np.ndarray, weight_scale: float):
    """out f32 [m, n_rows] and the exact integer sums int64 [m, n_rows]."""
    w = np.ascontiguousarray(w, dtype=np.uint8)
    q = np.ascontiguousarray(q, dtype=np.int8)
    deq = np.ascontiguousarray(deq, dtype=np.float32)
    m = q.size // k
    assert w.size >= n_rows * k // 4
    out = np.empty((m, n_rows), dtype=np.float32)
    sums = np.empty((m, n_rows), dtype=np.int64)
    lib().orc_i2s_gemv(_p(w), n_rows, k, _p(q), _p(deq), m, weight_scale, _p(out), _p(sums))
    return out, sums


def i2s_dequantize(w: np.ndarray, scale: float, n: int) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint8)
    y = np.empty(n, dtype=np.float32)
    lib().orc_i2s_dequantize(_p(w), scale, n, _p(y))
    return y


def i2s_trailer_scale(tensor: np.ndarray, n_rows: int, k: int) -> float:
    tensor = np.ascontiguousarray(tensor, dtype=np.uint8)
    return float(lib().orc_i2s_trailer_scale(_p(tensor), n_rows, k))


class RefI2S:
    """The reference's own scalar ggml_vec_dot_i2_i8_s (oracle/_ref, compiled from /root/reference by the Makefile)."""

    def __init__(self):
        self.lib = ctypes.CDLL(REF_I2S_PATH)
        # C++ symbol of ggml_vec_dot_i2_i8_s(int, float*, size_t, const void*, size_t, const void*, size_t, int, int)
        self.fn = getattr(self.lib, "_Z20ggml_vec_dot_i2_i8_siPfmPKvmS1_mii")
        self.fn.restype = None
        self.fn.argtypes = [ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_size_t,
                            ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int, ctypes.c_int]

    @staticmethod
    def available() -> bool:
        return os.path.exists(REF_I2S_PATH)

    def gemv_sums(self, w: np.ndarray, n_rows: int, k: int, q: np.ndarray) -> np.ndarray:
        """(float)sumi per row as the reference computes it (type 0 = Nx1, bx = k)."""
        w = np.ascontiguousarray(w, dtype=np.uint8)
        q = np.ascontiguousarray(q, dtype=np.int8)
        s = np.empty(n_rows, dtype=np.float32)
        self.fn(k, _p(s), 1, _p(w), k, _p(q), k, n_rows, 0)
        return s


class BitnetLayer(ctypes.Structure):
    """OrcBitnetLayer: one BitNet layer on the host (F32 norms, sub norms may be NULL; I2_S projections; scales)."""
    _fields_ = [(n, ctypes.c_void_p) for n in ("attn_norm", "attn_sub_norm", "ffn_norm", "ffn_sub_norm", "wq", "wk",
                                               "wv", "wo", "w_gate", "w_up", "w_down")] + \
               [(n, ctypes.c_float) for n in ("scale_wq", "scale_wk", "scale_wv", "scale_wo", "scale_w_gate",
                                              "scale_w_up", "scale_w_down")]


def bitnet_rms_norm(x: np.ndarray, w, eps: float) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    wp = None if w is None else _p(np.ascontiguousarray(w, dtype=np.float32))
    lib().orc_bitnet_rms_norm(_p(out), _p(x), wp, x.size, eps)
    return out


def bitnet_gemv_f16(w: np.ndarray, x: np.ndarray) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint16)
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(w.shape[0], np.float32)
    lib().orc_bitnet_gemv_f16(_p(out), _p(w), _p(x), w.shape[1], w.shape[0])
    return out


def bitnet_attention(q: np.ndarray, kc: np.ndarray, vc: np.ndarray, pos: int, n_kv_heads: int) -> np.ndarray:
    """q [n_heads, hd]; kc, vc [n_ctx, n_kv_heads * hd] of one layer; keys 0 .. pos."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    kc = np.ascontiguousarray(kc, dtype=np.float32)
    vc = np.ascontiguousarray(vc, dtype=np.float32)
    out = np.empty_like(q)
    lib().orc_bitnet_attention(_p(out), _p(q), _p(kc), _p(vc), pos, q.shape[0], n_kv_heads, q.shape[1])
    return out


class BitnetModel:
    """A BitNet model on the host for orc_bitnet_token: layers (list of dicts of numpy arrays and scales), caches
    [n_layers, n_ctx, kv] kept here between tokens."""

    def __init__(self, cfg: dict, layers: list, out_norm: np.ndarray, lm_head: np.ndarray):
        self.cfg = cfg
        self.keep = []
        arr = (BitnetLayer * len(layers))()
        for i, L in enumerate(layers):
            for n in ("attn_norm", "attn_sub_norm", "ffn_norm", "ffn_sub_norm", "wq", "wk", "wv", "wo", "w_gate",
                      "w_up", "w_down"):
                a = L.get(n)
                if a is not None:
                    a = np.ascontiguousarray(a)
                    self.keep.append(a)
                    setattr(arr[i], n, a.ctypes.data)
            for n in ("scale_wq", "scale_wk", "scale_wv", "scale_wo", "scale_w_gate", "scale_w_up", "scale_w_down"):
                setattr(arr[i], n, float(L.get(n, 1.0)))
        self.layers = arr
        self.out_norm = np.ascontiguousarray(out_norm, dtype=np.float32)
        self.lm_head = np.ascontiguousarray(lm_head, dtype=np.uint16)
        kv = cfg["n_kv_heads"] * cfg["head_dim"]
        self.kc = np.zeros((len(layers), cfg["n_ctx"], kv), np.float32)
        self.vc = np.zeros_like(self.kc)

    def token(self, pos: int, x: np.ndarray, logits: bool = True):
        c = self.cfg
        x = np.array(x, dtype=np.float32)
        lg = np.empty(self.lm_head.shape[0], np.float32) if logits else None
        lib().orc_bitnet_token(self.layers, len(self.layers), c["n_embd"], c["n_ffn"], c["n_heads"], c["n_kv_heads"],
                               c["head_dim"], c["n_ctx"], c["norm_eps"], c["rope_theta"], int(c["relu2"]),
                               _p(self.kc), _p(self.vc), pos, _p(x), _p(self.out_norm), _p(self.lm_head),
                               self.lm_head.shape[0], None if lg is None else _p(lg))
        return x, lg
