"""Python host binding of the BitNet b1.58 per-token GPU engine (libac_bitnet_hip.so).

Mirrors the reference's AcBitNetEngine (adapters/bitnet/src/core/ac_bitnet_engine.h: Configure, UploadLayer,
UploadOutput, EvalToken, LMHead) over the library's C entry points (include/ac_bitnet_engine_hip.h). Failures raise
AcBitNetError carrying the AcResult code and the engine's message, as the reference's C++ engine throws. Host arrays
are numpy; the engine copies them into HBM at upload and reads x / logits back at every EvalToken.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libac_bitnet_hip.so")
_LIB = None

LAYER_TENSORS = ("attn_norm", "attn_sub_norm", "ffn_norm", "ffn_sub_norm", "wq", "wk", "wv", "wo", "w_gate", "w_up",
                 "w_down")
LAYER_SCALES = ("scale_wq", "scale_wk", "scale_wv", "scale_wo", "scale_w_gate", "scale_w_up", "scale_w_down")


class ConfigC(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint32) for n in ("n_embd", "n_ffn", "n_heads", "n_kv_heads", "head_dim", "n_ctx",
                                               "n_layers")] + \
               [("norm_eps", ctypes.c_float), ("rope_theta", ctypes.c_float), ("relu2_ffn", ctypes.c_int32)]


class LayerC(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in LAYER_TENSORS] + [(n, ctypes.c_float) for n in LAYER_SCALES]


class AcBitNetError(RuntimeError):
    def __init__(self, msg: str, result: int):
        super().__init__(f"{msg} (AcResult {result})")
        self.result = result


def lib():
    """The loaded engine library; raises when it has not been built (there is no CPU fallback)."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"{_LIB_PATH} is missing: build it with __graft_entry__.build()")
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        L.ac_bitnet_engine_create.restype = P
        L.ac_bitnet_engine_configure.argtypes = [P, ctypes.POINTER(ConfigC)]
        L.ac_bitnet_engine_upload_layer.argtypes = [P, ctypes.c_uint32, ctypes.POINTER(LayerC)]
        L.ac_bitnet_engine_upload_output.argtypes = [P, P, P, ctypes.c_uint32]
        L.ac_bitnet_engine_eval_token.argtypes = [P, ctypes.c_uint32, P, P, P, ctypes.c_uint32]
        L.ac_bitnet_engine_lm_head.argtypes = [P, P, P]
        L.ac_bitnet_engine_last_error.argtypes = [P]
        L.ac_bitnet_engine_last_error.restype = ctypes.c_char_p
        L.ac_bitnet_engine_destroy.argtypes = [P]
        _LIB = L
    return _LIB


def _ptr(a):
    return None if a is None else a.ctypes.data


class BitNetEngine:
    """One engine on the current HIP device (ac_bitnet_engine.h's AcBitNetEngine)."""

    def __init__(self):
        L = lib()
        self._h = L.ac_bitnet_engine_create()
        if not self._h:
            raise AcBitNetError(L.ac_bitnet_engine_last_error(None).decode(), -1)
        self.cfg = None
        self.n_vocab = 0

    def _check(self, rc: int):
        if rc != 0:
            raise AcBitNetError(lib().ac_bitnet_engine_last_error(self._h).decode(), rc)

    def configure(self, n_embd, n_ffn, n_heads, n_kv_heads, head_dim, n_ctx, n_layers, norm_eps=1e-5,
                  rope_theta=10000.0, relu2_ffn=False):
        c = ConfigC(n_embd, n_ffn, n_heads, n_kv_heads, head_dim, n_ctx, n_layers, norm_eps, rope_theta,
                    int(bool(relu2_ffn)))
        self._check(lib().ac_bitnet_engine_configure(self._h, ctypes.byref(c)))
        self.cfg = c

    def upload_layer(self, index: int, layer: dict):
        """layer: the f32 norm vectors, the packed I2_S weights (uint8, rows x k/4) and the per-tensor scales, under
        the reference's BitNetGpuLayerHost field names; absent sub norms are None or missing."""
        keep = {n: (None if layer.get(n) is None else np.ascontiguousarray(layer[n])) for n in LAYER_TENSORS}
        lc = LayerC(*[_ptr(keep[n]) for n in LAYER_TENSORS], *[float(layer.get(n, 1.0)) for n in LAYER_SCALES])
        self._check(lib().ac_bitnet_engine_upload_layer(self._h, index, ctypes.byref(lc)))

    def upload_output(self, output_norm, lm_head_f16):
        """output_norm f32 [n_embd]; lm_head_f16 uint16 (f16 bits) or float16 [n_vocab, n_embd]."""
        on = np.ascontiguousarray(output_norm, np.float32)
        head = np.ascontiguousarray(lm_head_f16)
        if head.dtype == np.float16:
            head = head.view(np.uint16)
        self._check(lib().ac_bitnet_engine_upload_output(self._h, _ptr(on), _ptr(head), head.shape[0]))
        self.n_vocab = head.shape[0]

    def eval_token(self, pos: int, x_in, x_out=None, logits=None, chunk_layers: int = 0):
        """One token step at position pos; x_out / logits are filled when given (float32 arrays)."""
        x = np.ascontiguousarray(x_in, np.float32)
        self._check(lib().ac_bitnet_engine_eval_token(self._h, pos, _ptr(x), _ptr(x_out), _ptr(logits), chunk_layers))

    def lm_head(self, x_norm, logits):
        x = np.ascontiguousarray(x_norm, np.float32)
        self._check(lib().ac_bitnet_engine_lm_head(self._h, _ptr(x), _ptr(logits)))

    def close(self):
        if self._h:
            lib().ac_bitnet_engine_destroy(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
