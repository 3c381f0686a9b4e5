"""Host mirror of the reference's ggml backend operator surface for the quantized hot path, over the C ABI.

The reference backend executes ggml nodes (adapters/llama/ggml-ameva/ggml-ameva.cpp: enc_mul_mat 3607,
enc_rms_norm 3941, enc_rope 3965, enc_flash_attn 4204); these functions take the same operands with the same
meaning (ggml_mul_mat: dst = src0^T x src1, i.e. dst[m][n] = sum_k W[n][k] x[m][k]) as torch tensors on the GPU and
run the HIP kernels on torch's current stream. Unsupported shapes or types raise (the reference's FAIL-FAST), and
there is no CPU path.
"""
from __future__ import annotations

import torch

from ._lib import check, lib

# ggml_type values (reference include/ggml/ggml.h:394-437)
Q4_0, Q8_0, Q4_K, Q6_K, Q8_K, I2_S = 2, 8, 12, 14, 15, 36
# Q8_0 activation rounding rules (include/ameva_hip.h)
Q8_X86, Q8_ARM, Q8_REF = 0, 1, 2

BLOCK = {Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210), Q8_K: (256, 292)}


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _ptr(t: torch.Tensor | None):
    return None if t is None else t.data_ptr()


def _need_gpu(t: torch.Tensor, what: str) -> None:
    if not t.is_cuda:
        raise ValueError(f"{what}: tensor must be on the GPU (no CPU path)")
    if not t.is_contiguous():
        raise ValueError(f"{what}: tensor must be contiguous")


def act_type(wtype: int) -> int:
    """ggml vec_dot_type of a weight type: Q8_0 for Q4_0/Q8_0, Q8_K for the K-quants."""
    return Q8_K if wtype in (Q4_K, Q6_K) else Q8_0


def ggml_row_bytes(t: int, k: int) -> int:
    be, bb = BLOCK[t]
    if k % be:
        raise ValueError(f"row of {k} elements is not whole blocks of type {t}")
    return k // be * bb


class QWeight:
    """A quantized weight resident in HBM in the MI355X layout (what the reference's set_tensor produces for a
    WEIGHTS buffer, ggml-ameva-buffer.cpp:509). Same byte count as the ggml tensor; to_ggml() restores its bytes."""

    def __init__(self, wtype: int, n_rows: int, k: int, data: torch.Tensor):
        self.type, self.n_rows, self.k, self.data = wtype, n_rows, k, data

    @classmethod
    def from_ggml(cls, wtype: int, ggml_bytes: torch.Tensor, n_rows: int, k: int) -> "QWeight":
        _need_gpu(ggml_bytes, "QWeight.from_ggml")
        nbytes = lib().amv_weight_bytes(wtype, n_rows, k)
        if nbytes < 0 or ggml_bytes.numel() * ggml_bytes.element_size() < nbytes:
            raise ValueError(f"QWeight.from_ggml: type {wtype} {n_rows}x{k} needs {nbytes} bytes")
        out = torch.empty(nbytes, dtype=torch.uint8, device=ggml_bytes.device)
        check(lib().amv_repack(wtype, ggml_bytes.data_ptr(), out.data_ptr(), n_rows, k, _stream()), "amv_repack")
        return cls(wtype, n_rows, k, out)

    def to_ggml(self) -> torch.Tensor:
        out = torch.empty_like(self.data)
        check(lib().amv_unrepack(self.type, self.data.data_ptr(), out.data_ptr(), self.n_rows, self.k, _stream()),
              "amv_unrepack")
        return out

    @property
    def nbytes(self) -> int:
        return self.data.numel()


def quantize_act(x: torch.Tensor, atype: int = Q8_0, rule: int = Q8_X86, ggml: bool = False):
    """Quantize f32 activations [m, k] to the kernels' layout; with ggml=True also to ggml blocks.
    Returns (act uint8, ggml_blocks uint8 [m, row_bytes] or None)."""
    _need_gpu(x, "quantize_act")
    if x.dtype != torch.float32:
        raise ValueError("quantize_act: f32 input expected")
    x2 = x.reshape(-1, x.shape[-1])
    m, k = x2.shape
    n = lib().amv_act_bytes(atype, m, k)
    if n < 0:
        raise ValueError(f"quantize_act: type {atype} cannot hold rows of {k}")
    act = torch.empty(n, dtype=torch.uint8, device=x.device)
    g = torch.empty((m, ggml_row_bytes(atype, k)), dtype=torch.uint8, device=x.device) if ggml else None
    check(lib().amv_quantize_act(atype, x2.data_ptr(), m, k, rule, _ptr(g), act.data_ptr(), _stream()),
          "amv_quantize_act")
    return act, g


def quantize_q4_0(x: torch.Tensor) -> torch.Tensor:
    """f32 rows [n, k] -> ggml Q4_0 blocks [n, k/32*18] (ggml quantize_row_q4_0_ref)."""
    _need_gpu(x, "quantize_q4_0")
    x2 = x.reshape(-1, x.shape[-1])
    n, k = x2.shape
    y = torch.empty((n, ggml_row_bytes(Q4_0, k)), dtype=torch.uint8, device=x.device)
    check(lib().amv_quantize_q4_0(x2.data_ptr(), n, k, y.data_ptr(), _stream()), "amv_quantize_q4_0")
    return y


def mul_mat_q(w: QWeight, act: torch.Tensor, m: int, out: torch.Tensor | None = None) -> torch.Tensor:
    """dst [m, n_rows] f32 from already quantized activations (amv_quantize_act layout of m rows)."""
    _need_gpu(act, "mul_mat_q")
    if out is None:
        out = torch.empty((m, w.n_rows), dtype=torch.float32, device=act.device)
    check(lib().amv_mul_mat_vec(w.type, w.data.data_ptr(), w.n_rows, w.k, act.data_ptr(), m, out.data_ptr(),
                                w.n_rows, _stream()), "amv_mul_mat_vec")
    return out


def mul_mat(w: QWeight, x: torch.Tensor, rule: int = Q8_X86) -> torch.Tensor:
    """ggml_mul_mat(src0 = w, src1 = x): x f32 [m, k] -> [m, n_rows]; activations quantized to vec_dot_type."""
    x2 = x.reshape(-1, x.shape[-1])
    if x2.shape[1] != w.k:
        raise ValueError(f"mul_mat: k mismatch {x2.shape[1]} != {w.k}")
    act, _ = quantize_act(x2, act_type(w.type), rule)
    return mul_mat_q(w, act, x2.shape[0])


def block_sums(w: QWeight, act: torch.Tensor, m: int) -> torch.Tensor:
    """The exact per-block int32 sums of the GEMV kernels, [m, n_rows, nblk(*2 for Q4_K)]."""
    be = BLOCK[w.type][0]
    per = 2 if w.type == Q4_K else 1
    out = torch.empty((m, w.n_rows, w.k // be * per), dtype=torch.int32, device=act.device)
    check(lib().amv_mul_mat_block_sums(w.type, w.data.data_ptr(), w.n_rows, w.k, act.data_ptr(), m, out.data_ptr(),
                                       _stream()), "amv_mul_mat_block_sums")
    return out
