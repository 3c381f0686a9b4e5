"""Host mirror of the reference's ggml backend operator surface for the quantized hot path, over the C ABI.

The reference backend executes ggml nodes (adapters/llama/ggml-ameva/ggml-ameva.cpp: enc_mul_mat 3607,
enc_rms_norm 3941, enc_rope 3965, enc_flash_attn 4204); these functions take the same operands with the same
meaning (ggml_mul_mat: dst = src0^T x src1, i.e. dst[m][n] = sum_k W[n][k] x[m][k]) as torch tensors on the GPU and
run the HIP kernels on torch's current stream. Unsupported shapes or types raise (the reference's FAIL-FAST), and
there is no CPU path.
"""
from __future__ import annotations

import os

import torch

from ._lib import check, lib

# ggml_type values (reference include/ggml/ggml.h:394-437)
F32, F16, Q4_0, Q8_0, Q4_K, Q6_K, Q8_K, I2_S = 0, 1, 2, 8, 12, 14, 15, 36
# Q8_0 activation rounding rules (include/ameva_hip.h)
Q8_X86, Q8_ARM, Q8_REF = 0, 1, 2

BLOCK = {Q4_0: (32, 18), Q8_0: (32, 34), Q4_K: (256, 144), Q6_K: (256, 210), Q8_K: (256, 292)}


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _ptr(t: torch.Tensor | None):
    return None if t is None else t.data_ptr()


def _need_gpu(t: torch.Tensor, what: str, contiguous: bool = True) -> None:
    if not t.is_cuda:
        raise ValueError(f"{what}: tensor must be on the GPU (no CPU path)")
    if contiguous and not t.is_contiguous():
        raise ValueError(f"{what}: tensor must be contiguous")


# Q8_K activations with the f16 copies the batched Q4_K MUL_MAT reads (include/ameva_hip.h AMV_ACT_Q8_K_MMA)
Q8_K_MMA = 1015
Q8_0_MMA = 1008
# the same layouts with f16 q * d in place of f16 q: the scaled batched MUL_MAT (AMV_ACT_Q8_K_DEQ / AMV_ACT_Q8_0_DEQ)
Q8_K_DEQ = 1115
Q8_0_DEQ = 1108


# The batched MUL_MAT's arithmetic above MMQ16_MIN_M tokens: "exact" (the default: exact per-block integer sums and
# ggml's f32 epilogue, the reference's MMQ arithmetic) or "scaled" (operands rounded to f16 once, ~3e-4 relative L2
# from the exact value), chosen with AMEVA_MMQ_FORM.
MMQ_FORM = os.environ.get("AMEVA_MMQ_FORM", "exact")
if MMQ_FORM not in ("exact", "scaled"):
    raise ValueError(f"AMEVA_MMQ_FORM={MMQ_FORM!r}: exact or scaled")


def act_type(wtype: int, m: int = 1, exact: bool | None = None) -> int:
    """The activation layout a MUL_MAT of m tokens reads: ggml's vec_dot_type (Q8_0 for Q4_0/Q8_0, Q8_K for the
    K-quants) in the plain layout, except for batched Q4_K of MMQ_MIN_M..MMQ16_MIN_M tokens (the small-batch kernel
    reads the f16 copies of Q8_K_MMA) and for the scaled form above MMQ16_MIN_M tokens when exact is False (DEQ;
    None: MMQ_FORM decides). The exact tiled kernel above MMQ16_MIN_M tokens reads the plain layout."""
    if exact is None:
        exact = MMQ_FORM == "exact"
    if wtype in (Q4_0, Q8_0, Q4_K) and m > MMQ16_MIN_M and not exact:
        return Q8_K_DEQ if wtype == Q4_K else Q8_0_DEQ
    if wtype == Q4_K and MMQ_MIN_M <= m <= MMQ16_MIN_M:
        return Q8_K_MMA
    return Q8_K if wtype in (Q4_K, Q6_K) else Q8_0


def act_layout(wtype: int, act: torch.Tensor, m: int, k: int) -> int:
    """The activation type a buffer of m rows of k holds, told apart by its size (the extended layouts are larger)."""
    n = act.numel() * act.element_size()
    base = Q8_K if wtype in (Q4_K, Q6_K) else Q8_0
    for t in ((Q8_K_MMA,) if base == Q8_K else (Q8_0_MMA,)) + (base,):
        if n >= lib().amv_act_bytes(t, m, k) and (t == base or n == lib().amv_act_bytes(t, m, k)):
            return t
    return base


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
    gt = Q8_K if atype in (Q8_K_MMA, Q8_K_DEQ) else Q8_0 if atype in (Q8_0_MMA, Q8_0_DEQ) else atype
    g = torch.empty((m, ggml_row_bytes(gt, k)), dtype=torch.uint8, device=x.device) if ggml else None
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


# batch size from which MUL_MAT runs the int8-MFMA kernel (AMEVA_QGEMM_MIN_M of the reference, ggml-ameva.cpp:2486)
MMQ_MIN_M = 8
MMQ16_MIN_M = 64  # above this many tokens the tiled kernels run (amv_mmq.hip MMQ16_MIN_M)
MMQ_TYPES = (Q4_0, Q8_0, Q4_K, Q6_K)  # Q4_K of MMQ_MIN_M..MMQ16_MIN_M tokens: the activations must be Q8_K_MMA


def mul_mat_q_add(w: QWeight, act: torch.Tensor, m: int, add: torch.Tensor, act_t: int | None = None,
                  out: torch.Tensor | None = None) -> torch.Tensor:
    """mul_mat_q on the batched kernels followed by ADD of add f32 [m, n_rows] (amv_mul_mat_q_act_add)."""
    _need_gpu(act, "mul_mat_q_add")
    if add.shape != (m, w.n_rows) or add.dtype != torch.float32 or not add.is_contiguous():
        raise ValueError("mul_mat_q_add: add must be contiguous f32 [m, n_rows]")
    if out is None:
        out = torch.empty((m, w.n_rows), dtype=torch.float32, device=act.device)
    at = act_layout(w.type, act, m, w.k) if act_t is None else act_t
    check(lib().amv_mul_mat_q_act_add(w.type, w.data.data_ptr(), w.n_rows, w.k, act.data_ptr(), at, m, out.data_ptr(),
                                      w.n_rows, add.data_ptr(), _stream()), "amv_mul_mat_q_act_add")
    return out


def mul_mat_q(w: QWeight, act: torch.Tensor, m: int, out: torch.Tensor | None = None,
              kernel: str = "auto", act_t: int | None = None) -> torch.Tensor:
    """dst [m, n_rows] f32 from already quantized activations (amv_quantize_act layout of m rows).
    kernel: "auto" (the reference's routing: MFMA GEMM for m >= MMQ_MIN_M where the type has one), "mmv", "mmq".
    Q4_K on "mmq" needs Q8_K_MMA activations up to MMQ16_MIN_M tokens. act_t: the activation layout (the DEQ
    layouts have the MMA sizes, so they must be named; None: told apart by size, i.e. plain or MMA)."""
    _need_gpu(act, "mul_mat_q")
    if out is None:
        out = torch.empty((m, w.n_rows), dtype=torch.float32, device=act.device)
    use_mmq = kernel == "mmq" or (kernel == "auto" and m >= MMQ_MIN_M and w.type in MMQ_TYPES)
    if use_mmq:
        at = act_layout(w.type, act, m, w.k) if act_t is None else act_t
        check(lib().amv_mul_mat_q_act(w.type, w.data.data_ptr(), w.n_rows, w.k, act.data_ptr(), at, m,
                                      out.data_ptr(), w.n_rows, _stream()), "amv_mul_mat_q_act")
    else:
        check(lib().amv_mul_mat_vec(w.type, w.data.data_ptr(), w.n_rows, w.k, act.data_ptr(), m, out.data_ptr(),
                                    w.n_rows, _stream()), "amv_mul_mat_vec")
    return out


# GEMV epilogue modes (amv_mul_mat_vec_ep)
EP_NONE, EP_ADD, EP_SILU_MUL, EP_MUL_SILU, EP_SWIGLU_STACKED = 0, 1, 2, 3, 4


def mul_mat_vec_ep(w: QWeight, act: torch.Tensor, ep_mode: int, e: torch.Tensor | None = None,
                   write_dst: bool = True) -> tuple[torch.Tensor | None, torch.Tensor]:
    """One activation column through the GEMV with a fused epilogue: returns (dst, eout); dst (the MUL_MAT value,
    n_rows floats) is None when write_dst is False. eout has n_rows floats, n_rows / 2 for EP_SWIGLU_STACKED; with
    EP_NONE it is dst."""
    _need_gpu(act, "mul_mat_vec_ep")
    if e is not None and (e.dtype != torch.float32 or not e.is_contiguous() or e.numel() != w.n_rows):
        raise ValueError("mul_mat_vec_ep: e must be contiguous f32 with n_rows elements")
    f32 = dict(dtype=torch.float32, device=act.device)
    dst = torch.empty(w.n_rows, **f32) if write_dst or ep_mode == EP_NONE else None
    eout = None
    if ep_mode != EP_NONE:
        eout = torch.empty(w.n_rows // 2 if ep_mode == EP_SWIGLU_STACKED else w.n_rows, **f32)
    check(lib().amv_mul_mat_vec_ep(w.type, w.data.data_ptr(), w.n_rows, w.k, act.data_ptr(), _ptr(dst), ep_mode,
                                   _ptr(e), _ptr(eout), _stream()), "amv_mul_mat_vec_ep")
    return dst, (dst if eout is None else eout)


def add_norm_counter_words(n_rows: int) -> int:
    """Arrival-counter words of gemv_add_rms_norm (AMV_ADD_NORM_COUNTER_WORDS)."""
    return 32 * (n_rows // 32 + 2)


def swiglu_counter_words(n_rows: int) -> int:
    """Arrival-counter words of gemv_swiglu_act for a stacked weight of n_rows rows (AMV_SWIGLU_COUNTER_WORDS)."""
    return 32 * (n_rows // 64 + 1)


def gemv_add_rms_norm(w: QWeight, act: torch.Tensor, e: torch.Tensor, eps: float, norm_w: torch.Tensor | None,
                      act_t: int = Q8_0, rule: int = Q8_X86, counters: torch.Tensor | None = None):
    """eout = W act + e, then RMS_NORM (+ MUL by norm_w) of eout and its activation row of type act_t, in one
    launch. Returns (v = W act, eout, y = x * scale, o = y * norm_w or None, act_out)."""
    _need_gpu(act, "gemv_add_rms_norm")
    dev = act.device
    n = w.n_rows
    v = torch.empty(n, dtype=torch.float32, device=dev)
    eout = torch.empty(n, dtype=torch.float32, device=dev)
    y = torch.empty(n, dtype=torch.float32, device=dev)
    o = torch.empty(n, dtype=torch.float32, device=dev) if norm_w is not None else None
    a = torch.empty(lib().amv_act_bytes(act_t, 1, n), dtype=torch.uint8, device=dev)
    if counters is None:
        counters = torch.zeros(add_norm_counter_words(n), dtype=torch.int32, device=dev)
    check(lib().amv_gemv_add_rms_norm(w.type, w.data.data_ptr(), n, w.k, act.data_ptr(), v.data_ptr(), e.data_ptr(),
                                      eout.data_ptr(), eps, _ptr(norm_w), y.data_ptr(), _ptr(o), a.data_ptr(), act_t,
                                      rule, counters.data_ptr(), _stream()), "amv_gemv_add_rms_norm")
    return v, eout, y, o, a


def gemv_swiglu_act(w: QWeight, act: torch.Tensor, act_t: int = Q8_0, rule: int = Q8_X86,
                    counters: torch.Tensor | None = None):
    """Stacked gate/up GEMV + SWIGLU + the activation row of the result, one launch. Returns (v, h, act_out)."""
    _need_gpu(act, "gemv_swiglu_act")
    dev = act.device
    F = w.n_rows // 2
    v = torch.empty(w.n_rows, dtype=torch.float32, device=dev)
    h = torch.empty(F, dtype=torch.float32, device=dev)
    a = torch.empty(lib().amv_act_bytes(act_t, 1, F), dtype=torch.uint8, device=dev)
    if counters is None:
        counters = torch.zeros(swiglu_counter_words(w.n_rows), dtype=torch.int32, device=dev)
    check(lib().amv_gemv_swiglu_q8(w.type, w.data.data_ptr(), w.n_rows, w.k, act.data_ptr(), v.data_ptr(),
                                   h.data_ptr(), a.data_ptr(), act_t, rule, counters.data_ptr(), _stream()),
          "amv_gemv_swiglu_q8")
    return v, h, a


def gemv_rope_kv(w: QWeight, act: torch.Tensor, n_head: int, n_head_kv: int, pos: torch.Tensor,
                 k_cache: torch.Tensor, v_cache: torch.Tensor, kv_idx: torch.Tensor, freq_base: float = 500000.0,
                 freq_scale: float = 1.0, attn_factor: float = 1.0, bad: torch.Tensor | None = None) -> torch.Tensor:
    """q/k/v GEMV + ROPE NORMAL of q and k + f16 stores of k and v at cache row kv_idx[0]; returns qkv f32 [n_rows].
    Caches f16 [rows, n_head_kv * D]; pos int32 [1], kv_idx int64 [1] on the device."""
    _need_gpu(act, "gemv_rope_kv")
    D = w.n_rows // (n_head + 2 * n_head_kv)
    qkv = torch.empty(w.n_rows, dtype=torch.float32, device=act.device)
    check(lib().amv_gemv_rope_kv(w.type, w.data.data_ptr(), w.n_rows, w.k, act.data_ptr(), qkv.data_ptr(), n_head,
                                 n_head_kv, D, pos.data_ptr(), freq_base, freq_scale, attn_factor,
                                 k_cache.data_ptr(), v_cache.data_ptr(), k_cache.stride(0), kv_idx.data_ptr(),
                                 k_cache.shape[0], _ptr(bad), _stream()), "amv_gemv_rope_kv")
    return qkv


def mul_mat(w: QWeight, x: torch.Tensor, rule: int = Q8_X86) -> torch.Tensor:
    """ggml_mul_mat(src0 = w, src1 = x): x f32 [m, k] -> [m, n_rows]; activations quantized to vec_dot_type."""
    x2 = x.reshape(-1, x.shape[-1])
    if x2.shape[1] != w.k:
        raise ValueError(f"mul_mat: k mismatch {x2.shape[1]} != {w.k}")
    at = act_type(w.type, x2.shape[0])
    act, _ = quantize_act(x2, at, rule)
    return mul_mat_q(w, act, x2.shape[0], act_t=at)


def block_sums(w: QWeight, act: torch.Tensor, m: int, kernel: str = "mmv") -> torch.Tensor:
    """The exact per-block int32 sums of the GEMV ("mmv") or MFMA GEMM ("mmq") kernels, [m, n_rows, nblk(*2 Q4_K)]."""
    be = BLOCK[w.type][0]
    per = 2 if w.type == Q4_K else 1
    out = torch.empty((m, w.n_rows, w.k // be * per), dtype=torch.int32, device=act.device)
    if kernel == "mmq":
        check(lib().amv_mul_mat_q_act_block_sums(w.type, w.data.data_ptr(), w.n_rows, w.k, act.data_ptr(),
                                                 act_layout(w.type, act, m, w.k), m, out.data_ptr(), _stream()),
              "amv_mul_mat_q_act_block_sums")
    else:
        check(lib().amv_mul_mat_block_sums(w.type, w.data.data_ptr(), w.n_rows, w.k, act.data_ptr(), m,
                                           out.data_ptr(), _stream()), "amv_mul_mat_block_sums")
    return out


def quantize_k(x: torch.Tensor, wtype: int) -> torch.Tensor:
    """f32 rows [n, k] -> ggml Q4_K / Q6_K blocks with this library's own rule (see include/ameva_hip.h)."""
    _need_gpu(x, "quantize_k")
    x2 = x.reshape(-1, x.shape[-1])
    n, k = x2.shape
    y = torch.empty((n, ggml_row_bytes(wtype, k)), dtype=torch.uint8, device=x.device)
    check(lib().amv_quantize_k(wtype, x2.data_ptr(), n, k, y.data_ptr(), _stream()), "amv_quantize_k")
    return y


# ------------------------------------------------------------------------------------------------ BitNet I2_S
def i2s_quantize_act(x: torch.Tensor) -> torch.Tensor:
    """quantize_activation_int8 per row of x f32 [m, k] -> activation buffer (int8 q | {dequant, sum q} per row)."""
    _need_gpu(x, "i2s_quantize_act")
    x2 = x.reshape(-1, x.shape[-1])
    m, k = x2.shape
    act = torch.empty(lib().amv_i2s_act_bytes(m, k), dtype=torch.uint8, device=x.device)
    check(lib().amv_i2s_quantize_act(x2.data_ptr(), m, k, act.data_ptr(), _stream()), "amv_i2s_quantize_act")
    return act


def i2s_gemv(w: torch.Tensor, n_rows: int, k: int, act: torch.Tensor, m: int, weight_scale: float) -> torch.Tensor:
    """bitnet_gemv: [m, n_rows] f32 from the I2_S tensor bytes w (payload first) and i2s_quantize_act output."""
    _need_gpu(w, "i2s_gemv")
    out = torch.empty((m, n_rows), dtype=torch.float32, device=w.device)
    check(lib().amv_i2s_gemv(w.data_ptr(), n_rows, k, act.data_ptr(), m, weight_scale, out.data_ptr(), n_rows,
                             _stream()), "amv_i2s_gemv")
    return out


def i2s_gemv_sums(w: torch.Tensor, n_rows: int, k: int, act: torch.Tensor, m: int) -> torch.Tensor:
    out = torch.empty((m, n_rows), dtype=torch.int32, device=w.device)
    check(lib().amv_i2s_gemv_sums(w.data_ptr(), n_rows, k, act.data_ptr(), m, out.data_ptr(), _stream()),
          "amv_i2s_gemv_sums")
    return out


def i2s_tensor_scale(tensor_bytes: torch.Tensor, n_rows: int, k: int) -> float:
    """The f32 scale trailer right after the n_rows * k/4 byte payload (amuda_gguf.c:659-681); read on the host."""
    off = n_rows * k // 4
    return float(tensor_bytes[off:off + 4].cpu().view(torch.float32)[0])


# ------------------------------------------------------------------------------------ RMS_NORM, ROPE, SWIGLU
def rms_norm(x: torch.Tensor, eps: float, w: torch.Tensor | None = None, quantize: bool = False,
             rule: int = Q8_X86):
    """ggml_rms_norm (+ the fused MUL by w, + the fused Q8_0 quantization of the result).
    Returns y, or (y, o) with w, plus the activation buffer last when quantize=True."""
    _need_gpu(x, "rms_norm")
    x2 = x.reshape(-1, x.shape[-1])
    m, n = x2.shape
    y = torch.empty_like(x2)
    o = torch.empty_like(x2) if w is not None else None
    act = torch.empty(lib().amv_act_bytes(Q8_0, m, n), dtype=torch.uint8, device=x.device) if quantize else None
    check(lib().amv_rms_norm(x2.data_ptr(), m, n, eps, _ptr(w), y.data_ptr(), _ptr(o), _ptr(act), rule, _stream()),
          "amv_rms_norm")
    res = (y,) if o is None else (y, o)
    if quantize:
        res = res + (act,)
    return res[0] if len(res) == 1 else res


def rope(x: torch.Tensor, pos: torch.Tensor, n_dims: int, mode: int = 0, freq_base: float = 10000.0,
         freq_scale: float = 1.0, attn_factor: float = 1.0, out: torch.Tensor | None = None) -> torch.Tensor:
    """ggml_rope_ext (ext_factor 0): x f32 [n_tok, n_head, ne0], pos int32 [n_tok]."""
    _need_gpu(x, "rope")
    n_tok, n_head, ne0 = x.shape
    y = torch.empty_like(x) if out is None else out
    check(lib().amv_rope(x.data_ptr(), y.data_ptr(), pos.data_ptr(), n_tok, n_head, ne0, n_dims, mode, freq_base,
                         freq_scale, attn_factor, _stream()), "amv_rope")
    return y


def rope_kv_store(qkv: torch.Tensor, pos: torch.Tensor, n_head: int, n_head_kv: int, k_cache: torch.Tensor,
                  v_cache: torch.Tensor, kv_idx: torch.Tensor, n_dims: int | None = None, mode: int = 0,
                  freq_base: float = 10000.0, freq_scale: float = 1.0, attn_factor: float = 1.0,
                  bad: torch.Tensor | None = None) -> None:
    """ROPE of the q and k heads of qkv f32 [n_tok, n_head + 2 n_head_kv, D] in place, and the rotated k / the v heads
    stored as f16 at rows kv_idx (int64 [n_tok]) of k_cache / v_cache ([rows, n_head_kv * D] f16)."""
    _need_gpu(qkv, "rope_kv_store")
    n_tok, n_all, D = qkv.shape
    if n_all != n_head + 2 * n_head_kv or kv_idx.dtype != torch.int64 or pos.dtype != torch.int32:
        raise ValueError("rope_kv_store: bad operands")
    if k_cache.dtype != torch.float16 or v_cache.dtype != torch.float16 or k_cache.stride(0) != v_cache.stride(0):
        raise ValueError("rope_kv_store: caches must be f16 with the same row stride")
    check(lib().amv_rope_kv_store(qkv.data_ptr(), pos.data_ptr(), n_tok, n_head, n_head_kv, D,
                                  D if n_dims is None else n_dims, mode, freq_base, freq_scale, attn_factor,
                                  k_cache.data_ptr(), v_cache.data_ptr(), k_cache.stride(0), kv_idx.data_ptr(),
                                  k_cache.shape[0], _ptr(bad), _stream()), "amv_rope_kv_store")


def swiglu(g: torch.Tensor, u: torch.Tensor) -> torch.Tensor:
    _need_gpu(g, "swiglu")
    y = torch.empty_like(g)
    check(lib().amv_swiglu(g.data_ptr(), u.data_ptr(), y.data_ptr(), g.numel(), _stream()), "amv_swiglu")
    return y


def swiglu_rows(g: torch.Tensor, u: torch.Tensor, quantize: bool = False, rule: int = Q8_X86, act_type: int = Q8_0):
    """SWIGLU of row views g, u [n_rows, n] (contiguous rows, any row stride). Returns y, or (y, act) with the
    activation buffer of y (amv_quantize_act layout, act_type Q8_0 or Q8_K) when quantize."""
    _need_gpu(g, "swiglu_rows", contiguous=False)
    n_rows, n = g.shape
    if g.stride(1) != 1 or u.stride(1) != 1 or u.shape != g.shape:
        raise ValueError("swiglu_rows: g and u must be [n_rows, n] views with contiguous rows")
    y = torch.empty((n_rows, n), dtype=torch.float32, device=g.device)
    act = None
    if quantize:
        act = torch.empty(lib().amv_act_bytes(act_type, n_rows, n), dtype=torch.uint8, device=g.device)
    check(lib().amv_swiglu_rows_act(g.data_ptr(), g.stride(0), u.data_ptr(), u.stride(0), y.data_ptr(), n, n_rows, n,
                                    _ptr(act), act_type, rule, _stream()), "amv_swiglu_rows")
    return (y, act) if quantize else y


# ------------------------------------------------------------------------------------------- FLASH_ATTN_EXT
def flash_attn_decode(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float, n_kv: int | None = None,
                      mask: torch.Tensor | None = None, workspace: torch.Tensor | None = None,
                      act: torch.Tensor | None = None, rule: int = Q8_X86) -> torch.Tensor:
    """q f32 [n_head, D]; k, v f16 views [n_head_kv, n_keys, D] with any strides (a head-major cache, or llama.cpp's
    token-major one as k_cache[:, :n_kv].permute(1, 0, 2)); the first n_kv keys are used; mask f16 [n_kv] or None.
    act: optional buffer (amv_act_bytes(Q8_0, 1, n_head * D)) that also receives the output quantized to Q8_0."""
    _need_gpu(q, "flash_attn_decode")
    n_head, D = q.shape
    n_head_kv, n_keys, _ = k.shape
    n_kv = n_keys if n_kv is None else n_kv
    if k.stride(2) != 1 or v.stride(2) != 1:
        raise ValueError("flash_attn_decode: K/V rows must be contiguous")
    need = lib().amv_flash_attn_workspace_bytes(n_head, n_head_kv, n_kv, D)
    if need < 0:
        raise ValueError("flash_attn_decode: unsupported shape")
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    out = torch.empty_like(q)
    check(lib().amv_flash_attn_decode(q.data_ptr(), k.data_ptr(), v.data_ptr(), _ptr(mask), out.data_ptr(), n_head,
                                      n_head_kv, n_kv, D, k.stride(1), k.stride(0), v.stride(1), v.stride(0), scale,
                                      workspace.data_ptr(), need, _ptr(act), rule, _stream()), "amv_flash_attn_decode")
    return out


def flash_attn_decode_ex(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float, n_kv_max: int,
                         n_kv_dev: torch.Tensor | None = None, mask: torch.Tensor | None = None,
                         act: torch.Tensor | None = None, act_t: int = Q8_0, rule: int = Q8_X86,
                         counters: torch.Tensor | None = None, one_launch: bool = False,
                         workspace: torch.Tensor | None = None) -> torch.Tensor:
    """flash_attn_decode with the key count read from n_kv_dev (int32 [1] on the device) when given, capped at
    n_kv_max. act: optional activation row of type act_t (Q8_0 or Q8_K) that also receives the output. one_launch:
    the split merge runs in the split launch's last workgroups, on counters (int32 [>= 32 n_head_kv] zeros,
    allocated when None)."""
    _need_gpu(q, "flash_attn_decode_ex")
    n_head, D = q.shape
    n_head_kv = k.shape[0]
    if k.stride(2) != 1 or v.stride(2) != 1:
        raise ValueError("flash_attn_decode_ex: K/V rows must be contiguous")
    need = lib().amv_flash_attn_workspace_bytes(n_head, n_head_kv, n_kv_max, D)
    if need < 0:
        raise ValueError("flash_attn_decode_ex: unsupported shape")
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    if one_launch and counters is None:
        counters = torch.zeros(32 * n_head_kv, dtype=torch.int32, device=q.device)
    out = torch.empty_like(q)
    check(lib().amv_flash_attn_decode_ex(q.data_ptr(), k.data_ptr(), v.data_ptr(), _ptr(mask), out.data_ptr(),
                                         n_head, n_head_kv, n_kv_max, _ptr(n_kv_dev), D, k.stride(1), k.stride(0),
                                         v.stride(1), v.stride(0), scale, workspace.data_ptr(), need,
                                         _ptr(counters if one_launch else None), _ptr(act), act_t, rule, _stream()),
          "amv_flash_attn_decode_ex")
    return out


def flash_attn_decode_kv(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, kv_type: int, scale: float,
                         n_kv_max: int | None = None, n_kv_dev: torch.Tensor | None = None,
                         mask: torch.Tensor | None = None, act: torch.Tensor | None = None, act_t: int = Q8_0,
                         rule: int = Q8_X86, one_launch: bool = False,
                         workspace: torch.Tensor | None = None) -> torch.Tensor:
    """FLASH_ATTN_EXT decode over an F16 (kv_type 1), Q8_0 (8) or Q4_0 (2) cache: k, v [n_head_kv, n_keys, row] views
    (f16 elements, or the bytes of ggml blocks for the quantized types; any strides). A quantized K meets q quantized to
    Q8_0 with `rule` (ggml's CPU kernel); otherwise as flash_attn_decode_ex."""
    _need_gpu(q, "flash_attn_decode_kv")
    n_head, D = q.shape
    n_head_kv, n_keys = k.shape[0], k.shape[1]
    n_kv_max = n_keys if n_kv_max is None else n_kv_max
    if k.stride(2) != 1 or v.stride(2) != 1:
        raise ValueError("flash_attn_decode_kv: K/V rows must be contiguous")
    need = lib().amv_flash_attn_workspace_bytes(n_head, n_head_kv, n_kv_max, D)
    if need < 0:
        raise ValueError("flash_attn_decode_kv: unsupported shape")
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
    counters = torch.zeros(32 * n_head_kv, dtype=torch.int32, device=q.device) if one_launch else None
    ke, ve = k.element_size(), v.element_size()
    out = torch.empty_like(q)
    check(lib().amv_flash_attn_decode_kv(kv_type, q.data_ptr(), k.data_ptr(), v.data_ptr(), _ptr(mask),
                                         out.data_ptr(), n_head, n_head_kv, n_kv_max, _ptr(n_kv_dev), D,
                                         k.stride(1) * ke, k.stride(0) * ke, v.stride(1) * ve, v.stride(0) * ve, scale,
                                         workspace.data_ptr(), need, _ptr(counters), _ptr(act), act_t, rule,
                                         _stream()), "amv_flash_attn_decode_kv")
    return out


def flash_attn_prefill(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float, n_kv: int | None = None,
                       mask: torch.Tensor | None = None, causal_pos0: int = -1) -> torch.Tensor:
    """q f32 [n_tok, n_head, D] (any strides with contiguous rows); k, v f16 views [n_head_kv, n_keys, D] as in
    flash_attn_decode; mask f16 [n_tok, >= n_kv] or None; causal_pos0 >= 0: token t sees keys <= causal_pos0 + t.
    Returns f32 [n_tok, n_head, D]."""
    _need_gpu(q, "flash_attn_prefill", contiguous=False)
    n_tok, n_head, D = q.shape
    n_head_kv, n_keys, _ = k.shape
    n_kv = n_keys if n_kv is None else n_kv
    if q.stride(2) != 1 or k.stride(2) != 1 or v.stride(2) != 1:
        raise ValueError("flash_attn_prefill: q, K and V rows must be contiguous")
    if mask is not None and (mask.dtype != torch.float16 or mask.stride(1) != 1 or mask.shape[0] < n_tok):
        raise ValueError("flash_attn_prefill: mask must be f16 [n_tok, n_kv] with contiguous rows")
    out = torch.empty((n_tok, n_head, D), dtype=torch.float32, device=q.device)
    check(lib().amv_flash_attn_prefill(q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), v.data_ptr(), _ptr(mask),
                                       0 if mask is None else mask.stride(0), out.data_ptr(), n_tok, n_head,
                                       n_head_kv, n_kv, D, k.stride(1), k.stride(0), v.stride(1), v.stride(0), scale,
                                       causal_pos0, _stream()), "amv_flash_attn_prefill")
    return out


# ------------------------------------------------------------------------------------------------ glue ops
def add(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    """ggml_add with b broadcast over rows (b rows divide a rows)."""
    return _binary(0, a, b)


def mul(a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    return _binary(1, a, b)


def _binary(op: int, a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
    _need_gpu(a, "binary")
    _need_gpu(b, "binary")
    n = a.shape[-1]
    out = torch.empty_like(a)
    check(lib().amv_binary(op, a.data_ptr(), b.data_ptr(), out.data_ptr(), a.numel() // n, n, b.numel() // n,
                           _stream()), "amv_binary")
    return out


def set_rows_f16(dst: torch.Tensor, src: torch.Tensor, idx: torch.Tensor | None = None) -> None:
    """Rows of src f32 [r, n] into rows idx (int32/int64 [r]) of dst f16 [rows, n]; raises on out-of-range indices."""
    _need_gpu(src, "set_rows_f16")
    bad = torch.zeros(1, dtype=torch.int32, device=src.device)
    r, n = src.shape
    bits = 0 if idx is None else (64 if idx.dtype == torch.int64 else 32)
    check(lib().amv_set_rows_f16(src.data_ptr(), src.stride(0), dst.data_ptr(), dst.stride(0), r, n, _ptr(idx), bits,
                                 dst.shape[0], bad.data_ptr(), _stream()), "amv_set_rows_f16")
    if int(bad.item()) != 0:
        raise IndexError(f"set_rows_f16: {int(bad.item())} row indices out of range (FAIL-FAST)")


def set_rows_q(dst: torch.Tensor, src: torch.Tensor, dst_type: int, idx: torch.Tensor | None = None,
               rule: int = Q8_X86) -> None:
    """Rows of src f32 [r, n] quantized (Q8_0 with `rule`, or Q4_0) into rows idx of dst (uint8 [rows, >= row bytes],
    any row stride); raises on out-of-range indices."""
    _need_gpu(src, "set_rows_q")
    bad = torch.zeros(1, dtype=torch.int32, device=src.device)
    r, n = src.shape
    bits = 0 if idx is None else (64 if idx.dtype == torch.int64 else 32)
    check(lib().amv_set_rows_q(dst_type, src.data_ptr(), src.stride(0), dst.data_ptr(),
                               dst.stride(0) * dst.element_size(), r, n, _ptr(idx), bits, dst.shape[0], rule,
                               bad.data_ptr(), _stream()), "amv_set_rows_q")
    if int(bad.item()) != 0:
        raise IndexError(f"set_rows_q: {int(bad.item())} row indices out of range (FAIL-FAST)")


def get_rows(src: torch.Tensor, src_type: int, n: int, idx: torch.Tensor) -> torch.Tensor:
    """ggml_get_rows: f32 [len(idx), n] from rows of src (F32 = 0, F16 = 1, Q4_0, Q8_0, Q4_K, Q6_K in ggml layout)."""
    _need_gpu(idx, "get_rows")
    rb = 4 * n if src_type == 0 else 2 * n if src_type == 1 else ggml_row_bytes(src_type, n)
    rows = src.numel() * src.element_size() // rb
    out = torch.empty((idx.numel(), n), dtype=torch.float32, device=idx.device)
    bad = torch.zeros(1, dtype=torch.int32, device=idx.device)
    check(lib().amv_get_rows(src_type, src.data_ptr(), rows, n, idx.data_ptr(), idx.numel(), out.data_ptr(),
                             bad.data_ptr(), _stream()), "amv_get_rows")
    if int(bad.item()) != 0:
        raise IndexError("get_rows: row index out of range (FAIL-FAST)")
    return out


def argmax(x: torch.Tensor, token: torch.Tensor | None = None, history: torch.Tensor | None = None,
           step: torch.Tensor | None = None) -> torch.Tensor:
    """Greedy sampling on the device: token int32 [1] = first index of the maximum of x (f32, contiguous); with
    history (int32 [L]) and step (int32 [1]) also history[step] = token, step += 1."""
    _need_gpu(x, "argmax")
    if token is None:
        token = torch.empty(1, dtype=torch.int32, device=x.device)
    check(lib().amv_argmax(x.data_ptr(), x.numel(), token.data_ptr(), _ptr(history), _ptr(step),
                           0 if history is None else history.numel(), _stream()), "amv_argmax")
    return token
