"""One Llama-3-architecture decoder layer on quantized weights, as the sequence of hot-path kernels a ggml decode
graph of that layer runs (the reference's graph engine records the same nodes:
RMS_NORM+MUL, MUL_MAT q/k/v, ROPE, SET_ROWS into the KV cache, FLASH_ATTN_EXT, MUL_MAT o, ADD, RMS_NORM+MUL,
MUL_MAT gate/up, SWIGLU, MUL_MAT down, ADD).

MI355X-specific choices: q/k/v and gate/up are each one weight of stacked rows (one GEMV launch instead of three /
two; the rows are independent, so the outputs equal the separate MUL_MATs). The fused decode step is 8 launches:
the GEMVs carry the small ops after them (ROPE + KV stores; ADD; SWIGLU + the activation quantization), the norms
and the attention merge quantize their outputs for the next GEMV. Every buffer is allocated up front and the
position and key count live in device memory, so a decode step launches kernels only and a captured HIP graph
replays at any position.
"""
from __future__ import annotations

import torch

from . import ops
from ._lib import check, lib


class LlamaLayer:
    def __init__(self, wq: ops.QWeight, wo: ops.QWeight, wgu: ops.QWeight, wdown: ops.QWeight,
                 attn_norm: torch.Tensor, ffn_norm: torch.Tensor, n_head: int = 32, n_head_kv: int = 8,
                 head_dim: int = 128, ctx: int = 4096, eps: float = 1e-5, rope_base: float = 500000.0):
        dev = attn_norm.device
        self.wqkv, self.wo, self.wgu, self.wdown = wq, wo, wgu, wdown
        self.attn_norm, self.ffn_norm = attn_norm, ffn_norm
        self.n_head, self.n_head_kv, self.D, self.ctx = n_head, n_head_kv, head_dim, ctx
        self.eps, self.base = eps, rope_base
        self.H = n_head * head_dim
        self.kv = n_head_kv * head_dim
        self.FF = wgu.n_rows // 2
        assert wq.n_rows == self.H + 2 * self.kv and wq.k == self.H
        assert wdown.k == self.FF and wdown.n_rows == self.H and wo.n_rows == self.H
        # llama.cpp's cache layout: rows [token][n_head_kv * head_dim]
        self.k_cache = torch.zeros((ctx, self.kv), dtype=torch.float16, device=dev)
        self.v_cache = torch.zeros((ctx, self.kv), dtype=torch.float16, device=dev)
        f32 = dict(dtype=torch.float32, device=dev)
        self.t_norm = torch.empty(self.H, **f32)
        self.t_o = torch.empty(self.H, **f32)      # attention-norm output (y * w)
        self.t_o2 = torch.empty(self.H, **f32)     # FFN-norm output
        self.qkv = torch.empty(wq.n_rows, **f32)
        self.att = torch.empty(self.H, **f32)
        self.proj = torch.empty(self.H, **f32)
        self.x1 = torch.empty(self.H, **f32)
        self.gu = torch.empty(wgu.n_rows, **f32)
        self.h = torch.empty(self.FF, **f32)
        self.down = torch.empty(self.H, **f32)
        u8 = dict(dtype=torch.uint8, device=dev)
        L = lib()
        # activations of the GEMV inputs: Q8_0 for Q4_0 / Q8_0 weights, Q8_K for the K-quants
        self.atype = ops.act_type(wq.type)
        self.act_h = torch.empty(L.amv_act_bytes(self.atype, 1, self.H), **u8)
        self.act_att = torch.empty(L.amv_act_bytes(self.atype, 1, self.H), **u8)
        self.act_h2 = torch.empty(L.amv_act_bytes(self.atype, 1, self.H), **u8)
        self.act_ff = torch.empty(L.amv_act_bytes(self.atype, 1, self.FF), **u8)
        self.fa_ws = torch.empty(L.amv_flash_attn_workspace_bytes(n_head, n_head_kv, ctx, head_dim), **u8)
        self.pos = torch.zeros(1, dtype=torch.int32, device=dev)
        self.kv_idx = torch.zeros(1, dtype=torch.int64, device=dev)
        self.n_kv_dev = torch.ones(1, dtype=torch.int32, device=dev)
        self.n_kv = 1
        # arrival counters of the gate/up launch's quantization (self-resetting)
        self.cnt = torch.zeros(ops.swiglu_counter_words(wgu.n_rows), dtype=torch.int32, device=dev)
        # Q4_0 / Q4_K weights at H = 4096: the fused step folds both RMS_NORMs into the GEMV after them
        # (amv_rms_norm_gemv_rope_kv / amv_rms_norm_gemv_swiglu_q8, the same bytes as the norm launch)
        self.fold_norm = (wq.type in (ops.Q4_0, ops.Q4_K) and wgu.type == wq.type and self.H == 4096
                          and self.FF % (256 if wq.type == ops.Q4_K else 32) == 0)
        # measured on the 32-layer Q4_K model: the FFN fold of Q4_K costs more than its norm launch (1688 against
        # 1677 us per token with the attention fold alone), so Q4_K folds the attention norm only
        self.fold_attn = self.fold_norm
        self.fold_ffn = self.fold_norm and wq.type == ops.Q4_0

    @staticmethod
    def stack_rows(*blocks: torch.Tensor) -> torch.Tensor:
        """Rows of several ggml-layout weights with the same k, stacked (ggml blocks are whole rows)."""
        return torch.cat([b.reshape(b.shape[0], -1) for b in blocks], dim=0).contiguous()

    def set_position(self, pos: int) -> None:
        """Position of the next decode step, written into device memory (a captured graph picks it up)."""
        self.pos.fill_(pos)
        self.kv_idx.fill_(pos)
        self.n_kv_dev.fill_(pos + 1)
        self.n_kv = pos + 1

    def _quant(self, x_ptr: int, n: int, act: torch.Tensor, st) -> None:
        check(lib().amv_quantize_act(self.atype, x_ptr, 1, n, ops.Q8_X86, None, act.data_ptr(), st), "quantize")

    def decode(self, x: torch.Tensor, out: torch.Tensor, fused: bool = True, act_ready: bool = False,
               next_layer: "LlamaLayer | None" = None) -> None:
        """x f32 [H] -> out f32 [H] for the token at the position of set_position(); writes K/V into the cache.

        fused=True, 8 launches: RMS_NORM + MUL + quantization of x (skipped with act_ready: the previous layer put it
        in self.act_h); q/k/v GEMV + ROPE + KV stores; FA split; FA merge + quantization (key count from device
        memory); o GEMV + ADD; FFN RMS_NORM + MUL + quantization; gate/up GEMV + SWIGLU + quantization; down GEMV +
        ADD, then next_layer's attention RMS_NORM + quantization into next_layer.act_h when given (call
        next_layer.decode with act_ready=True). With fold_attn / fold_ffn (Q4_0 at H = 4096: both, 6 launches; Q4_K: the
        attention norm, 7) an RMS_NORM is computed inside the GEMV after it, per workgroup while its weights stream in
        (act_h / t_o or act_h2 / t_o2 are then not written, act_ready is ignored and next_layer gets no norm launch
        when it folds its own). Merged into the GEMV
        before them (amv_gemv_add_rms_norm) the norms ran slower on MI355X.
        fused=False: one launch per graph node (16 for Q4_0; the K-quant types quantize in separate launches and take
        19), the key count from the host. Both give identical results."""
        L, st = lib(), torch.cuda.current_stream().cuda_stream
        H, kv, D, FF, at = self.H, self.kv, self.D, self.FF, self.atype
        q8 = at == ops.Q8_0
        P = lambda t: t.data_ptr()  # noqa: E731
        if fused:
            if self.fold_attn:
                check(L.amv_rms_norm_gemv_rope_kv(P(x), P(self.attn_norm), self.eps, ops.Q8_X86, self.wqkv.type,
                                                  P(self.wqkv.data), self.wqkv.n_rows, H, P(self.qkv), self.n_head,
                                                  self.n_head_kv, D, P(self.pos), self.base, 1.0, 1.0,
                                                  P(self.k_cache), P(self.v_cache), kv, P(self.kv_idx), self.ctx,
                                                  None, st), "rms_norm + qkv + rope + kv store")
            else:
                if not act_ready:
                    check(L.amv_rms_norm_act(P(x), 1, H, self.eps, P(self.attn_norm), None, P(self.t_o),
                                             P(self.act_h), at, ops.Q8_X86, st), "rms_norm")
                check(L.amv_gemv_rope_kv(self.wqkv.type, P(self.wqkv.data), self.wqkv.n_rows, H, P(self.act_h),
                                         P(self.qkv), self.n_head, self.n_head_kv, D, P(self.pos), self.base, 1.0,
                                         1.0, P(self.k_cache), P(self.v_cache), kv, P(self.kv_idx), self.ctx, None,
                                         st), "qkv + rope + kv store")
            cnt = P(self.cnt)
            check(L.amv_flash_attn_decode_ex(P(self.qkv), P(self.k_cache), P(self.v_cache), None, P(self.att),
                                             self.n_head, self.n_head_kv, self.ctx, P(self.n_kv_dev), D, kv, D, kv, D,
                                             1.0 / (D ** 0.5), P(self.fa_ws), self.fa_ws.numel(), None,
                                             P(self.act_att), at, ops.Q8_X86, st),
                  "flash_attn (split, merge + quantization)")
            check(L.amv_mul_mat_vec_ep(self.wo.type, P(self.wo.data), H, H, P(self.act_att), None, ops.EP_ADD, P(x),
                                       P(self.x1), st), "wo + residual")
            if self.fold_ffn:
                check(L.amv_rms_norm_gemv_swiglu_q8(P(self.x1), P(self.ffn_norm), self.eps, ops.Q8_X86, self.wgu.type,
                                                    P(self.wgu.data), self.wgu.n_rows, H, None, P(self.h),
                                                    P(self.act_ff), cnt, st), "ffn norm + gate_up + swiglu + quant")
            else:
                check(L.amv_rms_norm_act(P(self.x1), 1, H, self.eps, P(self.ffn_norm), None, P(self.t_o2),
                                         P(self.act_h2), at, ops.Q8_X86, st), "ffn norm")
                check(L.amv_gemv_swiglu_q8(self.wgu.type, P(self.wgu.data), self.wgu.n_rows, H, P(self.act_h2), None,
                                           P(self.h), P(self.act_ff), at, ops.Q8_X86, cnt, st),
                      "gate_up + swiglu + quantization")
            check(L.amv_mul_mat_vec_ep(self.wdown.type, P(self.wdown.data), H, FF, P(self.act_ff), None,
                                       ops.EP_ADD, P(self.x1), P(out), st), "down + residual")
            if next_layer is not None and not next_layer.fold_attn:
                nl = next_layer
                check(L.amv_rms_norm_act(P(out), 1, H, nl.eps, P(nl.attn_norm), None, P(nl.t_o), P(nl.act_h),
                                         nl.atype, ops.Q8_X86, st), "next attention norm")
            return
        # unfused: one launch per node
        check(L.amv_rms_norm(P(x), 1, H, self.eps, P(self.attn_norm), P(self.t_norm), P(self.t_o),
                             P(self.act_h) if q8 else None, ops.Q8_X86, st), "rms_norm")
        if not q8:
            self._quant(P(self.t_o), H, self.act_h, st)
        check(L.amv_mul_mat_vec(self.wqkv.type, P(self.wqkv.data), self.wqkv.n_rows, H, P(self.act_h), 1,
                                P(self.qkv), self.wqkv.n_rows, st), "qkv")
        # RoPE of q and k: 40 contiguous heads of the qkv output, in place
        check(L.amv_rope(P(self.qkv), P(self.qkv), P(self.pos), 1, self.n_head + self.n_head_kv, D, D, 0, self.base,
                         1.0, 1.0, st), "rope")
        kp = P(self.qkv) + H * 4
        vp = kp + kv * 4
        check(L.amv_set_rows_f16(kp, kv, P(self.k_cache), kv, 1, kv, P(self.kv_idx), 64, self.ctx, None, st),
              "set_rows k")
        check(L.amv_set_rows_f16(vp, kv, P(self.v_cache), kv, 1, kv, P(self.kv_idx), 64, self.ctx, None, st),
              "set_rows v")
        ws = self.fa_ws.numel()
        check(L.amv_flash_attn_decode(P(self.qkv), P(self.k_cache), P(self.v_cache), None, P(self.att), self.n_head,
                                      self.n_head_kv, self.n_kv, D, kv, D, kv, D, 1.0 / (D ** 0.5), P(self.fa_ws), ws,
                                      P(self.act_att) if q8 else None, ops.Q8_X86, st), "flash_attn")
        if not q8:
            self._quant(P(self.att), H, self.act_att, st)
        check(L.amv_mul_mat_vec(self.wo.type, P(self.wo.data), H, H, P(self.act_att), 1, P(self.proj), H, st), "wo")
        check(L.amv_binary(0, P(self.proj), P(x), P(self.x1), 1, H, 1, st), "residual 1")
        check(L.amv_rms_norm(P(self.x1), 1, H, self.eps, P(self.ffn_norm), P(self.t_norm), P(self.t_o2),
                             P(self.act_h2) if q8 else None, ops.Q8_X86, st), "ffn norm")
        if not q8:
            self._quant(P(self.t_o2), H, self.act_h2, st)
        check(L.amv_mul_mat_vec(self.wgu.type, P(self.wgu.data), self.wgu.n_rows, H, P(self.act_h2), 1, P(self.gu),
                                self.wgu.n_rows, st), "gate_up")
        check(L.amv_swiglu(P(self.gu), P(self.gu) + FF * 4, P(self.h), FF, st), "swiglu")
        self._quant(P(self.h), FF, self.act_ff, st)
        check(L.amv_mul_mat_vec(self.wdown.type, P(self.wdown.data), H, FF, P(self.act_ff), 1, P(self.down), H, st),
              "down")
        check(L.amv_binary(0, P(self.down), P(self.x1), P(out), 1, H, 1, st), "residual 2")

    def _prefill_buffers(self, n_tok: int) -> dict:
        """Per-token-count buffers of prefill (allocated on first use; a captured graph must see them allocated)."""
        bufs = getattr(self, "_pf", None)
        if bufs is not None and bufs["n"] >= n_tok and bufs["at"] == ops.act_type(self.wqkv.type, n_tok):
            return bufs
        dev = self.attn_norm.device
        f32 = dict(dtype=torch.float32, device=dev)
        u8 = dict(dtype=torch.uint8, device=dev)
        L = lib()
        H, FF = self.H, self.FF
        at = ops.act_type(self.wqkv.type, n_tok)
        bufs = {"n": n_tok, "at": at,
                "t_o": torch.empty((n_tok, H), **f32), "qkv": torch.empty((n_tok, self.wqkv.n_rows), **f32),
                "att": torch.empty((n_tok, H), **f32),
                "x1": torch.empty((n_tok, H), **f32), "t_o2": torch.empty((n_tok, H), **f32),
                "gu": torch.empty((n_tok, self.wgu.n_rows), **f32),
                "act_h": torch.empty(L.amv_act_bytes(at, n_tok, H), **u8),
                "act_att": torch.empty(L.amv_act_bytes(at, n_tok, H), **u8),
                "act_h2": torch.empty(L.amv_act_bytes(at, n_tok, H), **u8),
                "act_ff": torch.empty(L.amv_act_bytes(at, n_tok, FF), **u8),
                "h": torch.empty((n_tok, FF), **f32) if at not in (ops.Q8_0, ops.Q8_K) else None,
                "pos": torch.zeros(n_tok, dtype=torch.int32, device=dev),
                "idx": torch.zeros(n_tok, dtype=torch.int64, device=dev)}
        self._pf = bufs
        return bufs

    def set_prefill_position(self, pos0: int, n_tok: int) -> None:
        """Positions pos0 .. pos0 + n_tok - 1 for the next prefill (device memory, so a captured graph picks them up)."""
        b = self._prefill_buffers(n_tok)
        r = torch.arange(pos0, pos0 + n_tok, device=self.attn_norm.device)
        b["pos"][:n_tok].copy_(r.to(torch.int32))
        b["idx"][:n_tok].copy_(r)
        self.pf_pos0, self.pf_n = pos0, n_tok

    def prefill(self, x: torch.Tensor, out: torch.Tensor) -> None:
        """A prompt chunk through the layer: x f32 [n_tok, H] at positions set_prefill_position(pos0, n_tok) ->
        out f32 [n_tok, H]; writes the chunk's K/V rows into the cache and attends causally over keys
        0 .. pos0 + t. The MUL_MATs run on the int8 MFMA kernel (n_tok >= 8, the reference's crossover) and the
        attention on the f16 MFMA prefill kernel; the residual ADDs in the epilogues of the o and down GEMMs:
        10 launches (13 where the activation layout is an extended one, whose quantization is a launch of its own)."""
        L, st = lib(), torch.cuda.current_stream().cuda_stream
        n, pos0 = self.pf_n, self.pf_pos0
        b = self._prefill_buffers(n)
        H, kv, D, FF = self.H, self.kv, self.D, self.FF
        P = lambda t: t.data_ptr()  # noqa: E731
        at = b["at"]
        if n >= ops.MMQ_MIN_M and self.wqkv.type in ops.MMQ_TYPES:
            def mm(wt, w, nr, k, act, m, dst, ldd, s):
                return L.amv_mul_mat_q_act(wt, w, nr, k, act, at, m, dst, ldd, s)

            def mm_add(wt, w, nr, k, act, m, dst, ldd, add, what):  # the residual ADD in the GEMM's epilogue
                check(L.amv_mul_mat_q_act_add(wt, w, nr, k, act, at, m, dst, ldd, add, st), what)
        else:
            mm = L.amv_mul_mat_vec

            def mm_add(wt, w, nr, k, act, m, dst, ldd, add, what):
                check(mm(wt, w, nr, k, act, m, dst, ldd, st), what)
                check(L.amv_binary(0, dst, add, dst, m, nr, m, st), what + " residual")
        q8 = at in (ops.Q8_0, ops.Q8_K)  # plain layouts: the norms and SWIGLU write them directly

        def quant(src, k, act):
            check(L.amv_quantize_act(at, src, n, k, ops.Q8_X86, None, P(act), st), "quantize")

        check(L.amv_rms_norm_act(P(x), n, H, self.eps, P(self.attn_norm), None, None if q8 else P(b["t_o"]),
                                 P(b["act_h"]) if q8 else None, at, ops.Q8_X86, st), "rms_norm")
        if not q8:
            quant(P(b["t_o"]), H, b["act_h"])
        nq = self.wqkv.n_rows
        check(mm(self.wqkv.type, P(self.wqkv.data), nq, H, P(b["act_h"]), n, P(b["qkv"]), nq, st), "qkv")
        check(L.amv_rope_kv_store(P(b["qkv"]), P(b["pos"]), n, self.n_head, self.n_head_kv, D, D, 0, self.base, 1.0,
                                  1.0, P(self.k_cache), P(self.v_cache), kv, P(b["idx"]), self.ctx, None, st),
              "rope + kv store")
        check(L.amv_flash_attn_prefill(P(b["qkv"]), nq, D, P(self.k_cache), P(self.v_cache), None, 0, P(b["att"]), n,
                                       self.n_head, self.n_head_kv, pos0 + n, D, kv, D, kv, D, 1.0 / (D ** 0.5), pos0,
                                       st), "flash_attn prefill")
        quant(P(b["att"]), H, b["act_att"])
        mm_add(self.wo.type, P(self.wo.data), H, H, P(b["act_att"]), n, P(b["x1"]), H, P(x), "wo + residual")
        check(L.amv_rms_norm_act(P(b["x1"]), n, H, self.eps, P(self.ffn_norm), None, None if q8 else P(b["t_o2"]),
                                 P(b["act_h2"]) if q8 else None, at, ops.Q8_X86, st), "ffn norm")
        if not q8:
            quant(P(b["t_o2"]), H, b["act_h2"])
        ng = self.wgu.n_rows
        check(mm(self.wgu.type, P(self.wgu.data), ng, H, P(b["act_h2"]), n, P(b["gu"]), ng, st), "gate_up")
        if q8:
            check(L.amv_swiglu_rows_act(P(b["gu"]), ng, P(b["gu"]) + FF * 4, ng, None, FF, n, FF, P(b["act_ff"]),
                                        at, ops.Q8_X86, st), "swiglu + quant")
        else:
            check(L.amv_swiglu_rows(P(b["gu"]), ng, P(b["gu"]) + FF * 4, ng, P(b["h"]), FF, n, FF, None, ops.Q8_X86,
                                    st), "swiglu")
            quant(P(b["h"]), FF, b["act_ff"])
        mm_add(self.wdown.type, P(self.wdown.data), H, FF, P(b["act_ff"]), n, P(out), H, P(b["x1"]), "down + residual")

    def prefill_ops(self, n_tok: int, n_kv: int) -> int:
        """Multiply-adds x 2 of one prefill chunk: the four weight products and the attention (causal half)."""
        w = sum(q.n_rows * q.k for q in (self.wqkv, self.wo, self.wgu, self.wdown))
        att = 4 * self.n_head * self.D * (n_tok * n_kv - n_tok * (n_tok - 1) // 2)
        return 2 * n_tok * w + att

    # algorithmic HBM bytes of one decode step at n_kv cached keys (weights + KV read + norms)
    def step_bytes(self, n_kv: int) -> int:
        w = sum(q.nbytes for q in (self.wqkv, self.wo, self.wgu, self.wdown))
        return w + 2 * n_kv * self.kv * 2 + 2 * self.H * 4


def random_layer(dev, seed: int = 0, H: int = 4096, n_head: int = 32, n_head_kv: int = 8, D: int = 128,
                 FF: int = 14336, ctx: int = 4096, wtype: int = ops.Q4_0) -> LlamaLayer:
    """A layer with seeded N(0, 0.02) weights quantized on the GPU (Q4_0 rule), norm weights 1 + N(0, 0.1)^."""
    g = torch.Generator(device=dev)
    g.manual_seed(seed)

    def q(n, k):
        wf = torch.randn((n, k), generator=g, device=dev) * 0.02
        b = ops.quantize_q4_0(wf) if wtype == ops.Q4_0 else ops.quantize_k(wf, wtype)
        del wf
        return b

    kv = n_head_kv * D
    wqkv = ops.QWeight.from_ggml(wtype, LlamaLayer.stack_rows(q(H, H), q(kv, H), q(kv, H)), H + 2 * kv, H)
    wo = ops.QWeight.from_ggml(wtype, q(H, H), H, H)
    wgu = ops.QWeight.from_ggml(wtype, LlamaLayer.stack_rows(q(FF, H), q(FF, H)), 2 * FF, H)
    wdown = ops.QWeight.from_ggml(wtype, q(H, FF), H, FF)
    an = 1 + 0.1 * torch.randn(H, generator=g, device=dev)
    fn = 1 + 0.1 * torch.randn(H, generator=g, device=dev)
    return LlamaLayer(wqkv, wo, wgu, wdown, an, fn, n_head, n_head_kv, D, ctx)
