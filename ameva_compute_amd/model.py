"""A Llama-3-architecture decoder stack on quantized weights (32 Q4_K layers, a Q6_K output head
of 128256 rows), run as the graph the reference's backend executes for llama.cpp: GET_ROWS of the token embedding,
the layers (ameva_compute_amd.llama.LlamaLayer), RMS_NORM + MUL of the last hidden state, the head MUL_MAT, and the
greedy sampler's argmax.

MI355X-specific choices: the prompt runs through every layer as one chunk (the int8 / f16 matrix-core GEMMs and the
f16-MFMA causal attention), the layers share one set of prompt buffers; a decode step is one HIP graph (about 8
launches per layer) whose token, position, cache row and key count live in device memory, so the graph is captured
once and replayed for every generated token without a host round trip: the argmax writes the next token where the
embedding lookup reads it and appends it to a device-side history, and the step ends by advancing the position.
"""
from __future__ import annotations

import torch

from . import ops
from ._lib import check, lib
from .llama import LlamaLayer, random_layer


class LlamaModel:
    def __init__(self, tok_embd: torch.Tensor, embd_type: int, layers: list[LlamaLayer], output_norm: torch.Tensor,
                 head: ops.QWeight, max_new: int = 1024):
        """tok_embd: ggml-layout rows [vocab, row bytes] of embd_type; head: the output MUL_MAT weight [vocab, H]."""
        dev = output_norm.device
        self.tok_embd, self.embd_type = tok_embd, embd_type
        self.layers, self.output_norm, self.head = layers, output_norm, head
        self.H, self.vocab = layers[0].H, head.n_rows
        self.ctx = layers[0].ctx
        self.eps = layers[0].eps
        assert head.k == self.H and tok_embd.shape[0] == self.vocab
        # one position / cache row / key count for all layers (device memory, advanced inside the decode graph)
        self.pos = torch.zeros(1, dtype=torch.int32, device=dev)
        self.kv_idx = torch.zeros(1, dtype=torch.int64, device=dev)
        self.n_kv_dev = torch.ones(1, dtype=torch.int32, device=dev)
        for lay in layers:
            lay.pos, lay.kv_idx, lay.n_kv_dev = self.pos, self.kv_idx, self.n_kv_dev
        f32 = dict(dtype=torch.float32, device=dev)
        self.x = [torch.empty(self.H, **f32) for _ in range(2)]
        self.t_out = torch.empty(self.H, **f32)
        self.hatype = ops.act_type(head.type)
        self.act_head = torch.empty(lib().amv_act_bytes(self.hatype, 1, self.H), dtype=torch.uint8, device=dev)
        self.logits = torch.empty(self.vocab, **f32)
        self.token = torch.zeros(1, dtype=torch.int32, device=dev)
        self.history = torch.zeros(max_new, dtype=torch.int32, device=dev)
        self.step = torch.zeros(1, dtype=torch.int32, device=dev)
        self.argmax_ws = torch.zeros(2, dtype=torch.int64, device=dev)  # amv_argmax_ex's 16 bytes, left zero
        self._pf = None

    # ---------------------------------------------------------------------------------------------- helpers
    def _embed(self, idx: torch.Tensor, out: torch.Tensor, n: int, st) -> None:
        check(lib().amv_get_rows(self.embd_type, self.tok_embd.data_ptr(), self.vocab, self.H, idx.data_ptr(), n,
                                 out.data_ptr(), None, st), "get_rows (token embedding)")

    def _head(self, x_last: torch.Tensor, st, advance: bool = False) -> None:
        """RMS_NORM + MUL of the last hidden state, the head MUL_MAT, the argmax into token / history / step; with
        advance, the same launch moves the decode position (pos, cache row, key count) on by one."""
        L = lib()
        check(L.amv_rms_norm_act(x_last.data_ptr(), 1, self.H, self.eps, self.output_norm.data_ptr(), None,
                                 self.t_out.data_ptr(), self.act_head.data_ptr(), self.hatype, ops.Q8_X86, st),
              "output norm")
        check(L.amv_mul_mat_vec(self.head.type, self.head.data.data_ptr(), self.vocab, self.H,
                                self.act_head.data_ptr(), 1, self.logits.data_ptr(), self.vocab, st), "output head")
        adv = (self.pos.data_ptr(), self.kv_idx.data_ptr(), self.n_kv_dev.data_ptr()) if advance else (None,) * 3
        check(L.amv_argmax_ex(self.logits.data_ptr(), self.vocab, self.token.data_ptr(), self.history.data_ptr(),
                              self.step.data_ptr(), self.history.numel(), *adv, self.argmax_ws.data_ptr(), st),
              "argmax")

    def set_position(self, pos: int) -> None:
        self.pos.fill_(pos)
        self.kv_idx.fill_(pos)
        self.n_kv_dev.fill_(pos + 1)
        for lay in self.layers:
            lay.n_kv = pos + 1

    def reset(self) -> None:
        self.step.zero_()
        self.history.zero_()

    # ---------------------------------------------------------------------------------------------- prompt
    def prefill(self, tokens: torch.Tensor) -> None:
        """The prompt (int32 [n] on the device, n <= ctx) through all layers at positions 0 .. n - 1; samples the
        first new token (token, history[step]) and sets the decode position to n."""
        n = tokens.numel()
        st = torch.cuda.current_stream().cuda_stream
        if self._pf is None or self._pf[0].shape[0] < n:
            f32 = dict(dtype=torch.float32, device=tokens.device)
            self._pf = (torch.empty((n, self.H), **f32), torch.empty((n, self.H), **f32))
            shared = None
            for lay in self.layers:  # one set of prompt buffers for all layers
                if shared is None:
                    shared = lay._prefill_buffers(n)
                lay._pf = shared
        a, b = self._pf[0][:n], self._pf[1][:n]
        self._embed(tokens, a, n, st)
        self.layers[0].set_prefill_position(0, n)  # shared position buffers
        for lay in self.layers:
            lay.pf_pos0, lay.pf_n = 0, n
            lay.prefill(a, b)
            a, b = b, a
        self._head(a[n - 1], st)

    def prefill_ops(self, n: int) -> int:
        """Multiply-adds x 2 of a prompt of n tokens: the layers and the head on the last token."""
        return sum(lay.prefill_ops(n, n) for lay in self.layers) + 2 * self.vocab * self.H

    # ---------------------------------------------------------------------------------------------- decode
    def decode_step(self, fused: bool = True) -> None:
        """One generated token: embeds `token` (the previous sample), runs the layers at the current position,
        samples the next token into token / history[step] and advances the position (in the argmax launch). Launches
        only, on the current stream, so it can be captured once and replayed."""
        st = torch.cuda.current_stream().cuda_stream
        x, y = self.x
        self._embed(self.token, x, 1, st)
        nl = len(self.layers)
        for i, lay in enumerate(self.layers):
            nxt = self.layers[i + 1] if fused and i + 1 < nl else None
            lay.decode(x, y, fused=fused, act_ready=fused and i > 0, next_layer=nxt)
            x, y = y, x
        self._head(x, st, advance=True)

    def decode_bytes(self, n_kv: int) -> int:
        """Algorithmic HBM bytes of one decode step at n_kv cached keys: every weight once, the KV rows, the
        embedding row and the logits."""
        return (sum(lay.step_bytes(n_kv) for lay in self.layers) + self.head.nbytes
                + ops.ggml_row_bytes(self.embd_type, self.H) + 4 * self.vocab)


def random_model(dev, n_layers: int = 32, H: int = 4096, n_head: int = 32, n_head_kv: int = 8, D: int = 128,
                 FF: int = 14336, vocab: int = 128256, ctx: int = 1024, seed: int = 0, wtype: int = ops.Q4_K,
                 head_type: int = ops.Q6_K, embd_type: int = ops.Q4_K, max_new: int = 1024) -> LlamaModel:
    """Seeded random weights of the architecture (N(0, 0.02) quantized on the GPU with this library's Q4_K / Q6_K
    rule; norm weights 1 + N(0, 0.1)): there is no checkpoint to load."""
    g = torch.Generator(device=dev)
    g.manual_seed(seed)

    def table(rows: int, t: int) -> torch.Tensor:
        out = torch.empty((rows, ops.ggml_row_bytes(t, H)), dtype=torch.uint8, device=dev)
        chunk = 16384
        for r0 in range(0, rows, chunk):
            r1 = min(rows, r0 + chunk)
            wf = torch.randn((r1 - r0, H), generator=g, device=dev) * 0.02
            out[r0:r1] = (ops.quantize_q4_0(wf) if t == ops.Q4_0 else ops.quantize_k(wf, t)).reshape(r1 - r0, -1)
            del wf
        return out

    emb = table(vocab, embd_type)
    head = ops.QWeight.from_ggml(head_type, table(vocab, head_type), vocab, H)
    layers = [random_layer(dev, seed=seed * 1000 + 1 + i, H=H, n_head=n_head, n_head_kv=n_head_kv, D=D, FF=FF,
                           ctx=ctx, wtype=wtype) for i in range(n_layers)]
    on = 1 + 0.1 * torch.randn(H, generator=g, device=dev)
    return LlamaModel(emb, embd_type, layers, on, head, max_new=max_new)
