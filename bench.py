"""Benchmark of the quantized ggml hot path on one MI355X.

Headline (BASELINE.json metric "Q4_0 GEMV GB/s (% HBM peak) + bs1 decode tok/s, Llama-8B-shape layer"):
  one step = one Q4_0 x Q8_0 decode GEMV (MUL_MAT, M = 1) at the Llama-3-8B FFN gate/up shape 14336 x 4096, weights
  N(0, 0.02) quantized on the GPU with ggml's Q4_0 rule, activation N(0, 1) quantized to Q8_0 (x86 rule) once.
  The weights rotate over COPIES distinct copies (> 512 MiB in total, twice the 256 MiB Infinity Cache), so every
  step streams its weight from HBM ("cold"); a "hot" figure (one copy, cache-resident) is reported beside it.
  value = algorithmic bytes per GEMV (weights + Q8_0 activation + f32 output) / time per step.
Timing: W untimed warm-up steps, then K steps bracketed by torch.cuda.synchronize() and HIP events on the stream the
kernels run on. The CPU baseline times the oracle's multithreaded C restatement of ggml's vec_dot_q4_0_q8_0 on the
host cores over a bounded sample of the same GEMV.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
N_ROWS, K = 14336, 4096
COPIES = 20          # 20 x 33 MB = 661 MB of distinct weights, > 2 x the 256 MiB Infinity Cache
GRAPH_STEPS = 100    # steps captured in one HIP graph


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def gemv_bytes(n: int, k: int, wtype_bytes_per_block: int = 18) -> int:
    # weights + Q8_0 activation (34 B per 32) + f32 output
    return n * (k // 32) * wtype_bytes_per_block + (k // 32) * 34 + n * 4


def make_weights(ops, torch, n, k, copies, seed, dev, wtype):
    g = torch.Generator(device=dev)
    ws = []
    for c in range(copies):
        g.manual_seed(seed + c)
        wf = torch.randn((n, k), generator=g, device=dev, dtype=torch.float32) * 0.02
        if wtype == ops.Q4_0:
            wg = ops.quantize_q4_0(wf)
        elif wtype in (ops.Q4_K, ops.Q6_K):
            wg = ops.quantize_k(wf, wtype)
        else:
            act, wg = ops.quantize_act(wf, ops.Q8_0, ops.Q8_REF, ggml=True)
            del act
        ws.append(ops.QWeight.from_ggml(wtype, wg, n, k))
        del wf, wg
    torch.cuda.synchronize()
    return ws


def time_steps(torch, fn, steps, warmup):
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    e0.record()
    for i in range(steps):
        fn(i)
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps  # ms per step


def time_steps_graph(torch, fn, steps, warmup, per_graph=GRAPH_STEPS, info=None, min_reps=1, median=False):
    """fn(i) for i in 0..per_graph-1 captured once in a HIP graph; the graph is replayed so that K >= steps steps
    (and at least min_reps replays) run back to back with no host launch cost between kernels. Returns ms per step:
    the mean over all replays, or with median=True the median of the replays, each timed by its own pair of events
    on the replay stream. info (a dict), when given, receives the step counts that actually ran: 'timed' (replays x
    per_graph), 'warmup' (the eager pass before the capture plus the untimed replays) and 'replays'."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for i in range(per_graph):
            fn(i)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for i in range(per_graph):
            fn(i)
    reps = max(min_reps, (steps + per_graph - 1) // per_graph)
    wreps = max(1, warmup // per_graph)
    if info is not None:
        info["timed"] = reps * per_graph
        info["warmup"] = (1 + wreps) * per_graph
        info["replays"] = reps
    if median:
        for _ in range(wreps):
            graph.replay()
        torch.cuda.synchronize()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(reps + 1)]
        ev[0].record()
        for r in range(reps):
            graph.replay()
            ev[r + 1].record()
        torch.cuda.synchronize()
        per = sorted(ev[r].elapsed_time(ev[r + 1]) for r in range(reps))
        ms = per[reps // 2] if reps % 2 else 0.5 * (per[reps // 2 - 1] + per[reps // 2])
    else:
        ms = time_steps(torch, lambda i: graph.replay(), reps, wreps)
    del graph
    return ms / per_graph


def _cpu_q4_0_weights(rng, n, k):
    """Random Q4_0 blocks (random nibbles, d = 0.01) of an n x k weight: the CPU baseline's timing does not depend on
    the values, and random bytes avoid quantizing a 900 MB f32 matrix on the host."""
    import numpy as np
    w = np.frombuffer(rng.bytes(n * (k // 32) * 18), np.uint8).reshape(n, k // 32, 18).copy()
    w[:, :, 0:2] = np.frombuffer(np.float16(0.01).tobytes(), np.uint8)
    return w.reshape(n, -1)


def _timed(fn, seconds, min_runs=3):
    import time as _t
    fn()  # warm-up
    n, t0 = 0, _t.perf_counter()
    while True:
        fn()
        n += 1
        el = _t.perf_counter() - t0
        if el >= seconds and n >= min_runs:
            return el / n, n, el


def cpu_layer_decode(oracle, rng, seconds):
    """One bs1 decode step of the Llama-3-8B Q4_0 layer at 4096 cached keys on the host cores: the GEMVs and the
    attention on the AVX2 baseline kernels (oracle/cpu_simd.c), the O(4096)-element steps (RMS norm, Q8_0
    quantization, RoPE, SwiGLU) on the oracle's C. Returns (s per token, steps, seconds)."""
    import numpy as np
    H, F, NH, NKV, D, CTX = 4096, 14336, 32, 8, 128, 4096
    wqkv = _cpu_q4_0_weights(rng, (NH + 2 * NKV) * D, H)
    wo = _cpu_q4_0_weights(rng, H, NH * D)
    wgu = _cpu_q4_0_weights(rng, 2 * F, H)
    wd = _cpu_q4_0_weights(rng, H, F)
    kc = rng.standard_normal((CTX, NKV, D)).astype(np.float16)
    vc = rng.standard_normal((CTX, NKV, D)).astype(np.float16)
    nw = np.ones(H, np.float32)
    x0 = rng.standard_normal(H).astype(np.float32)
    pos = np.array([CTX - 1], np.int32)

    def step():
        y, o = oracle.rms_norm(x0[None, :], 1e-5, nw)
        a = oracle.quantize_q8_0(o, oracle.Q8_X86)
        qkv = oracle.simd_mul_mat_q4_0(wqkv, wqkv.shape[0], H, a, 1)[0]
        q = oracle.rope(qkv[:NH * D].reshape(1, NH, D), pos, D)
        k = oracle.rope(qkv[NH * D:(NH + NKV) * D].reshape(1, NKV, D), pos, D)
        kc[CTX - 1] = k[0].astype(np.float16)
        vc[CTX - 1] = qkv[(NH + NKV) * D:].reshape(NKV, D).astype(np.float16)
        att = oracle.simd_flash_attn_decode(q[0], kc, vc, 1.0 / np.sqrt(D))
        x1 = x0 + oracle.simd_mul_mat_q4_0(wo, H, NH * D, oracle.quantize_q8_0(att.reshape(1, -1), oracle.Q8_X86), 1)[0]
        y, o = oracle.rms_norm(x1[None, :], 1e-5, nw)
        gu = oracle.simd_mul_mat_q4_0(wgu, 2 * F, H, oracle.quantize_q8_0(o, oracle.Q8_X86), 1)[0]
        h = oracle.swiglu(gu[:F], gu[F:])
        return x1 + oracle.simd_mul_mat_q4_0(wd, H, F, oracle.quantize_q8_0(h[None, :], oracle.Q8_X86), 1)[0]

    return _timed(step, seconds)


CPU_COPIES = 12


def cpu_baseline(seconds: float = 10.0):
    """The headline GEMV on the host cores (plus, beside it, the M = 512 GEMM and the layer decode step): ggml's AVX2
    vec_dot_q4_0_q8_0 algorithm (oracle/cpu_simd.c, OpenMP) where the CPU has AVX2 / FMA / F16C, else the oracle's
    scalar C. Each figure is timed for a bounded sample (about `seconds` of CPU work for the GEMV, a third of it for
    each of the other two)."""
    import numpy as np
    import oracle
    rng = np.random.default_rng(1234)
    simd = oracle.cpu_simd() is not None
    x = rng.standard_normal((1, K)).astype(np.float32)
    aq = oracle.quantize_q8_0(x, oracle.Q8_X86)
    if simd:
        # cold like the GPU figure: CPU_COPIES rotating weight copies (~400 MB, beyond the host's L3)
        wqs = [_cpu_q4_0_weights(rng, N_ROWS, K) for _ in range(CPU_COPIES)]
        wq = wqs[0]
        out = np.empty((1, N_ROWS), np.float32)
        turn = [0]

        def gemv_cold():
            oracle.simd_mul_mat_q4_0(wqs[turn[0] % CPU_COPIES], N_ROWS, K, aq, 1, out)
            turn[0] += 1
        per, n, el = _timed(gemv_cold, seconds)
        threads = oracle.cpu_simd().cpu_num_threads()
        how = (f"ggml's AVX2 vec_dot_q4_0_q8_0 algorithm (oracle/cpu_simd.c, OpenMP), cold: {CPU_COPIES} rotating "
               f"weight copies ({CPU_COPIES * N_ROWS * K * 18 // 32 / 1e6:.0f} MB, beyond the host's L3)")
    else:
        w = (rng.standard_normal((N_ROWS, K)) * 0.02).astype(np.float32)
        wq = oracle.quantize_q4_0(w)
        del w
        per, n, el = _timed(lambda: oracle.mul_mat(oracle.Q4_0, wq, N_ROWS, K, aq, 1), seconds)
        threads = oracle.num_threads()
        how = "oracle vec_dot_q4_0_q8_0 (scalar C, OpenMP; this CPU lacks AVX2 / FMA / F16C)"
    res = {
        "value": round(gemv_bytes(N_ROWS, K) / per / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{n} Q4_0 GEMVs 14336x4096 (M=1) in {el:.1f} s, {how}, {per * 1e3:.3f} ms each; "
                  f"host CPU: {cpu_model()}",
    }
    if simd:
        rows, m = 1792, 512  # a row slice of the 14336 x 4096 GEMM at 512 tokens
        a5 = oracle.quantize_q8_0(rng.standard_normal((m, K)).astype(np.float32), oracle.Q8_X86)
        w5 = np.ascontiguousarray(wq[:rows])
        o5 = np.empty((m, rows), np.float32)
        per5, n5, el5 = _timed(lambda: oracle.simd_mul_mat_q4_0(w5, rows, K, a5, m, o5), seconds / 3)
        res["gemm_m512_gops"] = round(2.0 * rows * K * m / per5 / 1e9, 1)
        res["gemm_sample"] = (f"{n5} Q4_0 x Q8_0 GEMMs of {rows} of the 14336 rows x 4096 x 512 tokens in {el5:.1f} s "
                              f"({per5 * 1e3:.1f} ms each; the full 14336-row GEMM scales by 8)")
        del wq, wqs, w5, a5, o5
        perl, nl, ell = cpu_layer_decode(oracle, rng, seconds / 3)
        res["layer_decode_tok_s"] = round(1.0 / perl, 2)
        res["layer_decode_sample"] = (f"{nl} bs1 decode steps of one Llama-3-8B Q4_0 layer at 4096 cached keys in "
                                      f"{ell:.1f} s ({perl * 1e3:.2f} ms each): GEMVs and attention on "
                                      f"oracle/cpu_simd.c, norms / quantization / RoPE / SwiGLU on the oracle's C")
    return res


def bench_layer(torch, dev, args):
    """bs1 decode of a Llama-3-8B-shape layer at position 4095 (4096 cached keys): LAYERS
    different random layers chained (cold weights: 4 x 140 MB), the chain captured once in a HIP graph and replayed.
    Reported per layer; tok/s = 1 / (time of one layer)."""
    from ameva_compute_amd.llama import random_layer
    layers_n = 4
    layers = [random_layer(dev, seed=100 + i) for i in range(layers_n)]
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    for lay in layers:
        lay.k_cache.copy_(torch.randn(lay.k_cache.shape, generator=g, device=dev).half())
        lay.v_cache.copy_(torch.randn(lay.v_cache.shape, generator=g, device=dev).half())
        lay.set_position(lay.ctx - 1)
    xs = [torch.randn(4096, generator=g, device=dev)] + [torch.empty(4096, device=dev) for _ in range(layers_n)]

    def chain(fused=True):
        # fused: 6 launches per layer, each RMS_NORM folded into the GEMV after it (Q4_0 at H = 4096)
        for i, lay in enumerate(layers):
            nxt = layers[i + 1] if fused and i + 1 < layers_n else None
            lay.decode(xs[i], xs[i + 1], fused=fused, act_ready=fused and i > 0, next_layer=nxt)

    def graph_ms(fused):
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            chain(fused)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            chain(fused)
        t = time_steps(torch, lambda i: graph.replay(), 200, 20) / layers_n
        del graph
        return t

    ms_eager = time_steps(torch, lambda i: chain(), 50, 5) / layers_n
    ms_unfused = graph_ms(False)
    ms = graph_ms(True)
    nbytes = layers[0].step_bytes(layers[0].ctx)
    gbs = nbytes / (ms * 1e-3) / 1e9
    pf = bench_prefill(torch, dev, layers[0], 512)
    log(f"bench: layer decode {ms * 1e3:.2f} us/layer (graph, 6 launches), {ms_unfused * 1e3:.2f} us "
        f"unfused (16 launches), {ms_eager * 1e3:.2f} us eager; {nbytes / 1e6:.1f} MB -> {gbs:.0f} GB/s")
    del layers
    torch.cuda.empty_cache()
    return {"layer_decode_us": round(ms * 1e3, 3), "layer_decode_tok_s": round(1e3 / ms, 1),
            "layer_decode_gbs": round(gbs, 1), "layer_decode_eager_us": round(ms_eager * 1e3, 3),
            "layer_decode_unfused_us": round(ms_unfused * 1e3, 3), **pf,
            "layer_decode_bytes": nbytes,
            "layer_decode_note": "Llama-3-8B layer, Q4_0, bs1, 4096 cached keys, 4 chained cold layers in one HIP graph"}


def bench_plugin_layer(torch, dev, layers=4):
    """bs1 decode of Llama-3-8B-shape Q4_0 layers at 4096 cached keys through the drop-in boundary: the ggml graph
    llama.cpp builds per layer (RMS_NORM, MUL, q/k/v MUL_MATs, ROPE, SET_ROWS into the f16 cache, FLASH_ATTN_EXT,
    o MUL_MAT + ADD, RMS_NORM, MUL, gate/up MUL_MATs, SWIGLU, down MUL_MAT + ADD), `layers` of them chained in one
    graph (each with its own weights and KV cache: 4 x 140 MB, more than the 256 MB Infinity Cache, so the weights
    stream from HBM as in a whole model), handed to libggml-ameva.so's graph_compute, which runs it on its stream and
    returns after the stream completes (as the reference's ggml_backend_graph_compute does,
    adapters/llama/ameva_backend_bench.cpp:38-79). The ggml host side is the stand-in the plugin tests use
    (tests/ggml_plugin.py: ggml's structs and the buffer calls the plugin binds to). Weights: random Q4_0 blocks
    (d = 0.01). Reported: wall time of one graph_compute call, and that time per layer."""
    import ctypes
    import numpy as np
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    import ggml_plugin as gp
    rng = np.random.default_rng(2024)
    H, NH, NKV, D, FF, CTX = 4096, 32, 8, 128, 14336, 4096
    pos_t = CTX - 1

    def wq4(n, k):
        w = np.frombuffer(rng.bytes(n * (k // 32) * 18), np.uint8).reshape(n, k // 32, 18).copy()
        w[:, :, 0:2] = np.frombuffer(np.float16(0.01).tobytes(), np.uint8)
        return w.reshape(n, -1)
    shapes = {"q": (NH * D, H), "k": (NKV * D, H), "v": (NKV * D, H), "o": (H, NH * D), "gate": (FF, H),
              "up": (FF, H), "down": (H, FF)}
    wbytes = sum(n * (k // 32) * 18 for n, k in shapes.values())
    g = gp.Graph(layers * (wbytes + 16 * 4096), (64 << 20) + layers * (32 << 20))
    try:
        X = g.tensor(gp.F32, [H, 1], "c", "inp")
        g.set(X, rng.standard_normal((1, H)).astype(np.float32))
        POS = g.tensor(gp.I32, [1], "c", "pos")
        g.set(POS, np.array([pos_t], np.int32))
        IDX = g.tensor(gp.I64, [1], "c", "kv_idx")
        g.set(IDX, np.array([pos_t], np.int64))
        MASK = g.tensor(gp.F16, [CTX, 1], "c", "mask")
        g.set(MASK, np.zeros(CTX, np.float16))
        x = X
        for _ in range(layers):
            T = {}
            for k_, (n, k) in shapes.items():
                T[k_] = g.tensor(gp.Q4_0, [k, n], "w", k_)
                g.set(T[k_], wq4(n, k))
            AN, FN = g.tensor(gp.F32, [H], "w", "attn_norm"), g.tensor(gp.F32, [H], "w", "ffn_norm")
            g.set(AN, (1 + 0.1 * rng.standard_normal(H)).astype(np.float32))
            g.set(FN, (1 + 0.1 * rng.standard_normal(H)).astype(np.float32))
            KC = g.tensor(gp.F16, [NKV * D, CTX], "c", "k_cache")
            VC = g.tensor(gp.F16, [NKV * D, CTX], "c", "v_cache")
            g.set(KC, rng.standard_normal((CTX, NKV * D)).astype(np.float16))
            g.set(VC, rng.standard_normal((CTX, NKV * D)).astype(np.float16))
            cur = g.mul(g.rms_norm(x, 1e-5), AN)
            q = g.rope(g.reshape_3d(g.mul_mat(T["q"], cur), D, NH, 1), POS, D, 0, 500000.0)
            k = g.rope(g.reshape_3d(g.mul_mat(T["k"], cur), D, NKV, 1), POS, D, 0, 500000.0)
            v = g.mul_mat(T["v"], cur)
            g.set_rows(KC, g.view_nd(k, gp.OP_RESHAPE, [NKV * D, 1], [4, NKV * D * 4, NKV * D * 4, NKV * D * 4]),
                       IDX)
            g.set_rows(VC, v, IDX)
            kv_nb = [2, NKV * D * 2, D * 2, NKV * D * 2 * CTX]
            att = g.flash_attn_ext(g.view_nd(q, gp.OP_PERMUTE, [D, 1, NH], [4, D * NH * 4, D * 4, D * NH * 4]),
                                   g.view_nd(KC, gp.OP_VIEW, [D, CTX, NKV], kv_nb),
                                   g.view_nd(VC, gp.OP_VIEW, [D, CTX, NKV], kv_nb), MASK, 1.0 / np.sqrt(D))
            ffn_inp = g.add(g.mul_mat(T["o"], g.view_nd(att, gp.OP_RESHAPE, [H, 1], [4, H * 4, H * 4, H * 4])), x)
            cur = g.mul(g.rms_norm(ffn_inp, 1e-5), FN)
            ff = g.swiglu(g.mul_mat(T["gate"], cur), g.mul_mat(T["up"], cur))
            x = g.add(g.mul_mat(T["down"], ff), ffn_inp)
        for _ in range(5):  # the first call repacks the weights in place, the second captures the HIP graph
            assert g.compute() == gp.STATUS_SUCCESS
        g.plugin.ggml_backend_ameva_reset_counters()
        # the cgraph of the last call, handed over again as a host would (no Python rebuilding per call)
        compute, be, cg = g.backend.iface.graph_compute, g.backend_ptr, ctypes.addressof(g._keep[1])
        n = 200
        t0 = time.perf_counter()
        for _ in range(n):
            compute(be, cg)
        el = (time.perf_counter() - t0) / n
        nodes = len(g.nodes)
        fused = gp.counter(g.plugin, "fused_pair_count") // n
    finally:
        g.free()
    per = el / layers
    log(f"bench: plugin decode, {layers} layers in one graph_compute ({nodes} ggml nodes, {fused} fused) "
        f"{el * 1e6:.2f} us/call = {per * 1e6:.2f} us/layer")
    return {"plugin_layer_decode_us": round(per * 1e6, 2), "plugin_layer_decode_tok_s": round(1.0 / per, 1),
            "plugin_graph_compute_us": round(el * 1e6, 2), "plugin_graph_layers": layers,
            "plugin_graph_nodes": nodes, "plugin_graph_fused_nodes": fused,
            "plugin_layer_decode_note": f"{layers} chained Llama-3-8B Q4_0 layers (cold weights) in one ggml graph, "
                                        "bs1, 4096 cached keys, through libggml-ameva.so graph_compute (synchronous "
                                        "per call; the unchanged graph replays its HIP-graph capture); per layer = "
                                        "call time / layers"}


BLOCK_BYTES = {2: 18, 8: 34, 12: 144 * 32 // 256, 14: 210 * 32 // 256}  # bytes per 32 weights


def cold_gemv_us(ops, torch, dev, wtype, n, k, seed, steps=1000):
    """Time of one cold GEMV of wtype n x k (M = 1): enough distinct copies to exceed 512 MiB, rotated."""
    per = n * k // 32 * BLOCK_BYTES[wtype]
    copies = max(4, -(-(600 << 20) // per))
    ws = make_weights(ops, torch, n, k, copies, seed, dev, wtype)
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    x = torch.randn((1, k), generator=g, device=dev, dtype=torch.float32)
    act, _ = ops.quantize_act(x, ops.act_type(wtype), ops.Q8_X86)
    out = torch.empty((1, n), dtype=torch.float32, device=dev)
    ms = time_steps_graph(torch, lambda i: ops.mul_mat_q(ws[i % copies], act, 1, out), steps, steps // 10)
    del ws
    torch.cuda.empty_cache()
    return ms * 1e3, per + (k // 32) * 34 + n * 4


def secondary_gemvs(ops, torch, dev):
    """Cold M = 1 GEMVs of BASELINE configs 1 and 2 (Q4_0 4096 x 4096, the down shape, Q8_0 / Q4_K FFN shapes)."""
    res = {}
    for name, wtype, n, k in (("q4_0_4096x4096", ops.Q4_0, 4096, 4096), ("q4_0_4096x14336", ops.Q4_0, 4096, 14336),
                              ("q8_0_14336x4096", ops.Q8_0, 14336, 4096), ("q4_K_14336x4096", ops.Q4_K, 14336, 4096),
                              ("q4_K_4096x14336", ops.Q4_K, 4096, 14336)):
        us, nb = cold_gemv_us(ops, torch, dev, wtype, n, k, 99 + n + k)
        res[name + "_cold_gbs"] = round(nb / us / 1e3, 1)
        res[name + "_cold_us"] = round(us, 3)
        log(f"bench: {name} cold {us:.2f} us = {nb / us / 1e3:.0f} GB/s")
    return res


def bench_batched(ops, torch, dev):
    """Q4_0 / Q8_0 / Q4_K MUL_MAT at the Llama-3-8B FFN shapes with token batches 16 and 512, and
    Q6_K (ffn_down / attn_v of Q4_K_M files): the exact form (exact per-block integers on the int8 matrix cores, the
    default) and, at 512 tokens, the scaled f16 form (AMEVA_MMQ_FORM=scaled; not for Q6_K); 2 M N K ops per call."""
    res = {}
    g = torch.Generator(device=dev)
    for wname, wtype in (("q4_0", ops.Q4_0), ("q8_0", ops.Q8_0), ("q4_K", ops.Q4_K), ("q6_K", ops.Q6_K)):
        for n, k in ((14336, 4096), (4096, 14336)):
            w = make_weights(ops, torch, n, k, 1, 300 + n, dev, wtype)[0]
            forms = ((16, True), (512, True)) + (((512, False),) if wtype != ops.Q6_K else ())
            for m, exact in forms:
                g.manual_seed(m + n)
                x = torch.randn((m, k), generator=g, device=dev)
                at = ops.act_type(wtype, m, exact=exact)
                act, _ = ops.quantize_act(x, at, ops.Q8_X86)
                out = torch.empty((m, n), dtype=torch.float32, device=dev)
                ms = time_steps_graph(torch, lambda i: ops.mul_mat_q(w, act, m, out, act_t=at),
                                      50 if m == 512 else 200, 10, per_graph=10)
                tops = 2.0 * m * n * k / (ms * 1e-3) / 1e12
                key = f"{wname}_{n}x{k}_m{m}" + ("" if exact else "_scaled")
                res[key + "_us"] = round(ms * 1e3, 2)
                res[key + "_tops"] = round(tops, 1)
                log(f"bench: {key} {ms * 1e3:.1f} us = {tops:.1f} TOPS ({tops / INT8_MFMA_PEAK_TOPS * 100:.1f}% of "
                    f"int8 MFMA peak)")
            del w
            torch.cuda.empty_cache()
    return res


def bench_i2s(ops, torch, dev):
    """BitNet I2_S GEMV, batch 1, cold over 120 copies of each 4.4 MB weight."""
    res = {}
    g = torch.Generator(device=dev)
    for n, k in ((2560, 6912), (6912, 2560)):
        copies = 120
        ws = []
        for c in range(copies):
            g.manual_seed(500 + c)
            codes = torch.randint(0, 3, (n, k), generator=g, device=dev, dtype=torch.int32)
            # 128-weight blocks of 32 bytes: byte i holds the codes of weights i, 32 + i, 64 + i, 96 + i
            cb = codes.reshape(n, k // 128, 4, 32)
            packed = (cb[:, :, 0] << 6) | (cb[:, :, 1] << 4) | (cb[:, :, 2] << 2) | cb[:, :, 3]
            ws.append(packed.to(torch.uint8).reshape(n, k // 4).contiguous())
            del codes, cb, packed
        x = torch.randn((1, k), generator=g, device=dev)
        act = ops.i2s_quantize_act(x)
        out = torch.empty((1, n), dtype=torch.float32, device=dev)
        from ameva_compute_amd._lib import lib as _lib

        def step(i):
            _lib().amv_i2s_gemv(ws[i % copies].data_ptr(), n, k, act.data_ptr(), 1, 1.5, out.data_ptr(), n,
                                torch.cuda.current_stream().cuda_stream)
        ms = time_steps_graph(torch, step, 2000, 200)
        nbytes = n * k // 4 + k + n * 4
        res[f"i2s_{n}x{k}_b1_cold_gbs"] = round(nbytes / (ms * 1e-3) / 1e9, 1)
        res[f"i2s_{n}x{k}_b1_cold_us"] = round(ms * 1e3, 3)
        log(f"bench: I2_S {n}x{k} b1 cold {ms * 1e3:.2f} us = {nbytes / (ms * 1e-3) / 1e9:.0f} GB/s")
        # batch 128 (int8 MFMA): 2 n k 128 integer ops
        x128 = torch.randn((128, k), generator=g, device=dev)
        act128 = ops.i2s_quantize_act(x128)
        out128 = torch.empty((128, n), dtype=torch.float32, device=dev)

        def step128(i):
            _lib().amv_i2s_gemv(ws[i % copies].data_ptr(), n, k, act128.data_ptr(), 128, 1.5, out128.data_ptr(), n,
                                torch.cuda.current_stream().cuda_stream)
        ms128 = time_steps_graph(torch, step128, 1000, 100)
        tops = 2.0 * n * k * 128 / (ms128 * 1e-3) / 1e12
        res[f"i2s_{n}x{k}_b128_us"] = round(ms128 * 1e3, 3)
        res[f"i2s_{n}x{k}_b128_tops"] = round(tops, 1)
        res[f"i2s_{n}x{k}_b128_frac_int8_peak"] = round(tops / INT8_MFMA_PEAK_TOPS, 4)
        log(f"bench: I2_S {n}x{k} b128 {ms128 * 1e3:.2f} us = {tops:.0f} TOPS ({tops / INT8_MFMA_PEAK_TOPS * 100:.1f}% "
            f"of int8 MFMA peak)")
        del ws
        torch.cuda.empty_cache()
    return res


def bench_kv_cache(ops, torch, dev):
    """FLASH_ATTN_EXT decode at the Llama-3-8B layer shape (32 / 8 heads of 128, 4096 cached keys) over an F16, Q8_0
    and Q4_0 KV cache in llama.cpp's layout (token rows of all KV heads), cold: the caches rotate over copies totalling
    > 512 MiB. Algorithmic bytes: K + V rows read once."""
    res = {}
    NH, NKV, D, CTX = 32, 8, 128, 4096
    g = torch.Generator(device=dev)
    g.manual_seed(4096)
    q = torch.randn((NH, D), generator=g, device=dev)
    for name, t in (("f16", ops.F16), ("q8_0", ops.Q8_0), ("q4_0", ops.Q4_0)):
        rows = torch.randn((CTX, NKV * D), generator=g, device=dev)
        if t == ops.F16:
            base = [rows.half(), torch.randn((CTX, NKV * D), generator=g, device=dev).half()]
            rb = 2 * D
        else:
            rb = D // 32 * (34 if t == ops.Q8_0 else 18)
            base = []
            for _ in range(2):
                c = torch.empty((CTX, NKV * rb), dtype=torch.uint8, device=dev)
                ops.set_rows_q(c, torch.randn((CTX, NKV * D), generator=g, device=dev), t)
                base.append(c)
        per = 2 * CTX * NKV * rb
        copies = max(4, -(-(600 << 20) // per))
        kv = [(base[0].clone(), base[1].clone()) for _ in range(copies)]
        views = [(k.view(CTX, NKV, -1).permute(1, 0, 2), v.view(CTX, NKV, -1).permute(1, 0, 2)) for k, v in kv]
        ws = torch.empty(max(1, ops.lib().amv_flash_attn_workspace_bytes(NH, NKV, CTX, D)), dtype=torch.uint8,
                         device=dev)
        ms = time_steps_graph(torch, lambda i: ops.flash_attn_decode_kv(q, views[i % copies][0], views[i % copies][1],
                                                                       t, 0.0884, workspace=ws), 400, 40)
        res[f"fa_decode_ctx4096_{name}_us"] = round(ms * 1e3, 2)
        res[f"fa_decode_ctx4096_{name}_gbs"] = round(per / (ms * 1e-3) / 1e9, 1)
        log(f"bench: FA decode ctx {CTX} {name} KV cache, cold: {ms * 1e3:.2f} us, {per / 2**20:.1f} MiB K+V -> "
            f"{per / (ms * 1e-3) / 1e9:.0f} GB/s")
        del kv, views, base
        torch.cuda.empty_cache()
    return res


def bench_load_path(ops, torch, dev):
    """The weight load path (the reference's set_tensor repack, ggml-ameva-buffer.cpp:509-561): amv_repack (ggml blocks
    -> the MI355X layout) and amv_unrepack (back, as get_tensor does) of a 14336 x 4096 weight per type, cold over
    rotating sources > 512 MiB (the bytes are shuffled, not interpreted, so random bytes serve), read + write bytes
    counted; the raw-layout GEMV (ggml blocks read in place, amv_mul_mat_vec_raw) against a repack per use; and the
    pinned host -> HBM copy of the same bytes, the step a load cannot avoid."""
    from ameva_compute_amd._lib import lib as _lib
    res = {}
    n, k = 14336, 4096
    g = torch.Generator(device=dev)
    g.manual_seed(77)
    for name, wtype in (("q4_0", ops.Q4_0), ("q8_0", ops.Q8_0), ("q4_K", ops.Q4_K), ("q6_K", ops.Q6_K)):
        nb = _lib().amv_weight_bytes(wtype, n, k)
        copies = max(4, -(-(600 << 20) // nb))
        srcs = [torch.randint(0, 256, (nb,), generator=g, device=dev, dtype=torch.uint8) for _ in range(copies)]
        dst = torch.empty(nb, dtype=torch.uint8, device=dev)
        st = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731
        ms_r = time_steps_graph(torch, lambda i: _lib().amv_repack(wtype, srcs[i % copies].data_ptr(), dst.data_ptr(),
                                                                   n, k, st()), 200, 20, per_graph=copies)
        ms_u = time_steps_graph(torch, lambda i: _lib().amv_unrepack(wtype, srcs[i % copies].data_ptr(),
                                                                     dst.data_ptr(), n, k, st()), 200, 20,
                                per_graph=copies)
        res[f"repack_{name}_14336x4096_us"] = round(ms_r * 1e3, 2)
        res[f"repack_{name}_gbs"] = round(2 * nb / (ms_r * 1e-3) / 1e9, 1)
        res[f"unrepack_{name}_14336x4096_us"] = round(ms_u * 1e3, 2)
        log(f"bench: repack {name} 14336x4096 ({nb / 2**20:.1f} MiB) {ms_r * 1e3:.1f} us = "
            f"{2 * nb / (ms_r * 1e-3) / 1e9:.0f} GB/s read+write; unrepack {ms_u * 1e3:.1f} us")
        del srcs, dst
    # the raw-layout MUL_MAT (a quantized src0 outside a WEIGHTS buffer, M = 1): the GEMV on ggml's blocks in place,
    # against a repack into scratch per use followed by the repacked GEMV; cold over rotating copies of random blocks
    # whose f16 scales are kept finite
    st = lambda: torch.cuda.current_stream().cuda_stream  # noqa: E731
    for name, wtype, blk in (("q4_0", ops.Q4_0, 18), ("q8_0", ops.Q8_0, 34)):
        nb = n * k // 32 * blk
        copies = max(4, -(-(600 << 20) // nb))
        raws = [torch.randint(0, 256, (nb,), generator=g, device=dev, dtype=torch.uint8) for _ in range(copies)]
        for r in raws:
            r.view(n * k // 32, blk)[:, 1] = 0x20
        x = torch.randn((1, k), generator=g, device=dev)
        act, _ = ops.quantize_act(x, ops.Q8_0, ops.Q8_X86)
        y = torch.empty((1, n), dtype=torch.float32, device=dev)
        tmp = torch.empty(nb, dtype=torch.uint8, device=dev)
        ms_raw = time_steps_graph(torch, lambda i: _lib().amv_mul_mat_vec_raw(
            wtype, raws[i % copies].data_ptr(), k // 32 * blk, n, k, act.data_ptr(), 1, y.data_ptr(), n, None, st()),
            1000, 100, min_reps=10, median=True)

        def per_use(i):
            _lib().amv_repack(wtype, raws[i % copies].data_ptr(), tmp.data_ptr(), n, k, st())
            _lib().amv_mul_mat_vec(wtype, tmp.data_ptr(), n, k, act.data_ptr(), 1, y.data_ptr(), n, st())
        ms_pu = time_steps_graph(torch, per_use, 500, 50, min_reps=10, median=True)
        res[f"gemv_raw_{name}_14336x4096_us"] = round(ms_raw * 1e3, 3)
        res[f"gemv_raw_{name}_gbs"] = round(nb / (ms_raw * 1e-3) / 1e9, 1)
        res[f"gemv_repack_per_use_{name}_14336x4096_us"] = round(ms_pu * 1e3, 3)
        log(f"bench: raw-layout GEMV {name} 14336x4096 cold {ms_raw * 1e3:.2f} us = "
            f"{nb / (ms_raw * 1e-3) / 1e9:.0f} GB/s; repack per use + GEMV {ms_pu * 1e3:.2f} us")
        del raws, tmp
    nb = _lib().amv_weight_bytes(ops.Q4_0, n, k)
    host = torch.empty(nb, dtype=torch.uint8, pin_memory=True)
    dst = torch.empty(nb, dtype=torch.uint8, device=dev)
    ms_h = time_steps(torch, lambda i: dst.copy_(host, non_blocking=True), 50, 5)
    res["h2d_pinned_33MB_gbs"] = round(nb / (ms_h * 1e-3) / 1e9, 1)
    log(f"bench: pinned host -> HBM copy of {nb / 2**20:.1f} MiB: {ms_h * 1e3:.0f} us = "
        f"{nb / (ms_h * 1e-3) / 1e9:.1f} GB/s")
    del host, dst
    torch.cuda.empty_cache()
    return res


def copy_ceiling(torch, dev, nbytes):
    """Device-to-device copy of the headline's byte count (torch copy kernel), cold over 20 buffers: the HBM rate a
    single launch of a plain streaming kernel of that size reaches on this box, read + write bytes counted."""
    n = nbytes // 4
    srcs = [torch.randn(n, device=dev) for _ in range(20)]
    dsts = [torch.empty(n, device=dev) for _ in range(20)]
    ms = time_steps_graph(torch, lambda i: dsts[i % 20].copy_(srcs[i % 20]), 1000, 100)
    del srcs, dsts
    torch.cuda.empty_cache()
    return {"d2d_copy_33MB_gbs": round(2 * n * 4 / (ms * 1e-3) / 1e9, 1), "d2d_copy_33MB_us": round(ms * 1e3, 3)}


def pmc_probe(ops, torch, dev):
    """Dispatches for the HBM-traffic counters: the headline GEMV, eager (one dispatch each) over the rotating cold
    weights, the read-only probe of its mapping over the same weights, and torch's copy kernel moving a float32
    tensor of the GEMV's weight byte count, whose FETCH_SIZE and WRITE_SIZE must read that byte count (the scale of
    the counters)."""
    ws = make_weights(ops, torch, N_ROWS, K, COPIES, 42, dev, ops.Q4_0)
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    x = torch.randn((1, K), generator=g, device=dev, dtype=torch.float32)
    act, _ = ops.quantize_act(x, ops.Q8_0, ops.Q8_X86)
    out = torch.empty((1, N_ROWS), dtype=torch.float32, device=dev)
    for i in range(50):
        ops.mul_mat_q(ws[i % COPIES], act, 1, out)
    torch.cuda.synchronize()
    from ameva_compute_amd._lib import check, lib as _lib
    probe_out = torch.empty(N_ROWS, dtype=torch.int32, device=dev)
    for i in range(50):  # the read-only probe of the same mapping (k_gemv_read_probe<true>)
        check(_lib().amv_debug_gemv_read_probe(ws[i % COPIES].data.data_ptr(), N_ROWS, K, probe_out.data_ptr(), 1,
                                               torch.cuda.current_stream().cuda_stream), "read probe")
    torch.cuda.synchronize()
    wbytes = ws[0].nbytes
    del ws
    n = wbytes // 4
    srcs = [torch.randn(n, device=dev) for _ in range(COPIES)]
    dst = torch.empty(n, device=dev)
    torch.cuda.synchronize()
    for i in range(50):
        dst.copy_(srcs[i % COPIES])
    torch.cuda.synchronize()
    print(json.dumps({"gemv_dispatches": 50, "gemv_algorithmic_bytes": gemv_bytes(N_ROWS, K), "probe_dispatches": 50,
                      "copy_dispatches": 50, "copy_bytes_each_way": n * 4}), flush=True)


def pmc_gemm(ops, torch, dev, exact=True):
    """Dispatches for the matrix-core counters: the default (exact, int8 MFMA) batched Q4_K MUL_MAT at M = 512 on the
    Llama-3-8B FFN shapes (14336 x 4096, then 4096 x 14336, whose k is split: its launch is followed by
    k_splitk_sum), 20 eager launches each over one weight, then 20 plain copies of known size (the counters' scale).
    exact=False runs the scaled f16-MFMA form instead (Q8_K_DEQ activations)."""
    res = {}
    g = torch.Generator(device=dev)
    for n, k in ((14336, 4096), (4096, 14336)):
        w = make_weights(ops, torch, n, k, 1, 300 + n, dev, ops.Q4_K)[0]
        g.manual_seed(512 + n)
        x = torch.randn((512, k), generator=g, device=dev)
        at = ops.act_type(ops.Q4_K, 512, exact=exact)
        act, _ = ops.quantize_act(x, at, ops.Q8_X86)
        out = torch.empty((512, n), dtype=torch.float32, device=dev)
        for _ in range(20):
            ops.mul_mat_q(w, act, 512, out, act_t=at)
        torch.cuda.synchronize()
        res[f"q4_K_{n}x{k}_m512"] = {"dispatches": 20, "ops_each": 2 * 512 * n * k}
        del w
    # the scale of FETCH_SIZE / WRITE_SIZE: 20 plain copies of a float32 tensor of the Q4_K weight's byte count
    n_f = 14336 * 4096 // 256 * 144 // 4
    src, dst = torch.randn(n_f, device=dev), torch.empty(n_f, device=dev)
    for _ in range(20):
        dst.copy_(src)
    torch.cuda.synchronize()
    res["copy"] = {"dispatches": 20, "bytes_each_way": n_f * 4}
    print(json.dumps(res), flush=True)


def pmc_small(ops, torch, dev):
    """Dispatches for the counters of the small-batch (M = 16) MUL_MATs on the FFN gate/up shape 14336 x 4096: 20 eager
    launches each for Q4_K and Q6_K over 20 rotating cold weight copies."""
    res = {}
    g = torch.Generator(device=dev)
    for name, wtype in (("q4_K", ops.Q4_K), ("q6_K", ops.Q6_K)):
        ws = make_weights(ops, torch, 14336, 4096, 20, 700 + wtype, dev, wtype)
        g.manual_seed(16 + wtype)
        x = torch.randn((16, 4096), generator=g, device=dev)
        at = ops.act_type(wtype, 16)
        act, _ = ops.quantize_act(x, at, ops.Q8_X86)
        out = torch.empty((16, 14336), dtype=torch.float32, device=dev)
        torch.cuda.synchronize()
        for i in range(20):
            ops.mul_mat_q(ws[i], act, 16, out, act_t=at)
        torch.cuda.synchronize()
        res[f"{name}_14336x4096_m16"] = {"dispatches": 20, "weight_bytes": ws[0].nbytes}
        del ws
        torch.cuda.empty_cache()
    print(json.dumps(res), flush=True)


def pmc_i2s(ops, torch, dev):
    """Dispatches for the counters of the BitNet I2_S batch-128 MUL_MAT (BASELINE config 3 shapes, int8 MFMA): 20
    eager launches on each of 2560 x 6912 and 6912 x 2560 over one random ternary weight, then 20 plain copies of the
    first weight's byte count (the FETCH_SIZE scale)."""
    from ameva_compute_amd._lib import check, lib as _lib
    res = {}
    g = torch.Generator(device=dev)
    for n, k in ((2560, 6912), (6912, 2560)):
        g.manual_seed(500 + n)
        cb = torch.randint(0, 3, (n, k // 128, 4, 32), generator=g, device=dev, dtype=torch.int32)
        w = ((cb[:, :, 0] << 6) | (cb[:, :, 1] << 4) | (cb[:, :, 2] << 2) | cb[:, :, 3]).to(torch.uint8)
        w = w.reshape(n, k // 4).contiguous()
        x = torch.randn((128, k), generator=g, device=dev)
        act = ops.i2s_quantize_act(x)
        out = torch.empty((128, n), dtype=torch.float32, device=dev)
        torch.cuda.synchronize()
        for _ in range(20):
            check(_lib().amv_i2s_gemv(w.data_ptr(), n, k, act.data_ptr(), 128, 1.5, out.data_ptr(), n,
                                      torch.cuda.current_stream().cuda_stream), "amv_i2s_gemv")
        torch.cuda.synchronize()
        res[f"i2s_{n}x{k}_b128"] = {"dispatches": 20, "ops_each": 2 * 128 * n * k, "weight_bytes": n * k // 4,
                                    "act_bytes": 128 * k + 128 * 4}
    n_f = 2560 * 6912 // 4 // 4
    src, dst = torch.randn(n_f, device=dev), torch.empty(n_f, device=dev)
    for _ in range(20):
        dst.copy_(src)
    torch.cuda.synchronize()
    res["copy"] = {"dispatches": 20, "bytes_each_way": n_f * 4}
    print(json.dumps(res), flush=True)


def pmc_fa(ops, torch, dev):
    """Dispatches for the counters of FLASH_ATTN_EXT decode at the Llama-3-8B layer shape (32 / 8 heads of 128, 4096
    cached keys, F16 cache in llama.cpp's layout): 20 eager split + merge launches, each over its own cold copy of
    the K and V rows (20 x 16.8 MB)."""
    NH, NKV, D, CTX = 32, 8, 128, 4096
    g = torch.Generator(device=dev)
    g.manual_seed(4096)
    q = torch.randn((NH, D), generator=g, device=dev)
    kv = [(torch.randn((CTX, NKV * D), generator=g, device=dev).half(),
           torch.randn((CTX, NKV * D), generator=g, device=dev).half()) for _ in range(20)]
    views = [(k.view(CTX, NKV, -1).permute(1, 0, 2), v.view(CTX, NKV, -1).permute(1, 0, 2)) for k, v in kv]
    ws = torch.empty(max(1, ops.lib().amv_flash_attn_workspace_bytes(NH, NKV, CTX, D)), dtype=torch.uint8, device=dev)
    torch.cuda.synchronize()
    for i in range(20):
        ops.flash_attn_decode_kv(q, views[i][0], views[i][1], ops.F16, 0.0884, workspace=ws)
    torch.cuda.synchronize()
    print(json.dumps({"fa_dispatches": 20, "kv_bytes_each": 2 * CTX * NKV * D * 2}), flush=True)


INT8_MFMA_PEAK_TOPS = 5000.0  # MI355X dense int8 matrix peak (5.0 POPS)


def bench_prefill(torch, dev, layer, n_tok):
    """BASELINE config 4 prefill: a prompt of n_tok tokens from position 0 through one layer (int8-MFMA MUL_MATs,
    f16-MFMA causal attention), captured in a HIP graph and replayed; tok/s = n_tok / time of the layer."""
    g = torch.Generator(device=dev)
    g.manual_seed(9)
    x = torch.randn((n_tok, layer.H), generator=g, device=dev)
    out = torch.empty_like(x)
    layer.set_prefill_position(0, n_tok)
    layer.prefill(x, out)  # allocates the chunk buffers before the capture
    ms = time_steps_graph(torch, lambda i: layer.prefill(x, out), 50, 5, per_graph=5)
    ops_ = layer.prefill_ops(n_tok, n_tok)
    tops = ops_ / (ms * 1e-3) / 1e12
    log(f"bench: layer prefill {n_tok} tokens {ms * 1e3:.1f} us = {n_tok / (ms * 1e-3):.0f} tok/s, "
        f"{tops:.1f} TOPS ({tops / INT8_MFMA_PEAK_TOPS * 100:.1f}% of int8 MFMA peak)")
    return {"layer_prefill_512_us": round(ms * 1e3, 2), "layer_prefill_512_tok_s": round(n_tok / (ms * 1e-3), 1),
            "layer_prefill_512_tops": round(tops, 2),
            "layer_prefill_512_frac_int8_peak": round(tops / INT8_MFMA_PEAK_TOPS, 4),
            "layer_prefill_note": "one Llama-3-8B layer, Q4_0, 512-token prompt from position 0, HIP graph"}


def bench_model(torch, dev, n_prompt: int = 512, n_new: int = 256) -> dict:
    """the 32-layer Llama-3-8B-shape stack (Q4_K layers, Q6_K head of 128256 rows, Q4_K token
    embedding), seeded random weights and prompt token ids. A 512-token prefill (the prompt as one chunk through
    every layer, then the first token sampled), then 256 greedy decode steps, each one replay of a decode step
    captured once in a HIP graph (token, position and key count live in device memory; context 513 .. 768)."""
    from ameva_compute_amd.model import random_model
    t0 = time.time()
    m = random_model(dev, ctx=1024, max_new=n_new + 8)
    torch.cuda.synchronize()
    build_s = time.time() - t0
    g = torch.Generator(device=dev)
    g.manual_seed(11)
    prompt = torch.randint(0, m.vocab, (n_prompt,), generator=g, device=dev, dtype=torch.int32)
    m.reset()
    m.prefill(prompt)  # allocates the prompt buffers
    torch.cuda.synchronize()
    reps = 3
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(reps):
        m.reset()
        m.prefill(prompt)
    e1.record()
    torch.cuda.synchronize()
    ms_pf = e0.elapsed_time(e1) / reps
    first = int(m.token.item())
    # decode: one step captured (after a warm-up step on the capture stream), state rewound, then n_new replays
    m.set_position(n_prompt)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        m.decode_step()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        m.decode_step()
    m.set_position(n_prompt)
    m.step.fill_(1)
    m.token.fill_(first)
    torch.cuda.synchronize()
    e0.record()
    for _ in range(n_new):
        gr.replay()
    e1.record()
    torch.cuda.synchronize()
    ms_dec = e0.elapsed_time(e1) / n_new
    assert int(m.step.item()) == n_new + 1 and int(m.pos.item()) == n_prompt + n_new
    toks = m.history[: n_new + 1].cpu().tolist()
    nbytes = m.decode_bytes(n_prompt + n_new // 2)
    ops_pf = m.prefill_ops(n_prompt)
    log(f"bench: model (32 x Q4_K + Q6_K head) prefill {n_prompt} tokens {ms_pf:.1f} ms = "
        f"{n_prompt / (ms_pf * 1e-3):.0f} tok/s ({ops_pf / (ms_pf * 1e-3) / 1e12:.1f} TOPS); decode {ms_dec * 1e3:.1f} "
        f"us/token = {1e3 / ms_dec:.1f} tok/s, {nbytes / (ms_dec * 1e-3) / 1e9:.0f} GB/s; built in {build_s:.1f} s")
    del gr, m
    torch.cuda.empty_cache()
    return {"model_prefill_512_ms": round(ms_pf, 3), "model_prefill_512_tok_s": round(n_prompt / (ms_pf * 1e-3), 1),
            "model_prefill_512_tops": round(ops_pf / (ms_pf * 1e-3) / 1e12, 2),
            "model_decode_ms_per_token": round(ms_dec, 4), "model_decode_tok_s": round(1e3 / ms_dec, 2),
            "model_decode_bytes_per_token": nbytes, "model_decode_gbs": round(nbytes / (ms_dec * 1e-3) / 1e9, 1),
            "model_tokens_head": toks[:8],
            "model_note": "config 5: 32 Llama-3-8B layers Q4_K, Q6_K head 128256 x 4096, Q4_K embedding, random "
                          "weights and prompt ids, 512-token prefill (one chunk) + 256 greedy decode steps (one HIP "
                          "graph replayed per token)"}


def bench_bitnet(n_tok: int = 128) -> dict:
    """BitNet b1.58 2B decode through the per-token engine (libac_bitnet_hip.so, the reference's AcBitNetEngine):
    30 layers of 2560 / 6912 (20 / 5 heads of 128, ReLU^2 FFN with sub norms, RoPE theta 500000), random ternary I2_S
    weights (P = 1/3 each) and an f16 LM head of 128256 x 2560 (random rows). n_tok tokens from position 0, each one
    EvalToken call (x in from host memory, x out and all logits back), timed by the host clock around the calls, so
    the figure includes the two small copies and the graph launch. Bytes per token: every I2_S weight byte, the LM
    head, and the f32 K / V rows read by the attention (at the mean position)."""
    import numpy as np
    from ameva_compute_amd.bitnet_engine import BitNetEngine
    E, F, H, KVH, HD, NL, V, CTX = 2560, 6912, 20, 5, 128, 30, 128256, 4096
    rng = np.random.default_rng(2025)
    # every byte of 4 codes in {0, 1, 2} (code 1 = weight 0): 81 byte values
    c = np.array([(a << 6) | (b << 4) | (d << 2) | e for a in range(3) for b in range(3) for d in range(3)
                  for e in range(3)], np.uint8)
    t0 = time.time()
    eng = BitNetEngine()
    eng.configure(E, F, H, KVH, HD, CTX, NL, 1e-5, 500000.0, True)
    kv = KVH * HD
    nrm = lambda n: (1 + 0.1 * rng.standard_normal(n)).astype(np.float32)  # noqa: E731
    w = lambda r, k: c[rng.integers(0, 81, (r, k // 4))]  # noqa: E731
    wbytes = 0
    for i in range(NL):
        lay = dict(attn_norm=nrm(E), attn_sub_norm=nrm(E), ffn_norm=nrm(E), ffn_sub_norm=nrm(F), wq=w(E, E),
                   wk=w(kv, E), wv=w(kv, E), wo=w(E, E), w_gate=w(F, E), w_up=w(F, E), w_down=w(E, F),
                   scale_wq=1.2, scale_wk=1.1, scale_wv=0.9, scale_wo=0.03, scale_w_gate=0.8, scale_w_up=0.7,
                   scale_w_down=0.01)
        wbytes += sum(lay[n].nbytes for n in ("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down"))
        eng.upload_layer(i, lay)
    block = (rng.standard_normal((1024, E)) * 0.02).astype(np.float16).view(np.uint16)
    head = np.empty((V, E), np.uint16)
    for r0 in range(0, V, 1024):
        head[r0:r0 + 1024] = block[: min(1024, V - r0)]
    eng.upload_output(nrm(E), head)
    del head
    build_s = time.time() - t0
    x = (rng.standard_normal(E) * 0.5).astype(np.float32)
    xo = np.empty(E, np.float32)
    lg = np.empty(V, np.float32)
    for p in range(4):  # the first call captures the step graph
        eng.eval_token(p, x, xo, lg)
    res = {}
    for name, want_logits in (("with_logits", True), ("no_logits", False)):
        t0 = time.perf_counter()
        for p in range(n_tok):
            eng.eval_token(p, x, xo, lg if want_logits else None)
        s = (time.perf_counter() - t0) / n_tok
        kv_bytes = 2 * NL * (n_tok // 2) * kv * 4
        nbytes = wbytes + kv_bytes + (V * E * 2 if want_logits else 0)
        res[f"bitnet2b_decode_{name}_ms_per_token"] = round(s * 1e3, 4)
        res[f"bitnet2b_decode_{name}_tok_s"] = round(1 / s, 1)
        res[f"bitnet2b_decode_{name}_gbs"] = round(nbytes / s / 1e9, 1)
        log(f"bench: BitNet 2B decode ({name}) {s * 1e3:.3f} ms/token = {1 / s:.0f} tok/s, "
            f"{nbytes / 2**20:.0f} MiB/token -> {nbytes / s / 1e9:.0f} GB/s")
    assert np.isfinite(xo).all() and np.isfinite(lg).all()
    eng.close()
    res["bitnet2b_i2s_weight_bytes"] = wbytes
    res["bitnet2b_note"] = (f"30 BitNet b1.58 2B layers (I2_S) + f16 LM head {V} x {E}, random weights, {n_tok} tokens "
                            f"from position 0 through AcBitNetEngine::EvalToken (one HIP graph per token), host clock; "
                            f"built in {build_s:.1f} s")
    return res


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def load_traffic():
    """HBM bytes per launch of the headline kernel from the committed rocprofv3 --pmc summary (profiles/)."""
    path = os.path.join(ROOT, "profiles", "q4_0_gemv_14336x4096_traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get("traffic_bytes_per_launch")
    except (OSError, ValueError):
        return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only-headline", action="store_true", help="skip the secondary figures (for profiling)")
    ap.add_argument("--only-layer", action="store_true", help="only the layer decode figure (for profiling)")
    ap.add_argument("--only-i2s", action="store_true", help="only the BitNet I2_S figures (for profiling)")
    ap.add_argument("--only-batched", action="store_true", help="only the batched MUL_MAT figures (for profiling)")
    ap.add_argument("--only-model", action="store_true", help="only the 32-layer model figures (for profiling)")
    ap.add_argument("--no-model", action="store_true", help="skip the 32-layer model figures")
    ap.add_argument("--only-bitnet", action="store_true", help="only the BitNet 2B engine decode figures")
    ap.add_argument("--only-load", action="store_true", help="only the weight load path figures (repack, upload)")
    ap.add_argument("--only-kv", action="store_true", help="only the FA decode figures over the three KV caches")
    ap.add_argument("--only-plugin", action="store_true",
                    help="only the layer decode through libggml-ameva.so graph_compute")
    ap.add_argument("--pmc-gemm", action="store_true",
                    help="for rocprofv3 --pmc: 20 eager exact Q4_K MUL_MATs at M = 512 on each FFN shape")
    ap.add_argument("--pmc-probe", action="store_true",
                    help="for rocprofv3 --pmc: 50 eager cold headline GEMVs and 50 plain copies of the same byte "
                         "count (the counter scale reference); prints a JSON line of what ran")
    ap.add_argument("--pmc-gemm-scaled", action="store_true",
                    help="as --pmc-gemm, with the scaled f16-MFMA form (Q8_K_DEQ activations)")
    ap.add_argument("--pmc-small", action="store_true",
                    help="for rocprofv3 --pmc: 20 eager cold Q4_K and Q6_K MUL_MATs at M = 16 (14336 x 4096)")
    ap.add_argument("--pmc-i2s", action="store_true",
                    help="for rocprofv3 --pmc: 20 eager I2_S batch-128 MUL_MATs on each BitNet 2B shape")
    ap.add_argument("--pmc-fa", action="store_true",
                    help="for rocprofv3 --pmc: 20 eager cold FA decodes at 4096 keys over an F16 cache")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}",
              file=sys.stderr)
        sys.exit(2)

    import torch
    from ameva_compute_amd import ops
    assert torch.cuda.is_available(), "no GPU"
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    if args.pmc_probe:
        pmc_probe(ops, torch, dev)
        return
    if args.pmc_gemm or args.pmc_gemm_scaled:
        pmc_gemm(ops, torch, dev, exact=not args.pmc_gemm_scaled)
        return
    if args.pmc_i2s:
        pmc_i2s(ops, torch, dev)
        return
    if args.pmc_small:
        pmc_small(ops, torch, dev)
        return
    if args.pmc_fa:
        pmc_fa(ops, torch, dev)
        return
    if args.only_layer:
        print(json.dumps(bench_layer(torch, dev, args)), flush=True)
        return
    if args.only_batched:
        print(json.dumps(bench_batched(ops, torch, dev)), flush=True)
        return
    if args.only_i2s:
        print(json.dumps(bench_i2s(ops, torch, dev)), flush=True)
        return
    if args.only_model:
        print(json.dumps(bench_model(torch, dev)), flush=True)
        return
    if args.only_bitnet:
        print(json.dumps(bench_bitnet()), flush=True)
        return
    if args.only_load:
        print(json.dumps(bench_load_path(ops, torch, dev)), flush=True)
        return
    if args.only_kv:
        print(json.dumps(bench_kv_cache(ops, torch, dev)), flush=True)
        return
    if args.only_plugin:
        print(json.dumps(bench_plugin_layer(torch, dev)), flush=True)
        return

    log(f"bench: Q4_0 GEMV {N_ROWS}x{K}, {COPIES} weight copies, steps={args.steps} warmup={args.warmup}")
    ws = make_weights(ops, torch, N_ROWS, K, COPIES, 42, dev, ops.Q4_0)
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    x = torch.randn((1, K), generator=g, device=dev, dtype=torch.float32)
    act, _ = ops.quantize_act(x, ops.Q8_0, ops.Q8_X86)
    out = torch.empty((1, N_ROWS), dtype=torch.float32, device=dev)

    def step_cold(i):
        ops.mul_mat_q(ws[i % COPIES], act, 1, out)

    def step_hot(i):
        ops.mul_mat_q(ws[0], act, 1, out)

    ran = {}
    ms_cold = time_steps_graph(torch, step_cold, args.steps, args.warmup, info=ran, min_reps=10, median=True)
    nbytes = gemv_bytes(N_ROWS, K)
    gbs = nbytes / (ms_cold * 1e-3) / 1e9
    log(f"bench: cold {ms_cold * 1e3:.2f} us/GEMV = {gbs:.1f} GB/s ({gbs / HBM_PEAK_GBS * 100:.1f}% of HBM peak)")
    extra = {}
    # the read ceiling of the headline kernel's mapping: the same grid and weight / scale loads over the same cold
    # copies, without the activation and the arithmetic (amv_debug_gemv_read_probe)
    from ameva_compute_amd._lib import check, lib as _lib
    probe_out = torch.empty(N_ROWS, dtype=torch.int32, device=dev)

    def probe(w_ptr, n_rows, loads):
        check(_lib().amv_debug_gemv_read_probe(w_ptr, n_rows, K, probe_out.data_ptr(), loads,
                                               torch.cuda.current_stream().cuda_stream), "read probe")
    ms_probe = time_steps_graph(torch, lambda i: probe(ws[i % COPIES].data.data_ptr(), N_ROWS, 1), args.steps,
                                args.warmup, min_reps=10, median=True)
    ms_floor = time_steps_graph(torch, lambda i: probe(ws[i % COPIES].data.data_ptr(), N_ROWS, 0), args.steps,
                                args.warmup, min_reps=10, median=True)
    extra["gemv_read_probe_cold_us"] = round(ms_probe * 1e3, 3)
    extra["gemv_read_probe_cold_gbs"] = round(ws[0].nbytes / (ms_probe * 1e-3) / 1e9, 1)
    extra["gemv_grid_launch_floor_us"] = round(ms_floor * 1e3, 3)
    # the same mapping over 2 GiB (932,066 rows of 2304 bytes): its streaming rate with the fixed cost amortised
    big_rows = (2 << 30) // 2304 // 2 * 2
    big = torch.empty(big_rows * 2304, dtype=torch.uint8, device=dev)
    big_out = torch.empty(big_rows, dtype=torch.int32, device=dev)
    ms_big = time_steps_graph(torch, lambda i: check(_lib().amv_debug_gemv_read_probe(
        big.data_ptr(), big_rows, K, big_out.data_ptr(), 1, torch.cuda.current_stream().cuda_stream), "read probe"),
        20, 3, min_reps=10, median=True)
    extra["gemv_read_probe_2gib_gbs"] = round(big.numel() / (ms_big * 1e-3) / 1e9, 1)
    del big, big_out
    log(f"bench: read probe of the same mapping {ms_probe * 1e3:.2f} us (weights only: "
        f"{ws[0].nbytes / (ms_probe * 1e-3) / 1e9:.0f} GB/s); the grid without loads {ms_floor * 1e3:.2f} us; "
        f"the mapping over 2 GiB {extra['gemv_read_probe_2gib_gbs']:.0f} GB/s")
    if not args.only_headline:
        ms_hot = time_steps_graph(torch, step_hot, args.steps, args.warmup)
        extra["hot_gbs"] = round(nbytes / (ms_hot * 1e-3) / 1e9, 1)
        extra["hot_us"] = round(ms_hot * 1e3, 3)
        ms_eager = time_steps(torch, step_cold, 500, 50)
        extra["cold_eager_launch_us"] = round(ms_eager * 1e3, 3)

        act2 = torch.empty_like(act)

        def step_quant(i):
            _lib().amv_quantize_act(ops.Q8_0, x.data_ptr(), 1, K, ops.Q8_X86, None, act2.data_ptr(),
                                    torch.cuda.current_stream().cuda_stream)
        extra["q8_0_quantize_4096_us"] = round(time_steps_graph(torch, step_quant, 500, 100) * 1e3, 3)
        del ws
        torch.cuda.empty_cache()
        extra.update(secondary_gemvs(ops, torch, dev))
        extra.update(bench_batched(ops, torch, dev))
        extra.update(bench_i2s(ops, torch, dev))
        extra.update(bench_kv_cache(ops, torch, dev))
        extra.update(bench_load_path(ops, torch, dev))
        extra.update(copy_ceiling(torch, dev, nbytes))

    layer_info = None
    if not args.only_headline:
        layer_info = bench_layer(torch, dev, args)
        extra.update(layer_info)
        extra.update(bench_plugin_layer(torch, dev))
        if not args.no_model:
            extra.update(bench_model(torch, dev))
            extra.update(bench_bitnet())

    result = {
        "metric": "Q4_0 GEMV GB/s (% HBM peak) + bs1 decode tok/s, Llama-8B-shape layer",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": ran["timed"],
        "warmup": ran["warmup"],
        "ms_per_step": round(ms_cold, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_0 x q8_0 (int8 dot, f32 accumulate)",
        "data": "synthetic: seeded N(0,0.02) weights quantized on the GPU (ggml Q4_0 rule), N(0,1) activation",
        "config": {"workload": "Q4_0 GEMV 14336x4096 M=1 (Llama-3-8B FFN gate/up), Q8_0 activation, cold: "
                               f"{COPIES} rotating weight copies ({COPIES * N_ROWS * K * 18 // 32 / 2**20:.0f} MiB)",
                   "n_rows": N_ROWS, "k": K, "m": 1, "weight_copies": COPIES, "timing": f"HIP graph of {GRAPH_STEPS} GEMV launches replayed {ran['replays']} times, each "
                             f"replay timed by its own events, median replay / {GRAPH_STEPS} (steps = GEMVs timed, "
                             f"at least 10 replays whatever --steps says); warmup = {GRAPH_STEPS} eager GEMVs + "
                             f"{ran['warmup'] // GRAPH_STEPS - 1} untimed replays"},
        "roofline": {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": load_traffic()},
        "extra": extra,
    }
    if not args.no_cpu:
        log("bench: CPU baseline ...")
        result["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
