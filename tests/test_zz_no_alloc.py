"""amv_flash_attn_decode_noalloc (the decode attention that allocates nothing: split partials in the library's
static device scratch) against amv_flash_attn_decode_kv with a caller workspace, both called through the C ABI:
identical outputs and activation rows on two calls in a row, the second one smaller, and on a HIP-graph replay."""
import ctypes

import numpy as np
import pytest

torch = pytest.importorskip("torch")

F16, Q8_0 = 1, 8


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


def _case(dev, seed, n_head, n_head_kv, ctx, n_kv):
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    D = 128
    q = torch.randn((n_head, D), generator=g, device=dev)
    # llama.cpp's token-major cache view: element d of key j of KV head h at [j][h][d]
    kc = torch.randn((ctx, n_head_kv, D), generator=g, device=dev).half()
    vc = torch.randn((ctx, n_head_kv, D), generator=g, device=dev).half()
    mask = torch.zeros(ctx, dtype=torch.float16, device=dev)
    mask[n_kv // 3::7] = float("-inf")
    return q, kc, vc, mask


def _call(L, fn, q, kc, vc, mask, n_head, n_head_kv, n_kv, n_kv_dev, act, ws=None):
    out = torch.empty_like(q)
    D = 128
    args = [F16, q.data_ptr(), kc.data_ptr(), vc.data_ptr(), mask.data_ptr(), out.data_ptr(), n_head, n_head_kv,
            n_kv, n_kv_dev.data_ptr() if n_kv_dev is not None else None, D, kc.stride(0) * 2, kc.stride(1) * 2,
            vc.stride(0) * 2, vc.stride(1) * 2, ctypes.c_float(1.0 / np.sqrt(D))]
    st = torch.cuda.current_stream().cuda_stream
    if fn == "ws":
        rc = L.amv_flash_attn_decode_kv(*args, ws.data_ptr(), ws.numel(), None, act.data_ptr(), Q8_0, 0, st)
    else:
        rc = L.amv_flash_attn_decode_noalloc(*args, act.data_ptr(), Q8_0, 0, st)
    assert rc == 0, L.amv_last_error()
    return out


def test_noalloc_rejects_sizes_beyond_its_scratch():
    """Host-side rule, no GPU call: partials above the 8 MiB scratch are refused with a message before any launch."""
    from ameva_compute_amd._lib import lib
    L = lib()
    need = L.amv_flash_attn_workspace_bytes(64, 8, 131072, 128)
    assert need > L.amv_flash_attn_noalloc_max_bytes()
    rc = L.amv_flash_attn_decode_noalloc(F16, None, None, None, None, None, 64, 8, 131072, None, 128, 2048, 256,
                                         2048, 256, ctypes.c_float(0.1), None, Q8_0, 0, None)
    assert rc == -1 and b"scratch" in L.amv_last_error()


@pytest.mark.gpu
def test_noalloc_matches_workspace_entry(dev):
    from ameva_compute_amd._lib import lib
    L = lib()
    assert L.amv_flash_attn_noalloc_max_bytes() == 8 << 20
    # two calls in a row: the Llama-3-8B decode shape at 4096 keys, then a smaller one (fewer heads and keys) that
    # reuses the scratch the first call left behind
    for seed, (n_head, n_head_kv, ctx, n_kv) in enumerate([(32, 8, 4096, 4096), (8, 2, 700, 523)]):
        q, kc, vc, mask = _case(dev, 100 + seed, n_head, n_head_kv, ctx, n_kv)
        need = L.amv_flash_attn_workspace_bytes(n_head, n_head_kv, n_kv, 128)
        ws = torch.empty(need, dtype=torch.uint8, device=dev)
        nab = L.amv_act_bytes(Q8_0, 1, n_head * 128)
        act_w = torch.zeros(nab, dtype=torch.uint8, device=dev)
        act_n = torch.ones(nab, dtype=torch.uint8, device=dev)
        ref = _call(L, "ws", q, kc, vc, mask, n_head, n_head_kv, n_kv, None, act_w, ws)
        got = _call(L, "noalloc", q, kc, vc, mask, n_head, n_head_kv, n_kv, None, act_n)
        torch.cuda.synchronize()
        print(f"call {seed}: n_head {n_head} n_kv {n_kv} max |diff| {(got - ref).abs().max().item()}", flush=True)
        assert torch.isfinite(ref).all()
        assert torch.equal(got, ref), seed
        assert torch.equal(act_n, act_w), seed


@pytest.mark.gpu
def test_noalloc_key_count_in_device_memory_and_graph_replay(dev):
    """The key count read from device memory and the call captured in a HIP graph: every replay at a new count equals
    the workspace entry point at that count."""
    from ameva_compute_amd._lib import lib
    L = lib()
    n_head, n_head_kv, ctx = 32, 8, 2048
    q, kc, vc, mask = _case(dev, 7, n_head, n_head_kv, ctx, ctx)
    nkv = torch.tensor([1000], dtype=torch.int32, device=dev)
    act = torch.zeros(L.amv_act_bytes(Q8_0, 1, n_head * 128), dtype=torch.uint8, device=dev)
    act_ref = torch.zeros_like(act)
    ws = torch.empty(L.amv_flash_attn_workspace_bytes(n_head, n_head_kv, ctx, 128), dtype=torch.uint8, device=dev)
    out_holder = {}
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):  # the first call on the device (scratch lookup) and a warm-up, outside capture
        out_holder["o"] = _call(L, "noalloc", q, kc, vc, mask, n_head, n_head_kv, ctx, nkv, act)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        out_holder["o"] = _call(L, "noalloc", q, kc, vc, mask, n_head, n_head_kv, ctx, nkv, act)
    for n in (1000, 1, 2048, 333):
        nkv.fill_(n)
        out_holder["o"].zero_()
        torch.cuda.synchronize()
        gr.replay()
        torch.cuda.synchronize()
        ref = _call(L, "ws", q, kc, vc, mask, n_head, n_head_kv, ctx, nkv, act_ref, ws)
        torch.cuda.synchronize()
        assert torch.equal(out_holder["o"], ref), n
        assert torch.equal(act, act_ref), n
