"""The decoder stack of ameva_compute_amd.model (BASELINE config 5 architecture) and its new kernels: GET_ROWS of
Q4_K / Q6_K embedding rows against the oracle's dequantization (bit for bit), the greedy argmax, and generation of a
small random model: a decode step captured once in a HIP graph and replayed must produce the same tokens and logits
as eager steps (fused and one launch per node), and the prompt run as one prefill chunk must agree with the same
prompt decoded token by token within the chain bar."""
import numpy as np
import pytest

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")


@pytest.fixture(scope="module")
def ops():
    from ameva_compute_amd import ops
    return ops


def rel_l2(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-30))


def random_kquant(rng, t, n, k):
    bb = 144 if t == 12 else 210
    y = rng.integers(0, 256, (n, k // 256, bb), dtype=np.uint8)
    for off in ((0, 2) if t == 12 else (208,)):
        v = rng.uniform(-0.01, 0.01, (n, k // 256)).astype(np.float16)
        y[:, :, off:off + 2] = v.view(np.uint8).reshape(n, k // 256, 2)
    return y.reshape(n, -1)


@pytest.mark.parametrize("t", [12, 14])
def test_get_rows_kquant(dev, ops, orc, t):
    rng = np.random.default_rng(t)
    rows, n = 300, 1024
    tab = random_kquant(rng, t, rows, n)
    ids = np.array([0, 299, 17, 17, 150, 3], np.int32)
    got = ops.get_rows(torch.from_numpy(tab).to(dev), t, n, torch.from_numpy(ids).to(dev)).cpu().numpy()
    ref = orc.dequantize(t, tab, n)[ids]
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    with pytest.raises(IndexError):
        ops.get_rows(torch.from_numpy(tab).to(dev), t, n, torch.tensor([300], dtype=torch.int32, device=dev))


def test_argmax(dev, ops):
    rng = np.random.default_rng(4)
    for n in (1, 7, 1000, 128256):
        x = rng.standard_normal(n).astype(np.float32)
        tok = ops.argmax(torch.from_numpy(x).to(dev))
        assert int(tok.item()) == int(np.argmax(x)), n
    for where in ([100000, 40000, 5], [128255], [40963, 32768 + 4]):  # ties across rounds and threads, the last entry
        x = np.zeros(128257, np.float32)
        x[where] = 2.0
        assert int(ops.argmax(torch.from_numpy(x).to(dev)).item()) == min(where)
    x = np.zeros(5000, np.float32)
    x[[10, 4000, 4999]] = 3.0          # ties: the first index
    x[[1, 2]] = np.nan                 # NaN never wins
    hist = torch.full((3,), -1, dtype=torch.int32, device=dev)
    step = torch.zeros(1, dtype=torch.int32, device=dev)
    xg = torch.from_numpy(x).to(dev)
    for _ in range(4):                 # the 4th call is past the history: counted, not stored
        ops.argmax(xg, history=hist, step=step)
    assert hist.tolist() == [10, 10, 10] and int(step.item()) == 4


def test_argmax_ex_matches_argmax_and_advances(dev, ops):
    """amv_argmax_ex (every workgroup offers a (value, index) key to an atomic maximum, the last to arrive writes the
    token) gives amv_argmax's token: random rows, ties within and across workgroups (the first index), NaN never
    winning, -0 tied with +0, all-NaN and all -inf rows (token 0), lengths not a multiple of 4 or of a workgroup's
    8192 floats; the decode position (pos, kv_idx, n_kv) moves on by one per call, and ws is left zero."""
    lib = ops.lib()
    st = torch.cuda.current_stream().cuda_stream
    ws = torch.zeros(2, dtype=torch.int64, device=dev)
    pos = torch.tensor([7], dtype=torch.int32, device=dev)
    kv = torch.tensor([7], dtype=torch.int64, device=dev)
    nkv = torch.tensor([8], dtype=torch.int32, device=dev)
    rng = np.random.default_rng(44)
    cases = [rng.standard_normal(n).astype(np.float32) for n in (1, 3, 7, 1000, 8191, 8192, 8193, 128256, 128257)]
    for where in ([100000, 40000, 5], [128255], [40963, 32768 + 4], [8191, 8192], [16383, 16384, 0]):
        x = np.zeros(128257, np.float32)
        x[where] = 2.0
        cases.append(x)
    x = np.full(20000, -1.0, np.float32)
    x[[9000, 17000]] = -0.0
    x[[12000, 3]] = 0.0                # +0 and -0 tie: the first index of either
    cases.append(x)
    x = np.zeros(30000, np.float32)
    x[:] = np.nan
    x[29999] = -5.0                    # NaN never wins: the only number does
    cases.append(x)
    cases.append(np.full(20001, np.nan, np.float32))
    cases.append(np.full(9000, -np.inf, np.float32))
    for i, x in enumerate(cases):
        xg = torch.from_numpy(x).to(dev)
        want = int(ops.argmax(xg).item())
        tok = torch.full((1,), -1, dtype=torch.int32, device=dev)
        rc = lib.amv_argmax_ex(xg.data_ptr(), x.size, tok.data_ptr(), None, None, 0, pos.data_ptr(), kv.data_ptr(),
                               nkv.data_ptr(), ws.data_ptr(), st)
        assert rc == 0, lib.amv_last_error()
        torch.cuda.synchronize()
        assert int(tok.item()) == want, (i, x.size)
        assert not ws.any()
    n = len(cases)
    assert int(pos.item()) == 7 + n and int(kv.item()) == 7 + n and int(nkv.item()) == 8 + n
    # history and step as amv_argmax, without the position (NULL pointers)
    hist = torch.full((2,), -1, dtype=torch.int32, device=dev)
    step = torch.zeros(1, dtype=torch.int32, device=dev)
    xg = torch.from_numpy(cases[7]).to(dev)
    for _ in range(3):
        assert lib.amv_argmax_ex(xg.data_ptr(), xg.numel(), tok.data_ptr(), hist.data_ptr(), step.data_ptr(), 2, None,
                                 None, None, ws.data_ptr(), st) == 0
    torch.cuda.synchronize()
    assert hist.tolist() == [int(np.argmax(cases[7]))] * 2 and int(step.item()) == 3


def tiny_model(dev):
    from ameva_compute_amd.model import random_model
    return random_model(dev, n_layers=2, H=256, n_head=2, n_head_kv=1, D=128, FF=512, vocab=1000, ctx=64, seed=3,
                        max_new=16)


def test_model_generation_graph_replay(dev):
    m = tiny_model(dev)
    g = torch.Generator(device=dev)
    g.manual_seed(1)
    prompt = torch.randint(0, m.vocab, (12,), generator=g, device=dev, dtype=torch.int32)
    steps = 6

    def run(fused, graph):
        for lay in m.layers:
            lay.k_cache.zero_()
            lay.v_cache.zero_()
        m.reset()
        m.prefill(prompt)
        m.set_position(prompt.numel())
        logits = [m.logits.clone()]
        if graph:
            s = torch.cuda.Stream()
            s.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(s):
                m.decode_step(fused)  # warm-up (decodes the first sampled token)
            torch.cuda.current_stream().wait_stream(s)
            torch.cuda.synchronize()
            logits.append(m.logits.clone())
            gr = torch.cuda.CUDAGraph()
            with torch.cuda.graph(gr):
                m.decode_step(fused)
            for _ in range(steps - 1):
                gr.replay()
                torch.cuda.synchronize()
                logits.append(m.logits.clone())
        else:
            for _ in range(steps):
                if not fused:  # the per-node path reads the key count from the host
                    m.set_position(int(m.pos.item()))
                m.decode_step(fused)
                logits.append(m.logits.clone())
        torch.cuda.synchronize()
        return m.history[: steps + 1].cpu().tolist(), int(m.step.item()), torch.stack(logits)

    h_eager, n_eager, l_eager = run(True, False)
    assert n_eager == steps + 1
    h_graph, _, l_graph = run(True, True)
    assert h_graph == h_eager and torch.equal(l_graph, l_eager)
    h_node, _, l_node = run(False, False)
    assert h_node == h_eager and torch.equal(l_node, l_eager)
    # the argmax of each step's logits is the next token
    assert [int(torch.argmax(l).item()) for l in l_eager] == h_eager


def test_model_prefill_matches_token_by_token(dev):
    """The prompt as one prefill chunk (MFMA GEMMs, f16-MFMA causal attention) against the same prompt decoded one
    token at a time: the head logits after the last prompt token agree within the chain bar."""
    m = tiny_model(dev)
    g = torch.Generator(device=dev)
    g.manual_seed(2)
    prompt = torch.randint(0, m.vocab, (20,), generator=g, device=dev, dtype=torch.int32)
    m.reset()
    m.prefill(prompt)
    torch.cuda.synchronize()
    lp = m.logits.cpu().numpy().copy()
    for lay in m.layers:
        lay.k_cache.zero_()
        lay.v_cache.zero_()
    m.reset()
    for i in range(prompt.numel()):
        m.set_position(i)
        m.token.copy_(prompt[i:i + 1])
        m.decode_step(True)
    torch.cuda.synchronize()
    ld = m.logits.cpu().numpy()
    assert rel_l2(ld, lp) < 2e-2
