"""The device-resident decode step (include/gs_decode.h): the body of
generate_collect (src/main.rs:279-304) -- sample, stop check, max check,
recent push, generated push -- with the logits produced in HBM by gs_gemv
and the loop state on the device.

CPU: the oracle's loop (oracle.generate) is pinned against the oracle's
decode_trace (the sampler loop without stops) and the LCG's closed form:
a stop token or the max check ends the loop after consuming that step's
draw, and the FIFO is the last W ids.

GPU: a toy decoder (x = E[token], logits = lm_head x, Q6_K) runs on the
device; every step's logits are kept, and the oracle's loop over those same
logits must give the same tokens, stop reason, LCG state and window, row by
row (integer results: bit-exact).  A captured HIP graph of several steps,
replayed with eager work between replays, must reproduce the eager run.
"""
import ctypes

import numpy as np
import pytest

DEFAULTS = (0.7, 40, 0.9, 1.1)      # src/main.rs:24-31


# ---- oracle pins (CPU) --------------------------------------------------------
def _rand_logits(rng, steps, V):
    return (rng.standard_normal((steps, V)) * 3.0).astype(np.float32)


def test_generate_without_stops_is_decode_trace(oracle):
    rng = np.random.default_rng(7)
    lg = _rand_logits(rng, 30, 500)
    init = rng.integers(0, 500, 10).astype(np.uint32)
    g = oracle.generate(lg, DEFAULTS, 64, init, [], 1000, 42)
    want = oracle.decode_trace(lg, *DEFAULTS, 64, init, 42)
    assert np.array_equal(g["sampled"], want)
    assert g["done"] == 0 and np.array_equal(g["generated"], want.astype(np.uint32))
    _, st = oracle.lcg_draws(42, 30)
    assert g["state"] == st
    assert np.array_equal(g["recent"], np.concatenate([init, want.astype(np.uint32)])[-64:])


def test_generate_stop_and_max(oracle):
    """A stop token at step j: j+1 steps taken, j ids generated, j+1 draws
    consumed (src/main.rs:280-281).  max_new = m: m+1 steps, m ids."""
    rng = np.random.default_rng(8)
    lg = _rand_logits(rng, 40, 300)
    full = oracle.generate(lg, DEFAULTS, 16, [], [], 1000, 5)["sampled"]
    j = 17
    stop = int(full[j])
    j = int(np.nonzero(full == stop)[0][0])          # first occurrence
    g = oracle.generate(lg, DEFAULTS, 16, [], [stop, 299999], 1000, 5)
    assert g["done"] == 1 and len(g["sampled"]) == j + 1
    assert np.array_equal(g["generated"], full[:j].astype(np.uint32))
    assert g["state"] == oracle.lcg_draws(5, j + 1)[1]
    assert np.array_equal(g["recent"], full[:j][-16:].astype(np.uint32))
    m = 9
    g = oracle.generate(lg, DEFAULTS, 16, [], [], m, 5)
    assert g["done"] == 2 and len(g["sampled"]) == m + 1 and len(g["generated"]) == m
    assert g["state"] == oracle.lcg_draws(5, m + 1)[1]
    g = oracle.generate(lg, (0.0, 40, 0.9, 1.1), 16, [], [], m, 5)     # greedy: no draws
    assert g["state"] == 5


def test_decode_arguments_rejected_without_gpu():
    """Argument checks return before any HIP call."""
    import gs_sampler
    lib = gs_sampler.load_library()
    ctx = gs_sampler.DecodeCtx()
    assert lib.gs_decode_commit(None, None, None, None) == gs_sampler.GS_ERR_INVALID
    assert lib.gs_decode_commit(None, None, ctypes.byref(ctx), None) == gs_sampler.GS_ERR_INVALID
    ctx.B, ctx.rows, ctx.u, ctx.tokens = 4, 0x1000, 0x2000, 0x3000
    ctx.n_stop, ctx.stop = 1000, 0x4000
    assert lib.gs_decode_commit(None, None, ctypes.byref(ctx), None) == gs_sampler.GS_ERR_UNSUPPORTED
    ctx.n_stop, ctx.W, ctx.window = 0, 8, None
    assert lib.gs_decode_commit(None, None, ctypes.byref(ctx), None) == gs_sampler.GS_ERR_INVALID
    ctx.W = 0
    assert lib.gs_decode_commit(None, None, ctypes.byref(ctx), None) == gs_sampler.GS_ERR_INVALID   # no sampler
    assert lib.gs_decode_init(None, None, ctypes.byref(ctx), None, None, None) == gs_sampler.GS_ERR_INVALID
    ctx.W = 0
    assert lib.gs_decode_step(None, None, None, None, 0, 0, None, ctypes.byref(ctx), None) == gs_sampler.GS_ERR_INVALID


# ---- GPU ------------------------------------------------------------------------
class _Toy:
    """x_{t+1} = E[token_t]; logits = lm_head x (Q6_K, V x cols)."""

    def __init__(self, gpu, torch, V, cols, seed):
        import workloads
        rng = np.random.default_rng(seed)
        self.blocks = workloads.synth_qblocks(gpu.QTYPE_Q6_K, V, cols, seed=seed)
        self.m = gpu.QMatrix(gpu.QTYPE_Q6_K, self.blocks, V, cols)
        self.E = torch.from_numpy((rng.standard_normal((V, cols)) * 0.1).astype(np.float32)).cuda()
        self.V, self.cols = V, cols

    def embed(self, torch, tokens, x):
        torch.index_select(self.E, 0, tokens, out=x)


def _run_eager(gpu, torch, toy, dec, sampler, first, steps, params=None):
    B = dec.B
    x = torch.empty((B, toy.cols), dtype=torch.float32, device="cuda")
    logits = torch.empty((B, toy.V), dtype=torch.float32, device="cuda")
    hist = torch.empty((steps, B, toy.V), dtype=torch.float32, device="cuda")
    dec.next.copy_(torch.as_tensor(first, dtype=torch.int32).cuda())
    for t in range(steps):
        toy.embed(torch, dec.next, x)
        dec.step(sampler, logits=logits, lm_head=toy.m, x=x, params=params)
        hist[t].copy_(logits)
    torch.cuda.synchronize()
    return hist.cpu().numpy()


def _check_rows(oracle, dec, hist, row_params, W, init, stops, max_new, seeds):
    st = dec.row_state()
    gen = dec.generated_ids()
    win = dec.window.cpu().numpy().view(np.uint32)
    wl = dec.window_len.cpu().numpy()
    for b in range(dec.B):
        o = oracle.generate(hist[:, b], row_params[b], W, init[b], stops, max_new, seeds[b])
        assert o["done"] != 0, ("loop did not end in the steps run", b)
        assert int(st["done"][b]) == o["done"], (b, st[b], o["done"])
        assert np.array_equal(gen[b], o["generated"]), (b, gen[b], o["generated"])
        assert int(st["last"][b]) == int(o["sampled"][-1]), b
        assert int(st["rng"][b]) == o["state"], b
        assert int(st["n_gen"][b]) == len(o["generated"])
        if W:
            # the ring holds the FIFO's ids; oldest slot at wpos % W once full
            n = int(wl[b])
            assert n == len(o["recent"]), b
            wp = int(st["wpos"][b])
            ring = win[b, :W]
            fifo = np.concatenate([ring[wp % W:], ring[:wp % W]]) if wp >= W else ring[:n]
            assert np.array_equal(fifo, o["recent"]), (b, fifo, o["recent"])
    return st


@pytest.mark.gpu
def test_decode_step_matches_reference_loop(gpu, torch, oracle):
    """Four rows, each with its own params (default CLI, greedy, full
    vocabulary with a nucleus, top-1 with a strong penalty), its own seed and
    start window, a shared stop set and max_new; the GEMV produces each step's
    logits on the device."""
    V, cols, B, W, max_new = 32000, 1024, 4, 64, 40
    toy = _Toy(gpu, torch, V, cols, seed=21)
    row_params = [DEFAULTS, (0.0, 40, 0.9, 1.1), (1.0, 0, 0.95, 1.0), (0.8, 1, 1.0, 1.3)]
    d_params = torch.from_numpy(gpu.params_array(row_params).view(np.uint8)).cuda()
    seeds = [42, 7, 123456789, 2 ** 63 + 5]
    rng = np.random.default_rng(3)
    init = [rng.integers(0, V, n).astype(np.uint32) for n in (0, 5, 64, 30)]
    first = [11, 12, 13, 14]
    sampler = gpu.Sampler(*DEFAULTS, seed=1)
    sampler.reserve(B, V)
    # run 1: no stops, to learn the streams; then stop on ids seen mid-run
    dec = gpu.Decoder(B, W=W, max_new=max_new, stop=())
    dec.init(sampler, seeds, init, params=d_params)
    hist = _run_eager(gpu, torch, toy, dec, sampler, first, max_new + 1, d_params)
    _check_rows(oracle, dec, hist, row_params, W, init, [], max_new, seeds)
    g1 = dec.generated_ids()
    stops = [int(g1[0][9]), int(g1[2][4]), V + 5]
    dec2 = gpu.Decoder(B, W=W, max_new=max_new, stop=stops)
    dec2.init(sampler, seeds, init, params=d_params)
    hist2 = _run_eager(gpu, torch, toy, dec2, sampler, first, max_new + 1, d_params)
    st = _check_rows(oracle, dec2, hist2, row_params, W, init, stops, max_new, seeds)
    assert st["done"][0] == gpu.DONE_STOP and st["done"][2] == gpu.DONE_STOP
    assert int(dec2.n_active.cpu()[0]) == 0
    toy.m.close()


@pytest.mark.gpu
def test_decode_single_row_reference_defaults(gpu, torch, oracle):
    """B = 1, the CLI's defaults and seed (src/main.rs:24-31, 54), a window
    carried over from an earlier turn, the sampler's own params (no per-row
    params), logits given directly (no GEMV)."""
    V, W = 32000, 64
    rng = np.random.default_rng(12)
    steps = 60
    lg = (rng.standard_normal((steps, V)) * 3.0).astype(np.float32)
    lg[:, rng.integers(0, V, 5)] += 10.0
    init = [rng.integers(0, V, 64).astype(np.uint32)]
    stops = [int(oracle.decode_trace(lg, *DEFAULTS, W, init[0], 42)[33])]
    sampler = gpu.Sampler(*DEFAULTS, seed=42)
    dec = gpu.Decoder(1, W=W, max_new=50, stop=stops)
    dec.init(sampler, [42], init)
    d_lg = torch.from_numpy(lg).cuda()
    for t in range(steps):
        dec.step(sampler, logits=d_lg[t:t + 1])
    torch.cuda.synchronize()
    st = _check_rows(oracle, dec, lg[:, None, :], [DEFAULTS], W, init, stops, 50, [42])
    assert st["done"][0] == gpu.DONE_STOP


@pytest.mark.gpu
def test_decode_graph_replays(gpu, torch, oracle):
    """Eight steps (embed, GEMV, draw, sample, commit) captured in one HIP
    graph and replayed four times, with a host read and eager work between
    replays; every replay must leave the state the eager run left after the
    same number of steps."""
    V, cols, B, W, K, R = 32000, 1024, 3, 64, 8, 4
    toy = _Toy(gpu, torch, V, cols, seed=5)
    seeds = [42, 43, 44]
    first = [1, 2, 3]
    sampler = gpu.Sampler(*DEFAULTS, seed=1)
    sampler.reserve(B, V)

    def fresh():
        d = gpu.Decoder(B, W=W, max_new=K * R + 5, stop=())
        d.init(sampler, seeds)
        d.next.copy_(torch.tensor(first, dtype=torch.int32).cuda())
        return d

    x = torch.empty((B, cols), dtype=torch.float32, device="cuda")
    logits = torch.empty((B, V), dtype=torch.float32, device="cuda")
    eager = fresh()
    snaps = []
    for r in range(R):
        for _ in range(K):
            toy.embed(torch, eager.next, x)
            eager.step(sampler, logits=logits, lm_head=toy.m, x=x)
        torch.cuda.synchronize()
        snaps.append((eager.row_state(), eager.generated.cpu().numpy().copy(), eager.window.cpu().numpy().copy()))

    dec = fresh()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):                      # warm-up on the capture stream
        toy.embed(torch, dec.next, x)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    dec.init(sampler, seeds)
    dec.next.copy_(torch.tensor(first, dtype=torch.int32).cuda())
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        s = torch.cuda.current_stream()
        for _ in range(K):
            toy.embed(torch, dec.next, x)
            dec.step(sampler, logits=logits, lm_head=toy.m, x=x, stream=s)
    torch.cuda.synchronize()
    # capture recorded the launches without running them: the state is still fresh
    assert int(dec.row_state()["n_gen"].sum()) == 0
    junk = torch.randn(1 << 20, device="cuda")
    for r in range(R):
        g.replay()
        torch.cuda.synchronize()
        st, gen, win = dec.row_state(), dec.generated.cpu().numpy(), dec.window.cpu().numpy()
        want = snaps[r]
        assert np.array_equal(st, want[0]), (r, st, want[0])
        assert np.array_equal(gen, want[1]), r
        assert np.array_equal(win, want[2]), r
        junk.mul_(1.0001).add_(0.5)                    # eager work between replays
        torch.cuda.synchronize()
    # and the eager run itself is the reference loop
    toy.m.close()


@pytest.mark.gpu
def test_decode_commit_entry_and_errors(gpu, torch, oracle):
    """gs_decode_commit after the caller's own gs_sample_batch gives the same
    state as gs_decode_step; a NaN logit ends its row with GS_DONE_ERROR and
    n_active counts the rows still running."""
    V, B, W, steps = 50000, 2, 64, 12
    rng = np.random.default_rng(9)
    lg = (rng.standard_normal((steps, B, V)) * 3).astype(np.float32)
    lg[5, 1, 1234] = np.nan
    d_lg = torch.from_numpy(lg).cuda()
    sampler = gpu.Sampler(*DEFAULTS, seed=1)
    sampler.reserve(B, V)
    a = gpu.Decoder(B, W=W, max_new=100)
    b = gpu.Decoder(B, W=W, max_new=100)
    a.init(sampler, [42, 43])
    b.init(sampler, [42, 43])
    lib = gpu.load_library()
    for t in range(steps):
        a.step(sampler, logits=d_lg[t])
        sampler.sample_batch(d_lg[t], b.tokens, recent=b.window, recent_len=b.window_len, u=b.u, status=b.status)
        assert lib.gs_decode_commit(sampler._h, None, ctypes.byref(b.ctx), None) == 0
    torch.cuda.synchronize()
    sa, sb = a.row_state(), b.row_state()
    assert np.array_equal(sa, sb)
    assert sa["done"][1] == gpu.DONE_ERROR and sa["n_gen"][1] == 5 and sa["done"][0] == gpu.DONE_RUNNING
    assert int(a.n_active.cpu()[0]) == 1 and int(b.n_active.cpu()[0]) == 1
    assert np.array_equal(a.generated.cpu().numpy(), b.generated.cpu().numpy())
    o = oracle.generate(lg[:, 0], DEFAULTS, W, [], [], 100, 42)
    assert np.array_equal(a.generated_ids()[0], o["sampled"].astype(np.uint32))


@pytest.mark.gpu
def test_decode_large_vocab_split_rows(gpu, torch, oracle):
    """A large vocabulary (V = 152064), a few rows, uniform params: the
    decode step's sampler takes the split top-k path (chunk selection over
    the chip, then the virtual row).  Tokens, stop reasons, LCG states and
    windows must equal the oracle's loop over the same logits; a captured
    graph of the same steps must reproduce the eager run."""
    V, cols, B, W, max_new, steps = 152064, 256, 3, 64, 14, 16
    import workloads
    blocks = workloads.synth_qblocks(gpu.QTYPE_Q6_K, V, cols, seed=31)
    m = gpu.QMatrix(gpu.QTYPE_Q6_K, blocks, V, cols)
    g = torch.Generator(device="cuda")
    g.manual_seed(7)
    E = torch.randn((V, cols), generator=g, device="cuda") * 0.2
    sampler = gpu.Sampler(*DEFAULTS, seed=1)
    sampler.reserve(B, V)
    seeds = [42, 5, 77]
    rng = np.random.default_rng(8)
    init = [np.concatenate([[1023, 1024, 1024, V - 1], rng.integers(0, V, 20)]).astype(np.uint32),
            np.zeros(0, np.uint32), rng.integers(0, V, 64).astype(np.uint32)]
    x = torch.empty((B, cols), dtype=torch.float32, device="cuda")
    logits = torch.empty((B, V), dtype=torch.float32, device="cuda")

    def run(dec, stops, capture=False):
        dec.init(sampler, seeds, init)
        dec.next.copy_(torch.tensor([3, 4, 5], dtype=torch.int32).cuda())
        hist = torch.empty((steps, B, V), dtype=torch.float32, device="cuda")
        for t in range(steps):
            torch.index_select(E, 0, dec.next, out=x)
            dec.step(sampler, logits=logits, lm_head=m, x=x)
            hist[t].copy_(logits)
        torch.cuda.synchronize()
        return hist.cpu().numpy()

    dec = gpu.Decoder(B, W=W, max_new=max_new)
    hist = run(dec, [])
    _check_rows(oracle, dec, hist, [DEFAULTS] * B, W, init, [], max_new, seeds)
    g1 = dec.generated_ids()
    stops = [int(g1[1][6]), V + 1]
    dec2 = gpu.Decoder(B, W=W, max_new=max_new, stop=stops)
    hist2 = run(dec2, stops)
    st = _check_rows(oracle, dec2, hist2, [DEFAULTS] * B, W, init, stops, max_new, seeds)
    assert st["done"][1] == gpu.DONE_STOP
    # the same steps in a graph, replayed twice
    dec3 = gpu.Decoder(B, W=W, max_new=max_new, stop=stops)
    s_ = torch.cuda.Stream()
    s_.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s_):
        torch.index_select(E, 0, dec3.next, out=x)
    torch.cuda.current_stream().wait_stream(s_)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        cs = torch.cuda.current_stream()
        for t in range(steps):
            torch.index_select(E, 0, dec3.next, out=x)
            dec3.step(sampler, logits=logits, lm_head=m, x=x, stream=cs)
    for rep in range(2):
        dec3.init(sampler, seeds, init)
        dec3.next.copy_(torch.tensor([3, 4, 5], dtype=torch.int32).cuda())
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert np.array_equal(dec3.row_state(), dec2.row_state()), rep
        assert np.array_equal(dec3.generated.cpu().numpy(), dec2.generated.cpu().numpy()), rep
    m.close()


@pytest.mark.gpu
def test_decode_optional_buffers(gpu, torch, oracle):
    """gs_decode_step with no window (W = 0), no generated ids, no next
    tokens, no statuses and no active count; rows on the full-vocabulary path
    (top_k = 0) and on the split path (V > 32768, k = 40)."""
    lib = gpu.load_library()
    for V, params in ((40000, (1.0, 0, 0.9, 1.0)), (50000, (0.8, 40, 0.95, 1.0))):
        B, steps = 2, 6
        rng = np.random.default_rng(V)
        lg = (rng.standard_normal((steps, B, V)) * 2).astype(np.float32)
        d_lg = torch.from_numpy(lg).cuda()
        sampler = gpu.Sampler(*params, seed=1)
        sampler.reserve(B, V)
        rows = torch.zeros(B * 24, dtype=torch.uint8, device="cuda")
        u = torch.zeros(B, dtype=torch.float32, device="cuda")
        tok = torch.zeros(B, dtype=torch.int32, device="cuda")
        ctx = gpu.DecodeCtx(B, rows.data_ptr(), None, 0, 0, None, None, 0, 1000, None, 0, None,
                            u.data_ptr(), tok.data_ptr(), None, None)
        seeds = np.array([42, 9], np.uint64)
        assert lib.gs_decode_init(sampler._h, None, ctypes.byref(ctx), seeds.ctypes.data, None, None) == 0
        toks = []
        for t in range(steps):
            assert lib.gs_decode_step(sampler._h, None, None, d_lg[t].data_ptr(), V, V, None,
                                      ctypes.byref(ctx), None) == 0
            torch.cuda.synchronize()
            toks.append(tok.cpu().numpy().astype(np.int64).copy())
        st = rows.cpu().numpy().view(gpu.decode_row_dtype())
        for b in range(B):
            o = oracle.generate(lg[:, b], params, 0, [], [], 1000, int(seeds[b]))
            assert [int(x[b]) for x in toks] == o["sampled"].tolist(), (V, b)
            assert int(st["n_gen"][b]) == steps and int(st["wpos"][b]) == 0
