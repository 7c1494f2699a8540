"""The chunked top-k path: batches of fewer rows than CUs whose rows have
V > 32768 and 0 < k <= 128 are cut into balanced chunks of at most 32768
logits; each chunk keeps its best round_up(k, 4) (penalized, in index
order) and a second kernel samples the virtual rows.  Tokens must equal the
oracle's on the same rows and draws: per-row params (rows of other kinds in
the same batch take the other paths), ties on a grid and all-equal rows
(the index order decides), penalty ids on chunk edges, duplicates and ids
>= V, extreme temperatures and a NaN row."""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _rows(rng, B, V, shape):
    if shape == "normal":
        return (rng.standard_normal((B, V)) * 2.5).astype(np.float32)
    if shape == "grid":
        return (rng.integers(-40, 40, size=(B, V)) / 4.0).astype(np.float32)
    if shape == "equal":
        return np.full((B, V), 0.75, np.float32)
    x = (rng.standard_normal((B, V)) * 0.5).astype(np.float32)
    for b in range(B):
        x[b, rng.integers(0, V, 40)] += rng.uniform(5, 12, 40).astype(np.float32)
    return x


def _edges(V, nch):
    return [(c * V) // nch for c in range(1, nch)]


@pytest.mark.parametrize("V,B,shape", [
    (32772, 40, "normal"),      # two chunks, just above the register row
    (65537, 9, "grid"),         # odd V: unaligned rows, three chunks
    (128256, 64, "spike"),      # C2's shape
    (200003, 255, "normal"),    # one row short of the CU count
    (262144, 17, "equal"),      # the largest vocabulary the path takes (8 chunks)
])
def test_chunked_rows(gpu, torch, oracle, V, B, shape):
    import workloads
    rng = np.random.default_rng(V + B)
    x = _rows(rng, B, V, shape)
    nch = -(-V // 32768)
    W = 96
    rec = rng.integers(0, V, size=(B, W)).astype(np.uint32)
    e = _edges(V, nch)
    rec[:, :6] = [e[0] - 1, e[0], e[0], e[-1], V - 1, V + 3]      # chunk edges, a duplicate, ids >= V
    rec[:, 6:12] = rec[:, 12:18]
    ks = np.array([1, 4, 40, 127, 128, 5, 0, 129][:] * (B // 8 + 1), np.uint32)[:B]   # 0 / 129: other paths
    T = rng.choice([0.7, 1.0, 1.3, 1e-3, 40.0], B).astype(np.float32)
    T[::11] = 0.0                                                    # greedy rows
    p = rng.choice([0.5, 0.9, 1.0], B).astype(np.float32)
    rep = rng.choice([1.0, 1.15, 2.0], B).astype(np.float32)
    params = workloads.params_rows(zip(T, ks, p, rep))
    u = rng.random(B).astype(np.float32)
    u[0] = 0.0
    _say("chunked V", V, "B", B, shape, "chunks", nch)
    d_lg = torch.from_numpy(x).cuda()
    d_pr = torch.from_numpy(np.ascontiguousarray(params).view(np.uint8)).cuda()
    d_rec = torch.from_numpy(rec.view(np.int32)).cuda()
    d_u = torch.from_numpy(u).cuda()
    tok = torch.zeros(B, dtype=torch.int32, device="cuda")
    st = torch.full((B,), 99, dtype=torch.int32, device="cuda")
    s = gpu.Sampler(0.7, 40, 0.9, 1.1, seed=1)
    s.sample_batch(d_lg, tok, params=d_pr, recent=d_rec, u=d_u, status=st)
    torch.cuda.synchronize()
    got = tok.cpu().numpy().astype(np.int64)
    assert (st.cpu().numpy() == 0).all()
    want = oracle.sample_batch(x, params, u, recent=rec, nthreads=16, fast_topk=True)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, (bad[:8], got[bad[:8]], want[bad[:8]], ks[bad[:8]], T[bad[:8]])
    # uniform params: every row on the chunked path (k = 40)
    s.sample_batch(d_lg, tok, recent=d_rec, u=d_u, status=st)
    torch.cuda.synchronize()
    want_u = oracle.sample_batch(x, [(0.7, 40, 0.9, 1.1)] * B, u, recent=rec, nthreads=16, fast_topk=True)
    assert np.array_equal(tok.cpu().numpy().astype(np.int64), want_u)


def test_chunked_nan_row(gpu, torch, oracle):
    """A NaN in any chunk makes its row an error and leaves the others."""
    rng = np.random.default_rng(2)
    V, B = 100000, 6
    x = (rng.standard_normal((B, V)) * 2).astype(np.float32)
    x[2, 99999] = np.nan
    x[4, 33333] = np.nan
    u = rng.random(B).astype(np.float32)
    d_lg = torch.from_numpy(x).cuda()
    tok = torch.zeros(B, dtype=torch.int32, device="cuda")
    st = torch.zeros(B, dtype=torch.int32, device="cuda")
    s = gpu.Sampler(0.8, 20, 0.9, 1.0, seed=1)
    s.sample_batch(d_lg, tok, u=torch.from_numpy(u).cuda(), status=st)
    torch.cuda.synchronize()
    stv = st.cpu().numpy()
    assert list(stv) == [0, 0, gpu.GS_ERR_NAN, 0, gpu.GS_ERR_NAN, 0], stv
    ok = [0, 1, 3, 5]
    want = oracle.sample_batch(x[ok], [(0.8, 20, 0.9, 1.0)] * 4, u[ok], nthreads=4, fast_topk=True)
    assert np.array_equal(tok.cpu().numpy()[ok].astype(np.int64), want)


def test_chunked_graph_replays(gpu, torch, oracle):
    """The one-launch chunked path in a HIP graph: its per-row chunk counters
    return to zero after every call, so each replay (new logits copied in
    between, eager calls on other batches between the replays) samples
    exactly.  Rows of both kinds (per-row params) and a row whose chunks
    fall back to the whole row (all equal)."""
    import workloads
    rng = np.random.default_rng(77)
    V, B = 131072, 12
    params = workloads.params_rows([(0.8, k, 0.9, 1.2) for k in (40, 128, 1, 7, 0, 200, 40, 64, 3, 100, 40, 2)])
    rec = rng.integers(0, V, size=(B, 64)).astype(np.uint32)
    u = rng.random(B).astype(np.float32)
    d_lg = torch.zeros((B, V), dtype=torch.float32, device="cuda")
    d_pr = torch.from_numpy(np.ascontiguousarray(params).view(np.uint8)).cuda()
    d_rec = torch.from_numpy(rec.view(np.int32)).cuda()
    d_u = torch.from_numpy(u).cuda()
    tok = torch.zeros(B, dtype=torch.int32, device="cuda")
    s = gpu.Sampler(0.7, 40, 0.9, 1.1, seed=1)
    s.reserve(B, V)
    s.sample_batch(d_lg, tok, params=d_pr, recent=d_rec, u=d_u)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        s.sample_batch(d_lg, tok, params=d_pr, recent=d_rec, u=d_u)
    other = torch.randn((5, V), device="cuda")
    tother = torch.zeros(5, dtype=torch.int32, device="cuda")
    for rep in range(4):
        x = (rng.standard_normal((B, V)) * 2.5).astype(np.float32)
        x[3] = 0.5                                    # the bound cannot be decided: whole-row fallback
        d_lg.copy_(torch.from_numpy(x))
        _say("chunked graph replay", rep)
        tok.fill_(-1)
        g.replay()
        torch.cuda.synchronize()
        want = oracle.sample_batch(x, params, u, recent=rec, nthreads=12, fast_topk=True)
        assert np.array_equal(tok.cpu().numpy().astype(np.int64), want), rep
        s.sample_batch(other, tother, recent=d_rec[:5], u=d_u[:5])   # eager, uniform params, same sampler
        torch.cuda.synchronize()


@pytest.mark.parametrize("V,B", [(524288, 3), (524292, 2)])
def test_chunked_widest_and_window_lengths(gpu, torch, oracle, V, B):
    """The widest virtual row of the one-launch form (16 chunks of 32768,
    k = 128: 2048 entries) and the first vocabulary beyond it (17 chunks: the
    two-launch form), with per-row window lengths (recent_len) and a window
    of 1024 ids."""
    import workloads
    rng = np.random.default_rng(V)
    x = (rng.standard_normal((B, V)) * 2.0).astype(np.float32)
    W = 1024
    rec = rng.integers(0, V, size=(B, W)).astype(np.uint32)
    rec[:, :8] = [0, 32767, 32768, V - 1, V - 1, V + 1, 65535, 65536]
    rl = np.array([W, 17, 0][:B], np.uint32)
    params = workloads.params_rows([(0.9, 128, 0.95, 1.3), (0.6, 3, 0.5, 1.05), (1.4, 64, 1.0, 2.0)][:B])
    u = rng.random(B).astype(np.float32)
    d_lg = torch.from_numpy(x).cuda()
    d_pr = torch.from_numpy(np.ascontiguousarray(params).view(np.uint8)).cuda()
    d_rec = torch.from_numpy(rec.view(np.int32)).cuda()
    d_rl = torch.from_numpy(rl.view(np.int32)).cuda()
    tok = torch.zeros(B, dtype=torch.int32, device="cuda")
    st = torch.full((B,), 99, dtype=torch.int32, device="cuda")
    s = gpu.Sampler(0.7, 40, 0.9, 1.1, seed=1)
    _say("chunked widest V", V, "B", B)
    s.sample_batch(d_lg, tok, params=d_pr, recent=d_rec, recent_len=d_rl, u=torch.from_numpy(u).cuda(), status=st)
    torch.cuda.synchronize()
    assert (st.cpu().numpy() == 0).all()
    want = oracle.sample_batch(x, params, u, recent=rec, recent_len=rl, nthreads=8, fast_topk=True)
    assert np.array_equal(tok.cpu().numpy().astype(np.int64), want)
