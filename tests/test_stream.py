"""Top-k rows longer than the register row (V > 32768, V % 4 == 0, V <=
262144, 16-byte aligned rows): the first 32768 logits sit in registers and
give the bound (the k-th largest unpenalized thread maximum of the head), the
rest of the row streams once and only elements at or above the bound join the
candidate list.  Tokens must equal the oracle's on the same rows and draws:
a tail of one float4, penalized ids in the head and the tail holding the
row's largest logits, a full 1024-id window, ascending rows whose every tail
element passes the bound (the list overflows and the general path takes the
row), NaN in the tail or the head, -inf heads, grid ties at the bound, the
largest vocabulary the path takes and the first one it does not."""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _run(gpu, torch, x, params, u, rec=None):
    B = x.shape[0]
    d_lg = torch.from_numpy(x).cuda()
    d_pr = torch.from_numpy(np.ascontiguousarray(params).view(np.uint8)).cuda()
    d_rec = None if rec is None else torch.from_numpy(rec.view(np.int32)).cuda()
    tok = torch.zeros(B, dtype=torch.int32, device="cuda")
    st = torch.full((B,), 99, dtype=torch.int32, device="cuda")
    s = gpu.Sampler(0.7, 40, 0.9, 1.1, seed=1)
    s.sample_batch(d_lg, tok, params=d_pr, recent=d_rec, u=torch.from_numpy(u).cuda(), status=st)
    torch.cuda.synchronize()
    return tok.cpu().numpy().astype(np.int64), st.cpu().numpy()


def _check(gpu, torch, oracle, x, params, u, rec=None):
    got, st = _run(gpu, torch, x, params, u, rec)
    want = oracle.sample_batch(x, params, u, recent=rec, nthreads=16, fast_topk=True)
    err = want < 0
    assert (st[~err] == 0).all(), st
    assert (st[err] != 0).all(), (st, want)
    bad = np.nonzero((got != want) & ~err)[0]
    assert bad.size == 0, (bad[:8], got[bad[:8]], want[bad[:8]])
    return st


@pytest.mark.parametrize("V,B,shape", [
    (32772, 256, "normal"),     # one float4 past the register head
    (65544, 256, "spike"),      # spikes penalized in the head and the tail
    (152064, 260, "grid"),      # ties at the bound
    (100000, 12, "wide_k"),     # k > 128: the chunked path does not take these rows
])
def test_stream_rows(gpu, torch, oracle, V, B, shape):
    import workloads
    rng = np.random.default_rng(V + B)
    if shape == "grid":
        x = (rng.integers(-40, 40, size=(B, V)) / 4.0).astype(np.float32)
    else:
        x = (rng.standard_normal((B, V)) * 2.0).astype(np.float32)
    W = 256
    rec = rng.integers(0, V, size=(B, W)).astype(np.uint32)
    if shape == "spike":
        for b in range(B):
            pos = rng.integers(0, V, 24)
            x[b, pos] += rng.uniform(6, 14, 24).astype(np.float32)
            rec[b, :12] = pos[:12]                       # half of the spikes are penalized
    rec[:, 12] = V + 5                                   # ids >= V are skipped
    rec[:, 13] = rec[:, 14]                              # a duplicate: two penalty ops
    if shape == "wide_k":
        ks = rng.choice([129, 300, 700, 1000, 1023], B).astype(np.uint32)
    else:
        ks = rng.choice([1, 2, 20, 50, 100, 128, 400], B).astype(np.uint32)
    T = rng.choice([0.5, 0.8, 1.0, 1.7, 1e-3], B).astype(np.float32)
    p = rng.choice([0.3, 0.9, 0.99, 1.0], B).astype(np.float32)
    rep = rng.choice([1.0, 1.15, 1.5], B).astype(np.float32)
    params = workloads.params_rows(zip(T, ks, p, rep))
    u = rng.random(B).astype(np.float32)
    u[0] = 0.0
    u[1] = np.float32(1.0) - np.float32(2.0 ** -24)
    _say("stream V", V, "B", B, shape)
    _check(gpu, torch, oracle, x, params, u, rec)


def test_stream_full_window(gpu, torch, oracle):
    """1024 distinct penalized ids, all among the head's largest logits: the
    thread maxima leave them out, the table brings them back penalized."""
    import workloads
    rng = np.random.default_rng(11)
    V, B = 98304, 8
    x = (rng.standard_normal((B, V)) * 1.5).astype(np.float32)
    rec = np.empty((B, 1024), np.uint32)
    for b in range(B):
        top = np.argsort(-x[b, :32768], kind="stable")[:1024]
        rec[b] = top
    params = workloads.params_rows([(0.9, k, 0.95, r) for k, r in
                                    zip([50, 200, 1000, 129, 64, 500, 8, 300], [1.3, 1.05, 3.0, 1.3, 1.01, 1.3, 2.0, 1.3])])
    u = rng.random(B).astype(np.float32)
    _say("stream full window")
    _check(gpu, torch, oracle, x, params, u, rec)


def test_stream_overflow_ascending(gpu, torch, oracle):
    """Ascending rows: every tail element passes the head's bound, the list
    overflows and the row goes to the general path."""
    import workloads
    V, B = 70000, 6
    base = (np.arange(V, dtype=np.float32) * np.float32(1e-4))
    x = np.stack([base * np.float32(1 + 0.1 * b) for b in range(B)]).astype(np.float32)
    params = workloads.params_rows([(1.0, k, 0.9, 1.0) for k in (200, 300, 500, 1000, 150, 129)])
    u = np.linspace(0.05, 0.95, B).astype(np.float32)
    _say("stream overflow")
    _check(gpu, torch, oracle, x, params, u)


def test_stream_nan_and_neg_inf(gpu, torch, oracle):
    """A NaN in the tail or in the head makes its row an error; a head of -inf
    (the bound falls to -inf) goes to the general path."""
    import workloads
    rng = np.random.default_rng(5)
    V, B = 131072, 8
    x = (rng.standard_normal((B, V)) * 2).astype(np.float32)
    x[1, 131071] = np.nan                  # the last element of the tail
    x[3, 40000] = np.nan
    x[5, 7] = np.nan                       # in the head
    x[6, :32768] = -np.inf                 # the head gives no finite bound
    x[7, 32768:] = -np.inf                 # a tail of -inf
    params = workloads.params_rows([(0.8, 200, 0.9, 1.0)] * B)
    u = rng.random(B).astype(np.float32)
    _say("stream nan")
    st = _check(gpu, torch, oracle, x, params, u)
    assert [int(v) for v in st] == [0, gpu.GS_ERR_NAN, 0, gpu.GS_ERR_NAN, 0, gpu.GS_ERR_NAN, 0, 0], st


@pytest.mark.parametrize("V", [262144, 262148])
def test_stream_largest(gpu, torch, oracle, V):
    """The largest vocabulary of the streamed path and the first beyond it
    (that one takes the two-pass path); penalized ids near the end."""
    import workloads
    rng = np.random.default_rng(V)
    B = 6
    x = (rng.standard_normal((B, V)) * 2).astype(np.float32)
    rec = rng.integers(V - 64, V, size=(B, 64)).astype(np.uint32)
    x[:, V - 64:] += 9.0
    params = workloads.params_rows([(0.8, k, 0.9, 1.4) for k in (129, 200, 1000, 600, 300, 1023)])
    u = rng.random(B).astype(np.float32)
    _say("stream largest V", V)
    _check(gpu, torch, oracle, x, params, u, rec)


@pytest.mark.parametrize("V,B", [(65544, 520), (152064, 600), (16388, 512)])
def test_stream_rows_many(gpu, torch, oracle, V, B):
    """Batches of more than two rows per CU with the sampler's own params: a
    window of 1024 ids with per-row lengths, ids >= V and duplicates, a row
    that overflows the candidate list, a NaN row, and k = 256 on rows that
    fit the registers."""
    rng = np.random.default_rng(V + B)
    x = (rng.standard_normal((B, V)) * 2.0).astype(np.float32)
    W = 1024
    rec = rng.integers(0, V, size=(B, W)).astype(np.uint32)
    rec[:, 0] = V + 3
    rec[:, 1:5] = rec[:, 5:9]
    for b in range(0, B, 7):                                  # spikes that the window penalizes
        x[b, rec[b, 10:20]] += np.float32(9.0)
    rl = rng.integers(0, W + 1, size=B).astype(np.uint32)
    rl[::5] = W
    x[3] = np.arange(V, dtype=np.float32) * np.float32(1e-3)  # ascending: the list overflows
    x[11, V // 2] = np.nan
    u = rng.random(B).astype(np.float32)
    T, k, p, rep = 0.7, 50, 0.9, 1.3
    if V == 16388:
        k = 256
    d_lg = torch.from_numpy(x).cuda()
    d_rec = torch.from_numpy(rec.view(np.int32)).cuda()
    d_rl = torch.from_numpy(rl.view(np.int32)).cuda()
    tok = torch.zeros(B, dtype=torch.int32, device="cuda")
    st = torch.full((B,), 99, dtype=torch.int32, device="cuda")
    s = gpu.Sampler(T, k, p, rep, seed=1)
    _say("stream many rows V", V, "B", B, "k", k)
    s.sample_batch(d_lg, tok, recent=d_rec, recent_len=d_rl, u=torch.from_numpy(u).cuda(), status=st)
    torch.cuda.synchronize()
    want = oracle.sample_batch(x, [(T, k, p, rep)] * B, u, recent=rec, recent_len=rl, nthreads=16, fast_topk=True)
    got, stv = tok.cpu().numpy().astype(np.int64), st.cpu().numpy()
    err = want < 0
    assert list(np.nonzero(err)[0]) == [11], np.nonzero(err)[0]
    assert stv[11] == gpu.GS_ERR_NAN and (stv[~err] == 0).all(), stv
    bad = np.nonzero((got != want) & ~err)[0]
    assert bad.size == 0, (bad[:8], got[bad[:8]], want[bad[:8]])
