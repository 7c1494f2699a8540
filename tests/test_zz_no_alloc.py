"""gs_sample_batch_noalloc (static scratch, no device allocation) against
gs_sample_batch on the same inputs, through the C ABI: two calls in a row on
each path, the second with a smaller batch, tokens and statuses identical
(and equal to the oracle's)."""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _call(gs, torch, s, x, params, u, recent, noalloc):
    B, V = x.shape
    d_lg = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    d_u = torch.from_numpy(np.ascontiguousarray(u, dtype=np.float32)).cuda()
    d_pr = torch.from_numpy(np.ascontiguousarray(params).view(np.uint8)).cuda()
    d_rec = None
    if recent is not None:
        d_rec = torch.from_numpy(np.ascontiguousarray(recent, dtype=np.uint32).view(np.int32)).cuda()
    d_tok = torch.full((B,), -1, dtype=torch.int32, device="cuda")
    d_st = torch.full((B,), 99, dtype=torch.int32, device="cuda")
    s.sample_batch(d_lg, d_tok, params=d_pr, recent=d_rec, u=d_u, status=d_st, noalloc=noalloc)
    torch.cuda.synchronize()
    return d_tok.cpu().numpy().astype(np.int64), d_st.cpu().numpy()


def _case(rng, B, V, kind):
    import workloads
    x = (rng.standard_normal((B, V), dtype=np.float32) * 2.5).astype(np.float32)
    x[np.arange(B), rng.integers(0, V, B)] += np.float32(7.0)
    if kind == "full":       # full-vocabulary rows (top_k = 0): the path with the largest scratch
        rows = [(float(rng.choice([0.8, 1.0])), 0, float(rng.choice([0.9, 0.95, 1.0])),
                 float(rng.choice([1.0, 1.2]))) for _ in range(B)]
    elif kind == "topk":
        rows = [(0.7, 40, 0.9, 1.1)] * B
    else:                    # heterogeneous: greedy, top-1, top-k and full rows in one call
        rows = [(float(rng.choice([0.0, 0.6, 1.3])), int(rng.choice([0, 1, 20, 100])),
                 float(rng.uniform(0.5, 1.0)), float(rng.uniform(1.0, 1.3))) for _ in range(B)]
    params = np.array(rows, dtype=workloads.PARAMS_DTYPE)
    u = rng.random(B, dtype=np.float32)
    recent = rng.integers(0, V, size=(B, 64), dtype=np.uint32)
    return x, params, u, recent


@pytest.mark.parametrize("kind,V,B1,B2", [("full", 152064, 6, 2), ("topk", 128256, 8, 3),
                                          ("mixed", 50000, 12, 5)])
def test_noalloc_matches_batch(gpu, torch, oracle, kind, V, B1, B2):
    rng = np.random.default_rng(V + B1)
    s_ref = gpu.Sampler(0.7, 40, 0.9, 1.1, seed=1)
    s_na = gpu.Sampler(0.7, 40, 0.9, 1.1, seed=1)
    for B in (B1, B2):                         # the second call is smaller
        x, params, u, recent = _case(rng, B, V, kind)
        _say("noalloc", kind, "V", V, "B", B)
        want_tok, want_st = _call(gpu, torch, s_ref, x, params, u, recent, noalloc=False)
        got_tok, got_st = _call(gpu, torch, s_na, x, params, u, recent, noalloc=True)
        assert (got_st == want_st).all(), (got_st, want_st)
        assert (got_tok == want_tok).all(), (got_tok, want_tok)
        ora = oracle.sample_batch(x, params, u, recent=recent, nthreads=8)
        assert (got_tok == ora).all(), (got_tok, ora)


def test_noalloc_rejects_oversize(gpu, torch):
    """A batch whose scratch exceeds the static array is refused, not run."""
    s = gpu.Sampler(1.0, 0, 0.95, 1.0, seed=1)
    V, B = 152064, 64                          # full-vocabulary scratch of 64 rows > 64 MiB
    d_lg = torch.zeros((B, V), dtype=torch.float32, device="cuda")
    d_u = torch.zeros(B, dtype=torch.float32, device="cuda")
    d_tok = torch.zeros(B, dtype=torch.int32, device="cuda")
    with pytest.raises(gpu.SamplerError) as e:
        s.sample_batch(d_lg, d_tok, u=d_u, noalloc=True)
    assert e.value.code == gpu.GS_ERR_UNSUPPORTED


def test_noalloc_topk_large_batch(gpu, torch, oracle):
    """Top-k rows with the sampler's own params (no d_params) need no
    full-vocabulary scratch: C5's shape (B = 1024, V = 152064, k = 50,
    1024-id windows) fits the static array, on two calls in a row, the second
    smaller, with the same tokens as gs_sample_batch and the oracle."""
    import workloads
    V = 152064
    rng = np.random.default_rng(1024)
    s_ref = gpu.Sampler(0.7, 50, 0.9, 1.3, seed=1)
    s_na = gpu.Sampler(0.7, 50, 0.9, 1.3, seed=1)
    for B in (1024, 300):
        x = (rng.standard_normal((B, V), dtype=np.float32) * 3.0).astype(np.float32)
        u = rng.random(B, dtype=np.float32)
        recent = rng.integers(0, V, size=(B, 1024), dtype=np.uint32)
        d_lg = torch.from_numpy(x).cuda()
        d_u = torch.from_numpy(u).cuda()
        d_rec = torch.from_numpy(recent.view(np.int32)).cuda()
        _say("noalloc topk V", V, "B", B)
        out = []
        for s, na in ((s_ref, False), (s_na, True)):
            d_tok = torch.full((B,), -1, dtype=torch.int32, device="cuda")
            d_st = torch.full((B,), 99, dtype=torch.int32, device="cuda")
            s.sample_batch(d_lg, d_tok, recent=d_rec, u=d_u, status=d_st, noalloc=na)
            torch.cuda.synchronize()
            out.append((d_tok.cpu().numpy().astype(np.int64), d_st.cpu().numpy()))
        (want_tok, want_st), (got_tok, got_st) = out
        assert (got_st == 0).all() and (want_st == 0).all()
        assert (got_tok == want_tok).all()
        params = np.array([(0.7, 50, 0.9, 1.3)] * B, dtype=workloads.PARAMS_DTYPE)
        ora = oracle.sample_batch(x, params, u, recent=recent, nthreads=8)
        assert (got_tok == ora).all(), np.nonzero(got_tok != ora)
