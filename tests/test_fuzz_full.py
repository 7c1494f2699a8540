"""Seeded parity fuzz of the exact full-vocabulary path (top_k = 0 rows; the
kernel that replays src/sampler.rs:53-78 without sorting the row) aimed at
its hard row shapes, against the oracle on the same inputs:

  pow2     S = sum of expf(y - max) just above a power of two (the last
           binade crossing of the running sum falls in the dense tail);
  deep     draws u in [0.9, 1) into a wide nucleus;
  grid     logits on a 1/4 grid: many exact ties of y, and of the summands;
  spikes   spikes inside a penalty window (rep in [1.1, 1.3]);
  flat     a near-uniform row (a huge nucleus, tiny summands);
  mixed    T, top_p (including 1.0: no nucleus) and u drawn per row.

V in {4099, 50000, 152064, 256000}.  Each case is fixed by its seed (the
inputs are regenerated from it, so a failing seed is a CPU-reproducible
fixture: rerun make_case(seed) against the oracle).  Tokens must be
identical; the rows the binned path hands to the sort path are counted and
reported (their tokens are checked too)."""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

SHAPES = ["pow2", "deep", "grid", "spikes", "flat", "mixed"]
VS = [4099, 50000, 152064, 256000]
ROWS = 16
W = 64


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _pow2_row(rng, V, T):
    """Logits whose f32 softmax sum S lies just above 2^n: the top logit is
    raised by delta so that 1 + R exp(-delta) = 2^n (1 + eps)."""
    x = (rng.standard_normal(V) * rng.uniform(1.0, 3.0)).astype(np.float32)
    y = x.astype(np.float64) / T
    i = int(np.argmax(y))
    rest = np.delete(y, i)
    R = float(np.exp(rest - y[i]).sum())
    n = int(np.floor(np.log2(1.0 + R)))
    eps = rng.choice([1e-7, 1e-6, 1e-5, 1e-4, 1e-3])
    target = 2.0 ** n * (1.0 + eps)
    delta = np.log(R / (target - 1.0)) if 0.0 < target - 1.0 < R else 0.0
    x[i] = np.float32((y[i] + delta) * T)
    return x


def make_case(seed, V, shape):
    """B = ROWS rows of one shape: (logits, params, u, recent)."""
    import workloads
    rng = np.random.default_rng(seed)
    B = ROWS
    lg = np.empty((B, V), np.float32)
    T = np.ones(B, np.float32)
    p = np.full(B, 0.95, np.float32)
    rep = np.ones(B, np.float32)
    u = rng.random(B, dtype=np.float32)
    rec = rng.integers(0, V, (B, W)).astype(np.uint32)
    for b in range(B):
        if shape == "pow2":
            T[b] = rng.choice([0.7, 1.0, 1.3])
            p[b] = rng.choice([0.9, 0.95, 0.99, 1.0])
            lg[b] = _pow2_row(rng, V, float(T[b]))
        elif shape == "deep":
            lg[b] = rng.standard_normal(V).astype(np.float32) * rng.uniform(1.0, 2.5)
            p[b] = rng.uniform(0.9, 0.999)
            u[b] = np.float32(rng.uniform(0.9, 1.0))
        elif shape == "grid":
            lg[b] = (rng.integers(-48, 24, V) / 4.0).astype(np.float32)
            T[b] = rng.choice([1.0, 0.5, 0.8])
            p[b] = rng.uniform(0.5, 1.0)
        elif shape == "spikes":
            lg[b] = rng.standard_normal(V).astype(np.float32) * 3.0
            pos = rng.choice(V, 8, replace=False)
            lg[b, pos] += rng.uniform(5, 12, 8).astype(np.float32)
            rec[b, :16] = np.repeat(pos[:4], 4)     # spikes penalized, several times
            rep[b] = rng.uniform(1.1, 1.3)
            T[b] = rng.uniform(0.5, 1.5)
            p[b] = rng.uniform(0.5, 1.0)
        elif shape == "flat":
            lg[b] = (rng.standard_normal(V) * 0.05).astype(np.float32)
            p[b] = rng.uniform(0.5, 0.99)
        else:
            lg[b] = rng.standard_normal(V).astype(np.float32) * rng.uniform(0.5, 4.0)
            T[b] = rng.uniform(0.3, 2.0)
            p[b] = rng.choice([rng.uniform(0.3, 1.0), 1.0])
            rep[b] = rng.choice([1.0, rng.uniform(0.8, 1.5)])
    params = workloads.params_rows(zip(T, np.zeros(B, np.uint32), p, rep))
    return lg, params, u, rec


@pytest.mark.parametrize("V", VS)
def test_full_vocab_fuzz(gpu, torch, oracle, V):
    total = fb_total = 0
    for si, shape in enumerate(SHAPES):
        seed = 7000 + 97 * VS.index(V) + si
        lg, params, u, rec = make_case(seed, V, shape)
        _say("fuzz V", V, "shape", shape, "seed", seed)
        B = lg.shape[0]
        d_lg = torch.from_numpy(lg).cuda()
        d_pr = torch.from_numpy(np.ascontiguousarray(params).view(np.uint8)).cuda()
        d_u = torch.from_numpy(u).cuda()
        d_rec = torch.from_numpy(rec.view(np.int32)).cuda()
        d_tok = torch.zeros(B, dtype=torch.int32, device="cuda")
        d_st = torch.full((B,), 99, dtype=torch.int32, device="cuda")
        s = gpu.Sampler(1.0, 0, 0.95, 1.0, seed=1)
        s.sample_batch(d_lg, d_tok, params=d_pr, recent=d_rec, u=d_u, status=d_st)
        torch.cuda.synchronize()
        fb = s.fallback_rows()
        got = d_tok.cpu().numpy().astype(np.int64)
        st = d_st.cpu().numpy()
        want = oracle.sample_batch(lg, params, u, recent=rec, nthreads=16)
        assert (st == 0).all(), (shape, seed, st)
        bad = np.nonzero(got != want)[0]
        assert bad.size == 0, "V %d shape %s seed %d: rows %s got %s want %s" % (
            V, shape, seed, bad[:8], got[bad[:8]], want[bad[:8]])
        total += B
        fb_total += fb
        _say("  rows", B, "sort-path rows", fb)
    _say("V", V, "rows checked", total, "sent to the sort path", fb_total)
