"""The caller-visible mutation of src/sampler.rs:37,41: after sample() the
reference leaves `logits` penalized (once per window occurrence, :23-30) and,
when T > 0, divided by T.  gs_sample_mut (single row, host or device) and
gs_logits_writeback (batched, device) must leave the row bit for bit as the
oracle's restatement of sample() leaves its copy (detail['logits'])."""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


CASES = [
    # (T, k, p, rep, window kind)
    (0.7, 40, 0.9, 1.1, "dups"),
    (1.3, 0, 0.95, 1.3, "dups"),
    (0.0, 40, 0.9, 1.2, "dups"),        # greedy: penalty only, no division (:39)
    (-1.0, 0, 1.0, 1.2, "plain"),
    (0.5, 1, 1.0, -1.0, "dups"),       # negative penalty: the sign flips per occurrence
    (0.9, 20, 0.8, 1.0, "dups"),       # rep == 1: no penalty (:24)
    (2.0, 100, 0.5, 0.0, "edge"),      # zero penalty; ids >= V ignored (:26)
    (1e-30, 5, 0.9, 1.1, "plain"),     # T tiny: +-inf after the division
]


def _window(kind, V, rng, W=64):
    if kind == "plain":
        return rng.integers(0, V, W).astype(np.uint32)
    if kind == "dups":
        w = rng.integers(0, V, W).astype(np.uint32)
        w[W // 2:] = w[:W - W // 2]          # every id at least twice
        w[-3:] = w[0]
        return w
    w = rng.integers(0, V, W).astype(np.uint32)
    w[:4] = [V, V + 7, 0xFFFFFFFF, V - 1]
    return w


@pytest.mark.parametrize("where", ["host", "device"])
@pytest.mark.parametrize("case", range(len(CASES)))
def test_sample_mut_single_row(gpu, torch, oracle, where, case):
    T, k, p, rep, kind = CASES[case]
    V = 32000 if case % 2 == 0 else 50021
    rng = np.random.default_rng(100 + case)
    lg = (rng.standard_normal(V) * 3).astype(np.float32)
    lg[rng.integers(0, V, 5)] += 10.0
    lg[:8] = [0.0, -0.0, 1e-38, -1e-38, 3e38, -3e38, 1.0, -1.0]
    win = _window(kind, V, rng)
    win[:2] = [0, 1]                          # the +-0 entries are penalized
    _say("sample_mut", where, case, "V", V, "T", T, "rep", rep)
    s = gpu.Sampler(T, k, p, rep, seed=77)
    st0 = s.state
    want_tok, det = oracle.sample(lg, T, k, p, rep, recent=win, state=st0, detail=True)
    if where == "host":
        row = lg.copy()
        tok = s.sample_mut(row, win)
        got = row
    else:
        d = torch.from_numpy(lg.copy()).cuda()
        tok = s.sample_mut(d, torch.from_numpy(win.view(np.int32)).cuda())
        got = d.cpu().numpy()
    assert tok == want_tok
    assert s.state == det["state"] if T > 0 else s.state == st0
    assert np.array_equal(got.view(np.uint32), det["logits"].view(np.uint32)), \
        np.nonzero(got.view(np.uint32) != det["logits"].view(np.uint32))[0][:8]


def test_logits_writeback_batch(gpu, torch, oracle):
    """C4-shaped batch: heterogeneous per-row T, k, p, rep over 256-id
    windows with per-row lengths, V = 256000 (the config's vocabulary),
    64 rows; ld > V."""
    import workloads
    w = workloads.make("c4", B=64, seed=5)
    lg, prm, rec = w["logits"], w["params"], w["recent"]
    B, V = lg.shape
    ld = V + 64
    buf = np.zeros((B, ld), np.float32)
    buf[:, :V] = lg
    buf[:, V:] = 7.0                                  # past V: never touched
    rng = np.random.default_rng(3)
    rlen = rng.integers(0, rec.shape[1] + 1, B).astype(np.uint32)
    rlen[:4] = [0, rec.shape[1], 1, 255]
    prm = prm.copy()
    prm["temperature"][:3] = [0.0, -0.5, 1.0]
    _say("writeback batch B", B, "V", V, "ld", ld)
    d_lg = torch.from_numpy(buf.copy()).cuda()
    d_rec = torch.from_numpy(np.ascontiguousarray(rec).view(np.int32)).cuda()
    d_len = torch.from_numpy(rlen.view(np.int32)).cuda()
    d_pr = torch.from_numpy(np.ascontiguousarray(prm).view(np.uint8)).cuda()
    d_u = torch.from_numpy(w["u"]).cuda()
    d_tok = torch.zeros(B, dtype=torch.int32, device="cuda")
    d_st = torch.zeros(B, dtype=torch.int32, device="cuda")
    s = gpu.Sampler(0.7, 40, 0.9, 1.1, seed=1)
    view = d_lg[:, :V]
    s.sample_batch(view, d_tok, params=d_pr, recent=d_rec, recent_len=d_len, u=d_u, status=d_st, ld=ld)
    s.logits_writeback(view, params=d_pr, recent=d_rec, recent_len=d_len, ld=ld)
    torch.cuda.synchronize()
    got = d_lg.cpu().numpy()
    tok = d_tok.cpu().numpy().astype(np.int64)
    assert (got[:, V:] == 7.0).all()
    for b in range(B):
        pr = prm[b]
        wt, det = oracle.sample(lg[b], float(pr["temperature"]), int(pr["top_k"]), float(pr["top_p"]),
                                float(pr["rep_penalty"]), recent=rec[b, :rlen[b]], r=float(w["u"][b]),
                                fast_topk=True, detail=True)
        assert tok[b] == wt, b
        assert np.array_equal(got[b, :V].view(np.uint32), det["logits"].view(np.uint32)), b
