"""The reference's intermediate results (src/sampler.rs:44-78) through
gs_sample_detail: for every row, the kept candidates after truncate(top_k)
in sorted order (ids bit-exact), their post-softmax probabilities a_j / S
(within 1e-5 relative, the stated tolerance; expected bit-exact), the count
kept, the nucleus cut, S and s2 (bit-exact), the token, and the per-row tie
flag (equal scaled logits at rank k, inside the kept prefix or at the cut),
against the oracle's detail output on the same inputs.  C2, C3 and C4 rows."""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def oracle_ties(y, n, cut, tok):
    """bit 0: equal values meeting inside [0, cut] of the sorted order, or at
    rank n (the truncation boundary); bit 1: the token's value is shared by
    another element.  y: scaled logits (the oracle's mutated row)."""
    V = y.size
    order = np.lexsort((np.arange(V), -y.astype(np.float64)))
    ys = y[order]
    hi = min(cut, V - 1)
    tie = int((ys[:hi] == ys[1:hi + 1]).any())
    if n < V:
        tie |= int(ys[n - 1] == ys[n])
    pos = int(np.nonzero(order == tok)[0][0])
    if (pos > 0 and ys[pos - 1] == ys[pos]) or (pos + 1 < V and ys[pos + 1] == ys[pos]):
        tie |= 2
    return tie


@pytest.mark.parametrize("name,B", [("c2", 64), ("c3", 256), ("c4", 96)])
def test_detail_matches_oracle(gpu, torch, oracle, name, B):
    import workloads
    w = workloads.make(name, B=B, seed=11)
    lg, prm, rec, u = w["logits"], w["params"], w["recent"], w["u"]
    B, V = lg.shape
    if name == "c4":
        prm = prm.copy()
        prm["top_k"][:8] = [1, 0, 20, 100, 0, 1, 0, 100]
    _say("detail", name, "B", B, "V", V)
    d_lg = torch.from_numpy(lg).cuda()
    d_u = torch.from_numpy(u).cuda()
    d_pr = torch.from_numpy(np.ascontiguousarray(prm).view(np.uint8)).cuda()
    d_rec = torch.from_numpy(rec.view(np.int32)).cuda() if rec is not None else None
    s = gpu.Sampler(0.7, 40, 0.9, 1.1, seed=3)
    tok_b = torch.zeros(B, dtype=torch.int32, device="cuda")
    tok_d = torch.zeros(B, dtype=torch.int32, device="cuda")
    st = torch.zeros(B, dtype=torch.int32, device="cuda")
    s.sample_batch(d_lg, tok_b, params=d_pr, recent=d_rec, u=d_u, status=st)
    cap = V if (prm["top_k"] == 0).any() else int(prm["top_k"].max())
    out = s.sample_detail(d_lg, tok_d, cap, params=d_pr, recent=d_rec, u=d_u, status=st)
    torch.cuda.synchronize()
    assert (st.cpu().numpy() == 0).all()
    tb = tok_b.cpu().numpy().astype(np.int64)
    td = tok_d.cpu().numpy().astype(np.int64)
    ids = out["ids"].cpu().numpy().view(np.uint32)
    p = out["p"].cpu().numpy()
    n_kept = out["n_kept"].cpu().numpy()
    cut = out["cut"].cpu().numpy()
    sums = out["sums"].cpu().numpy()
    ties = out["ties"].cpu().numpy()
    p_exact = p_total = 0
    n_ties = n_tok_ties = 0
    for b in range(B):
        pr = prm[b]
        want, det = oracle.sample(lg[b], float(pr["temperature"]), int(pr["top_k"]), float(pr["top_p"]),
                                  float(pr["rep_penalty"]), recent=rec[b] if rec is not None else (),
                                  r=float(u[b]), detail=True)
        assert tb[b] == want and td[b] == want, (b, tb[b], td[b], want)
        n = det["idx"].size
        assert n_kept[b] == n, (b, n_kept[b], n)
        assert cut[b] == det["cut"], (b, cut[b], det["cut"])
        assert sums[b, 0].view(np.uint32) == np.float32(det["sum"]).view(np.uint32), (b, sums[b, 0], det["sum"])
        assert sums[b, 1].view(np.uint32) == np.float32(det["s2"]).view(np.uint32), (b, sums[b, 1], det["s2"])
        m = min(n, cap)
        assert np.array_equal(ids[b, :m], det["idx"][:m]), b
        ref = det["p"][:m].astype(np.float64)
        rel = np.abs(p[b, :m].astype(np.float64) - ref) / np.maximum(np.abs(ref), 1e-38)
        assert rel.max() <= 1e-5, (b, rel.max())
        p_exact += int((p[b, :m].view(np.uint32) == det["p"][:m].view(np.uint32)).sum())
        p_total += m
        tie = oracle_ties(det["logits"], n, det["cut"], want)
        assert ties[b] == tie, (b, ties[b], tie)
        n_ties += tie & 1
        n_tok_ties += tie >> 1
    _say(name, "rows", B, "probabilities bit-exact", p_exact, "of", p_total, "tie rows", n_ties,
         "token on a tie", n_tok_ties)
