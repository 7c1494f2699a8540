"""GPU parity: the HIP sampler (through the C ABI) against the CPU oracle on
the same seeded inputs.  Integer outputs (token ids) must be identical.

The oracle's tie order (value descending, index ascending) stands in for the
reference's unspecified sort_unstable_by order on equal keys (src/sampler.rs:45).
"""
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def torch():
    import torch as _t
    if not _t.cuda.is_available():
        pytest.skip("no GPU")
    return _t


def run_batch(gs, torch, logits, params=None, u=None, recent=None, uniform=None, seed=0):
    """Sample B rows on the GPU; returns (tokens int64 numpy, status numpy)."""
    B, V = logits.shape
    d_lg = torch.from_numpy(np.ascontiguousarray(logits)).cuda()
    d_tok = torch.zeros(B, dtype=torch.int32, device="cuda")
    d_st = torch.full((B,), 99, dtype=torch.int32, device="cuda")
    d_u = torch.from_numpy(np.ascontiguousarray(u, dtype=np.float32)).cuda() if u is not None else None
    d_rec = torch.from_numpy(np.ascontiguousarray(recent, dtype=np.uint32).view(np.int32)).cuda() \
        if recent is not None else None
    d_pr = None
    if params is not None:
        d_pr = torch.from_numpy(np.ascontiguousarray(params).view(np.uint8)).cuda()
    up = uniform or (0.7, 40, 0.9, 1.1)
    s = gs.Sampler(*up, seed=seed)
    s.sample_batch(d_lg, d_tok, params=d_pr, recent=d_rec, u=d_u, status=d_st)
    torch.cuda.synchronize()
    tok = d_tok.cpu().numpy().astype(np.int64)
    st = d_st.cpu().numpy()
    return tok, st, s


def check_tokens(name, got, want, st=None):
    if st is not None:
        assert (st == 0).all(), (name, np.unique(st))
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, "%s: %d/%d rows differ, first %s got %s want %s" % (
        name, bad.size, got.size, bad[:5], got[bad[:5]], want[bad[:5]])


# --- golden vectors (independent pure-Python restatement) ---------------------
def test_golden_cases(gpu, torch):
    import json, os
    cases = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "sampler_cases.json")))
    for c in cases:
        _say("golden", c["name"], "V", len(c["logits"]))
        x = np.array([c["logits"]], np.float32)
        rec = np.array([c["recent"]], np.uint32) if c["recent"] else None
        tok, st, _ = run_batch(gpu, torch, x, u=[c["u"]], recent=rec,
                               uniform=(c["T"], c["k"], c["p"], c["rep"]))
        assert st[0] == 0, c["name"]
        assert tok[0] == c["token"], (c["name"], tok[0], c["token"])


# --- the five configurations (row counts reduced where the oracle is slow) ---
def test_c2_llama3(gpu, torch, oracle):
    import workloads
    w = workloads.make("c2", B=16)
    _say("c2 B=16 V", w["V"])
    tok, st, _ = run_batch(gpu, torch, w["logits"], params=w["params"], u=w["u"], recent=w["recent"])
    want = oracle.sample_batch(w["logits"], w["params"], w["u"], recent=w["recent"], nthreads=8,
                               fast_topk=True)
    check_tokens("c2", tok, want, st)


def test_c3_qwen_full_vocab(gpu, torch, oracle):
    import workloads
    w = workloads.make("c3", B=6)
    _say("c3 B=6 V", w["V"])
    tok, st, _ = run_batch(gpu, torch, w["logits"], params=w["params"], u=w["u"])
    want = oracle.sample_batch(w["logits"], w["params"], w["u"], nthreads=6)
    check_tokens("c3", tok, want, st)


def test_c4_gemma_hetero(gpu, torch, oracle):
    import workloads
    w = workloads.make("c4", B=16)
    _say("c4 B=16 V", w["V"], "k", list(w["params"]["top_k"]))
    tok, st, _ = run_batch(gpu, torch, w["logits"], params=w["params"], u=w["u"], recent=w["recent"])
    want = oracle.sample_batch(w["logits"], w["params"], w["u"], recent=w["recent"], nthreads=8)
    check_tokens("c4", tok, want, st)
    # top_k == 1 rows are the argmax of the penalized, scaled logits
    for b in np.nonzero(w["params"]["top_k"] == 1)[0]:
        assert tok[b] == want[b]



@pytest.mark.parametrize("name", ["c2", "c4"])
def test_full_batch(gpu, torch, oracle, name):
    """Every row of the configuration at its full size (C2 B=64 V=128256, C4
    B=512 V=256000): identical tokens, and no full-vocabulary row handed to
    the sort-based path.  (C3 at full size: test_c3_full_batch_256.)"""
    import workloads
    w = workloads.make(name)
    rec = w.get("recent")
    _say(name, "full batch B", w["B"], "V", w["V"])
    tok, st, s = run_batch(gpu, torch, w["logits"], params=w["params"], u=w["u"], recent=rec)
    assert s.fallback_rows() == 0
    want = oracle.sample_batch(w["logits"], w["params"], w["u"], recent=rec, nthreads=8,
                               fast_topk=name == "c2")
    check_tokens(name + " full", tok, want, st)

def test_c4_rows_with_zero_at_run_head(gpu, torch, oracle):
    """Rows 312-319 of the full C4 batch.  In row 315 a bin collected late
    starts a run of collected bins whose first list slot holds a zero (a
    penalized id's raw value, taken out); the run's compaction must not take
    its base from that slot, or an entry is listed twice and the sums drift."""
    import workloads
    w = workloads.make("c4")
    sl = slice(312, 320)
    lg = np.ascontiguousarray(w["logits"][sl])
    pr, u, rec = w["params"][sl], w["u"][sl], np.ascontiguousarray(w["recent"][sl])
    del w
    _say("c4 rows 312-319 V", lg.shape[1])
    tok, st, s = run_batch(gpu, torch, lg, params=pr, u=u, recent=rec)
    assert (pr["top_k"] == 0).any()        # rows on the full-vocabulary path
    assert s.fallback_rows() == 0          # every full-vocabulary row stayed on the binned path
    want = oracle.sample_batch(lg, pr, u, recent=rec, nthreads=8)
    check_tokens("c4 rows 312-319", tok, want, st)


def test_c1_decode_trace(gpu, torch, oracle):
    """Config C1 as specified: 256 sequential single-row calls on the
    sampler's own LCG stream (seed 42), against the reference loop."""
    import workloads
    w = workloads.make("c1")
    assert w["steps"] == 256
    _say("c1 steps", w["steps"])
    s = gpu.Sampler(w["T"], w["k"], w["p"], w["rep"], seed=w["seed"])
    recent = list(w["init_recent"])
    got = []
    for t in range(w["steps"]):
        tok = s.sample(w["logits"][t], np.array(recent, np.uint32))
        got.append(tok)
        recent.append(tok)
        if len(recent) > w["W"]:
            recent.pop(0)
    want = oracle.decode_trace(w["logits"], w["T"], w["k"], w["p"], w["rep"], w["W"],
                               w["init_recent"], w["seed"])
    check_tokens("c1", np.array(got), want)
    _, st = workloads.lcg_stream(w["seed"], w["steps"])
    assert s.state == st


def test_c5_device_loop(gpu, torch, oracle):
    """Device-resident loop: on-device logits, ring window, LCG draws."""
    import workloads
    w = workloads.make("c5", B=4, steps=6)
    B, V, W, steps = w["B"], w["V"], w["W"], w["steps"]
    _say("c5 B", B, "steps", steps)
    d_lg = torch.empty((B, V), dtype=torch.float32, device="cuda")
    d_win = torch.from_numpy(w["window"].view(np.int32)).cuda()
    d_tok = torch.zeros(B, dtype=torch.int32, device="cuda")
    s = gpu.Sampler(w["T"], w["k"], w["p"], w["rep"], seed=w["seed"])
    toks = []
    for t in range(steps):
        gpu.synth_logits(d_lg, w["synth_seed"], t * B * V, w["sigma"])
        s.sample_batch(d_lg, d_tok, recent=d_win)
        gpu.window_push(d_win, d_tok, t)
        toks.append(d_tok.cpu().numpy().astype(np.int64))
    u, _ = workloads.lcg_stream(w["seed"], steps * B)
    want, win = oracle.device_loop(B, V, steps, w["synth_seed"], w["sigma"],
                                   (w["T"], w["k"], w["p"], w["rep"]), w["window"], u, nthreads=4)
    check_tokens("c5", np.array(toks), want)
    assert (d_win.cpu().numpy().view(np.uint32) == win).all()


def test_synth_matches_host(gpu, torch, oracle):
    d = torch.empty((3, 1000), dtype=torch.float32, device="cuda")
    gpu.synth_logits(d, 77, 5, 3.0)
    h = oracle.synth_logits(3000, 77, 5, 3.0).reshape(3, 1000)
    assert (d.cpu().numpy().view(np.uint32) == h.view(np.uint32)).all()


# --- edge cases the reference's code paths reach -----------------------------
def test_edge_cases(gpu, torch, oracle):
    rng = np.random.default_rng(7)
    V = 4096
    cases = []
    x = np.zeros(V, np.float32)
    cases.append(("all_equal_k0", x, (1.0, 0, 0.9, 1.0)))
    cases.append(("all_equal_k40", x, (1.0, 40, 0.9, 1.0)))
    cases.append(("all_equal_k2000", x, (1.0, 2000, 0.95, 1.0)))
    x = (rng.integers(-3, 3, V) / 2).astype(np.float32)
    cases.append(("ties_k100", x, (0.7, 100, 0.9, 1.1)))
    cases.append(("ties_k0", x, (0.7, 0, 0.9, 1.1)))
    x = np.full(V, -np.inf, np.float32)
    x[[5, 77, 900]] = [1.0, 2.0, 1.5]
    cases.append(("masked_k40", x, (1.0, 40, 0.99, 1.0)))
    cases.append(("masked_k0", x, (1.0, 0, 0.99, 1.0)))
    x = rng.standard_normal(V).astype(np.float32)
    x[10] = np.inf
    cases.append(("posinf_k0", x, (1.0, 0, 0.9, 1.0)))
    cases.append(("posinf_k5", x, (1.0, 5, 0.9, 1.0)))
    x = rng.standard_normal(V).astype(np.float32)
    cases.append(("k_eq_V", x, (0.9, V, 0.8, 1.2)))
    cases.append(("k_1500_fullpath", x, (0.9, 1500, 0.8, 1.2)))
    cases.append(("k1", x, (0.9, 1, 0.5, 1.3)))
    cases.append(("greedy", x, (0.0, 40, 0.9, 1.3)))
    cases.append(("greedy_neg", x, (-1.0, 40, 0.9, 1.0)))
    cases.append(("top_p_0", x, (1.3, 0, 0.0, 1.0)))
    cases.append(("top_p_1", x, (1.3, 0, 1.0, 1.0)))
    cases.append(("tiny_T", x, (1e-3, 0, 0.9, 1.0)))
    cases.append(("big_T", x, (50.0, 0, 0.95, 1.0)))
    xz = x.copy()
    xz[::7] = -0.0
    xz[3::7] = 0.0
    cases.append(("signed_zeros", xz, (1.0, 0, 0.97, 1.0)))
    x = (rng.standard_normal(V) * 30).astype(np.float32)
    cases.append(("peaked_k0", x, (1.0, 0, 0.9, 1.0)))
    rec = np.concatenate([rng.integers(0, V, 60), [0, 0, 0, V + 5, 2 ** 31, 2 ** 32 - 1]]).astype(np.uint32)
    for name, x, (T, k, p, rep) in cases:
        for u in (0.0, 0.37, 0.9999):
            _say("edge", name, "u", u)
            tok, st, _ = run_batch(gpu, torch, x[None, :], u=[u], recent=rec[None, :],
                                   uniform=(T, k, p, rep))
            want = oracle.sample(x, T, k, p, rep, rec, r=u)
            assert st[0] == 0, (name, st[0])
            assert tok[0] == want, (name, u, tok[0], want)


@pytest.mark.parametrize("V", [32000, 32768, 4096, 1000, 8])
def test_topk_register_rows(gpu, torch, oracle, V):
    """Top-k rows held in registers (V <= 32768): penalties with rep below and
    above 1 (the penalized ids include the largest logits), windows up to the
    maximum, ids outside [0, V), ties, masked rows and k up to kMaxTopK."""
    import workloads
    rng = np.random.default_rng(V)
    W = 1024
    rows, prm, recs = [], [], []
    for case in range(24):
        kind = case % 6
        if kind == 0:
            x = (rng.standard_normal(V) * 3).astype(np.float32)
        elif kind == 1:
            x = (rng.integers(-4, 4, V) / 4).astype(np.float32)
        elif kind == 2:
            x = np.full(V, -np.inf, np.float32)
            x[rng.choice(V, min(V, 50), replace=False)] = rng.standard_normal(min(V, 50))
        elif kind == 3:
            x = np.zeros(V, np.float32)
        elif kind == 4:
            x = (rng.standard_normal(V) * 0.01 + 5).astype(np.float32)
        else:
            x = (rng.standard_normal(V) * 3).astype(np.float32)
            x[rng.choice(V, min(V, 5), replace=False)] += 10
        top = np.argsort(-x, kind="stable")[:16].astype(np.uint32)
        nrec = [0, 64, 1024, 300][case % 4]
        rec = np.full(W, 2 ** 32 - 1, np.uint32)
        body = np.concatenate([top, rng.integers(0, V, W).astype(np.uint32)])[:nrec]
        rec[:nrec] = body
        if nrec:
            rec[:3] = [V, 2 ** 31, 2 ** 31 + 7]
        k = [1, 2, 40, 100, 1000, 1024][case % 6]
        k = min(k, V - 1) if V > 1 else 1
        rep = [1.3, 0.7, 1.0, 1.1][(case // 6) % 4]
        T = [0.7, 1.0, 2.5, 0.3][case % 4]
        p = [0.9, 0.5, 1.0, 0.99][(case // 3) % 4]
        rows.append(x)
        prm.append((T, k, p, rep))
        recs.append(rec)
    x = np.stack(rows)
    pr = workloads.params_rows(prm)
    rec = np.stack(recs)
    for u0 in (0.0, 0.41, 0.9999):
        u = np.full(len(rows), u0, np.float32)
        _say("topk_register V", V, "u", u0)
        tok, st, _ = run_batch(gpu, torch, x, params=pr, u=u, recent=rec)
        want = oracle.sample_batch(x, pr, u, recent=rec)
        check_tokens("topk_reg V%d u%.2f" % (V, u0), tok, want, st)


@pytest.mark.parametrize("V", [32000, 32768, 4096, 64, 8, 40000])
def test_single_row_calls(gpu, torch, oracle, V):
    """gs_sample one row at a time (the reference's call shape): device and
    host logits, host windows short enough for the kernel arguments (<= 64
    ids) and longer ones, device windows; top-k and greedy rows; rows the
    register kernel hands back to the general kernel (k above the number of
    threads holding elements, too few finite logits).  The draw is the
    sampler's LCG, seeded per call."""
    rng = np.random.default_rng(V + 11)
    for case in range(30):
        kind = case % 5
        if kind == 0:
            x = (rng.standard_normal(V) * 3).astype(np.float32)
        elif kind == 1:
            x = (rng.integers(-4, 4, V) / 4).astype(np.float32)
        elif kind == 2:
            x = np.full(V, -np.inf, np.float32)
            x[rng.choice(V, min(V, 3), replace=False)] = rng.standard_normal(min(V, 3))
        elif kind == 3:
            x = (rng.standard_normal(V) * 3).astype(np.float32)
            x[rng.choice(V, min(V, 5), replace=False)] += 10
        else:
            x = (rng.standard_normal(V) * 0.01 + 5).astype(np.float32)
        nrec = [0, 64, 7, 300, 1024, 64][case % 6]
        top = np.argsort(-x, kind="stable")[:8].astype(np.uint32)
        rec = np.concatenate([top, rng.integers(0, V, 1024).astype(np.uint32)])[:nrec]
        if nrec > 4:
            rec[2:4] = [V, 2 ** 31 + 5]
        T = [0.7, 1.0, 0.0, 2.5, -1.0, 0.3][case % 6]
        k = [40, 1, 1000, 60, 20, 5][(case // 2) % 6]
        k = min(k, V - 1)
        p = [0.9, 1.0, 0.5][case % 3]
        rep = [1.1, 1.3, 0.8, 1.0][(case // 3) % 4]
        seed = 1000 + case
        dev_row = case % 2 == 0
        dev_win = case % 4 == 3
        xr = torch.from_numpy(x).cuda() if dev_row else x
        rr = torch.from_numpy(rec.view(np.int32)).cuda() if (dev_win and nrec) else rec
        s = gpu.Sampler(T, k, p, rep, seed=seed)
        want = oracle.sample(x, T, k, p, rep, recent=rec, state=seed)
        _say("single V", V, "case", case, "T", T, "k", k, "W", nrec, "dev", dev_row, dev_win)
        if want < 0:
            with pytest.raises(gpu.SamplerError) as ei:
                s.sample(xr, rr)
            assert ei.value.code == want, (case, ei.value.code, want)
        else:
            got = s.sample(xr, rr)
            assert got == want, (V, case, T, k, p, rep, nrec, got, want)
        assert s.state == (oracle.lcg_draws(seed, 1)[1] if T > 0 else seed), case


@pytest.mark.parametrize("V", [32000, 4096, 8, 40000])
def test_greedy_rows(gpu, torch, oracle, V):
    """Greedy (T <= 0) rows, register path (V <= 32768) and the row loop:
    ties (the last maximal index wins), -0 and +0, all -inf, a penalized
    maximum, penalties in both directions and NaN rows."""
    import workloads
    rng = np.random.default_rng(V + 7)
    rows, prm, recs = [], [], []
    W = 64
    for case in range(12):
        kind = case % 6
        if kind == 0:
            x = (rng.standard_normal(V) * 3).astype(np.float32)
        elif kind == 1:
            x = rng.integers(-3, 3, V).astype(np.float32)
        elif kind == 2:
            x = np.full(V, -np.inf, np.float32)
        elif kind == 3:
            x = np.where(rng.random(V) < 0.5, np.float32(-0.0), np.float32(0.0)).astype(np.float32)
        elif kind == 4:
            x = (rng.standard_normal(V) * 3).astype(np.float32)
            x[rng.choice(V, 3, replace=False)] = x.max()
        else:
            x = (rng.standard_normal(V) * 3).astype(np.float32)
            if case >= 6 and V > 1:
                x[rng.integers(0, V)] = np.nan
        top = np.argsort(-x, kind="stable")[:4].astype(np.uint32)
        rec = np.concatenate([top, rng.integers(0, V, W).astype(np.uint32)])[:W]
        rows.append(x)
        prm.append(([0.0, -1.0][case % 2], 40, 0.9, [1.0, 1.3, 0.6, 1.1][case % 4]))
        recs.append(rec)
    x = np.stack(rows)
    pr = workloads.params_rows(prm)
    rec = np.stack(recs)
    u = np.zeros(len(rows), np.float32)
    tok, st, _ = run_batch(gpu, torch, x, params=pr, u=u, recent=rec)
    want = oracle.sample_batch(x, pr, u, recent=rec)
    for j in range(len(rows)):
        if want[j] < 0:
            assert st[j] == want[j], (j, prm[j], st[j], want[j])
        else:
            assert st[j] == 0 and tok[j] == want[j], (j, prm[j], st[j], tok[j], want[j])


@pytest.mark.parametrize("V", [4096, 40000])
def test_odd_penalties(gpu, torch, oracle, V):
    """Penalties that push logits to +-inf, 0 or NaN (rep 0, negative, inf,
    NaN, tiny, huge) on the register path (V <= 32768), the longer top-k
    path and the full-vocabulary path; the window holds the largest logits,
    -inf entries and repeats.  A NaN the reference would panic on must come
    back as GS_ERR_NAN."""
    import workloads
    rng = np.random.default_rng(V + 1)
    W = 96
    reps = [0.0, -1.0, np.inf, np.nan, 1e-30, 1e30, 0.5, -0.0]
    rows, prm, recs = [], [], []
    for i, rep in enumerate(reps):
        for k in (40, 0):
            x = (rng.standard_normal(V) * 3).astype(np.float32)
            if i % 2:
                x[rng.choice(V, 5, replace=False)] = -np.inf
            top = np.argsort(-x, kind="stable")[:8].astype(np.uint32)
            neg = np.nonzero(x == -np.inf)[0].astype(np.uint32)
            rec = np.concatenate([top, top[:2], neg, rng.integers(0, V, W).astype(np.uint32)])[:W]
            rows.append(x)
            prm.append((0.7 if k else 1.0, k, 0.9, rep))
            recs.append(rec)
    x = np.stack(rows)
    pr = workloads.params_rows(prm)
    rec = np.stack(recs)
    for u0 in (0.0, 0.6):
        u = np.full(len(rows), u0, np.float32)
        _say("odd penalties V", V, "u", u0)
        tok, st, _ = run_batch(gpu, torch, x, params=pr, u=u, recent=rec)
        want = oracle.sample_batch(x, pr, u, recent=rec)
        for j in range(len(rows)):
            if want[j] < 0:
                assert st[j] == want[j], (j, prm[j], st[j], want[j])
            else:
                assert st[j] == 0 and tok[j] == want[j], (j, prm[j], st[j], tok[j], want[j])


def test_errors(gpu, torch):
    x = np.ones((3, 100), np.float32)
    x[1, 50] = np.nan
    tok, st, _ = run_batch(gpu, torch, x, u=[0.1, 0.1, 0.1], uniform=(0.7, 40, 0.9, 1.0))
    assert list(st) == [0, gpu.GS_ERR_NAN, 0]
    tok, st, _ = run_batch(gpu, torch, x, u=[0.1, 0.1, 0.1], uniform=(0.0, 40, 0.9, 1.0))
    assert list(st) == [0, gpu.GS_ERR_NAN, 0]
    tok, st, _ = run_batch(gpu, torch, x, u=[0.1, 0.1, 0.1], uniform=(0.7, 0, 0.9, 1.0))
    assert list(st) == [0, gpu.GS_ERR_NAN, 0]
    s = gpu.Sampler(0.7, 40, 0.9, 1.0, seed=1)
    with pytest.raises(gpu.SamplerError):
        s.sample(np.zeros(0, np.float32))
    assert s.sample(np.array([np.nan], np.float32)) == 0


def test_lcg_batch_stream(gpu, torch, oracle):
    """u == NULL: row b takes the b-th next draw of the sampler's stream."""
    import workloads
    rng = np.random.default_rng(3)
    B, V = 8, 2000
    x = (rng.standard_normal((B, V)) * 2).astype(np.float32)
    tok, st, s = run_batch(gpu, torch, x, uniform=(1.0, 0, 0.95, 1.0), seed=99)
    u, nxt = workloads.lcg_stream(99, B)
    pr = workloads.params_rows([(1.0, 0, 0.95, 1.0)] * B)
    want = oracle.sample_batch(x, pr, u)
    check_tokens("lcg_batch", tok, want, st)
    assert s.state == nxt


def test_reference_free_function_api(gpu, oracle):
    """set_seed + sample(logits, T, k, p, rep, recent) with the global stream."""
    import gs_sampler
    rng = np.random.default_rng(5)
    gs_sampler.set_seed(42)
    oracle.set_seed(42)
    for i in range(10):
        x = (rng.standard_normal(3000) * 3).astype(np.float32)
        T = 0.0 if i == 4 else 0.8
        rec = rng.integers(0, 3000, 32)
        a = gs_sampler.sample(x, T, 40, 0.9, 1.1, rec)
        b = oracle.sample(x, T, 40, 0.9, 1.1, rec)
        assert a == b


# --- full-vocabulary path (binned exact sums) -------------------------------
def test_c3_full_batch_256(gpu, torch, oracle):
    """All 256 rows of the benchmark batch, bit-exact, none on the sort path."""
    import workloads
    w = workloads.make("c3")
    _say("c3 B=256 V", w["V"])
    tok, st, s = run_batch(gpu, torch, w["logits"], params=w["params"], u=w["u"])
    assert s.fallback_rows() == 0
    want = oracle.sample_batch(w["logits"], w["params"], w["u"], nthreads=16)
    check_tokens("c3 B=256", tok, want, st)


def _sweep_rows(rng, B, V, shape):
    """Rows of several shapes: normal of various widths, a dominant maximum,
    values on a coarse grid (many exactly equal logits), heavy tails."""
    if shape == "normal":
        sig = rng.choice([0.3, 1.0, 2.0, 4.0, 8.0], size=(B, 1)).astype(np.float32)
        return (rng.standard_normal((B, V), dtype=np.float32) * sig).astype(np.float32)
    if shape == "spike":
        x = rng.standard_normal((B, V), dtype=np.float32) * 2.0
        x[np.arange(B), rng.integers(0, V, B)] += rng.uniform(6, 14, B).astype(np.float32)
        return x.astype(np.float32)
    if shape == "grid":
        return (np.round(rng.standard_normal((B, V)) * 4.0) / 2.0).astype(np.float32)
    # heavy tail: Student-like via normal / sqrt(chi2)
    z = rng.standard_normal((B, V))
    c = rng.chisquare(3, size=(B, V))
    return (z / np.sqrt(c / 3.0)).astype(np.float32)


@pytest.mark.parametrize("V,shape", [(100, "normal"), (4099, "grid"), (50000, "normal"),
                                     (50000, "spike"), (152064, "normal"), (152064, "grid"),
                                     (152064, "heavy"), (262144, "normal")])
def test_full_vocab_sweep(gpu, torch, oracle, V, shape):
    """Heterogeneous rows through the full-vocabulary path (top_k = 0):
    temperatures, top_p (including >= 1 and tiny), penalties with windows and
    draws over [0, 1), against the oracle bit for bit."""
    import workloads
    rng = np.random.default_rng(V * 7 + len(shape))
    B = 16
    x = _sweep_rows(rng, B, V, shape)
    rows = []
    for b in range(B):
        T = float(rng.choice([0.5, 1.0, 1.7]))
        p = float(rng.choice([0.3, 0.9, 0.95, 0.999, 1.0]))
        rep = float(rng.choice([1.0, 1.0, 1.2]))
        rows.append((T, 0, p, rep))
    params = np.array(rows, dtype=workloads.PARAMS_DTYPE)
    W = 64
    recent = rng.integers(0, V, size=(B, W), dtype=np.uint32)
    u = rng.random(B, dtype=np.float32)
    _say("sweep V", V, shape)
    tok, st, _ = run_batch(gpu, torch, x, params=params, u=u, recent=recent)
    want = oracle.sample_batch(x, params, u, recent=recent, nthreads=16)
    check_tokens("sweep V=%d %s" % (V, shape), tok, want, st)


def lcg_draw_table(seeds, steps):
    """u[t, b] = the t-th draw of an LCG seeded seeds[b] (src/sampler.rs:7-12),
    vectorised over rows with wrapping u64 arithmetic."""
    a, c = np.uint64(6364136223846793005), np.uint64(1442695040888963407)
    st = np.asarray(seeds, dtype=np.uint64).copy()
    u = np.empty((steps, st.size), np.float32)
    with np.errstate(over="ignore"):
        for t in range(steps):
            u[t] = (st >> np.uint64(33)).astype(np.float32) / np.float32(4294967295.0)
            st = st * a + c
    return u, st


def test_c5_hip_graph(gpu, torch, oracle):
    """Config C5 as specified: B = 1024 rows, V = 152064, 128 steps captured
    in one HIP graph (on-device logits, then the decode step: sample with
    the 1024-id ring window and commit), replayed once.  The rows' LCGs live
    on the device (gs_decode_*), so the draws come from the device state, not
    from values frozen at capture.  The whole token trace and the final
    windows must equal the oracle's loop over the same logits and draws."""
    import workloads
    w = workloads.make("c5")
    B, V, W, steps = w["B"], w["V"], w["W"], w["steps"]
    assert (B, V, W, steps) == (1024, 152064, 1024, 128)
    _say("c5 graph B", B, "V", V, "steps", steps)
    seeds = [w["seed"] + b for b in range(B)]
    s = gpu.Sampler(w["T"], w["k"], w["p"], w["rep"], seed=1)
    s.reserve(B, V)
    dec = gpu.Decoder(B, W=W, max_new=steps + 1, stop=())
    dec.init(s, seeds, init_recent=w["window"])
    d_lg = torch.empty((B, V), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        st = torch.cuda.current_stream()
        for t in range(steps):
            gpu.synth_logits(d_lg, w["synth_seed"], t * B * V, w["sigma"], stream=st)
            dec.step(s, logits=d_lg, stream=st)
    torch.cuda.synchronize()
    assert int(dec.row_state()["n_gen"].sum()) == 0     # capture ran nothing
    g.replay()
    torch.cuda.synchronize()
    rows = dec.row_state()
    gen = dec.generated.cpu().numpy().view(np.uint32)[:, :steps].astype(np.int64)
    win = dec.window.cpu().numpy().view(np.uint32)
    u, final = lcg_draw_table(seeds, steps + 1)          # + the draw made after the last step
    _say("c5 oracle")
    want, want_win = oracle.device_loop(B, V, steps, w["synth_seed"], w["sigma"],
                                        (w["T"], w["k"], w["p"], w["rep"]), w["window"],
                                        np.ascontiguousarray(u[:steps]).reshape(-1), nthreads=16)
    check_tokens("c5 graph", gen.T, want)
    assert (rows["n_gen"] == steps).all() and (rows["done"] == gpu.DONE_RUNNING).all()
    assert np.array_equal(rows["rng"], final)            # one draw ahead, as documented
    assert np.array_equal(win, want_win)


# --- a few top-k rows of a large vocabulary over many workgroups (split / chunked) ---
def _split_rows(rng, B, V, shape):
    if shape == "normal":
        x = rng.standard_normal((B, V)) * 2.0
    elif shape == "grid":        # many exact ties, before and after the division by T
        x = rng.integers(-40, 40, size=(B, V)) / 4.0
    elif shape == "equal":       # every logit equal: the top k are the k lowest ids
        x = np.full((B, V), 1.5)
    else:                        # spikes on a flat floor
        x = rng.standard_normal((B, V)) * 0.5
        for b in range(B):
            x[b, rng.integers(0, V, 30)] += rng.uniform(6, 12, 30)
    return x.astype(np.float32)


@pytest.mark.parametrize("V,B,k,shape,T", [
    (152064, 1, 40, "normal", 0.7),
    (152064, 8, 1, "normal", 0.7),
    (40000, 3, 100, "grid", 0.7),
    (262144, 2, 128, "grid", 1.3),
    (33000, 32, 40, "spike", 0.7),
    (200001, 5, 7, "normal", 0.9),
    (152064, 4, 40, "equal", 0.7),
    (837999, 1, 40, "spike", 1.0),
])
def test_split_rows(gpu, torch, oracle, V, B, k, shape, T):
    """Rows of V > 32768 with 0 < k <= 128 in batches of a few rows: rows of
    V % 4 == 0 take the one-launch chunked path (chunks of up to 32768), the
    odd vocabularies here the split path (chunks of 1024); every chunk keeps
    its best round_up(k, 4) elements.  Penalty window with duplicates, ids on
    chunk edges and ids >= V."""
    rng = np.random.default_rng(V + B + k)
    x = _split_rows(rng, B, V, shape)
    W = 64
    rec = rng.integers(0, V, size=(B, W)).astype(np.uint32)
    rec[:, :6] = [1023, 1024, 1024, V - 1, V + 5, 0]
    rec[:, 6:10] = rec[:, 10:14]                       # duplicates
    u = rng.random(B).astype(np.float32)
    u[0] = 0.0
    for rep in (1.0, 1.3):
        _say("split V", V, "B", B, "k", k, shape, "rep", rep)
        params = [(T, k, 0.9, rep)] * B
        tok, st, _ = run_batch(gpu, torch, x, u=u, recent=rec, uniform=(T, k, 0.9, rep))
        want = oracle.sample_batch(x, params, u, recent=rec, nthreads=8, fast_topk=True)
        check_tokens("split %s rep %s" % (shape, rep), tok, want, st)


def test_split_rows_nan_and_single_call(gpu, torch, oracle):
    """A NaN anywhere in a split row is an error for that row only; the
    single-row call (gs_sample) takes the same path and draws from the LCG."""
    rng = np.random.default_rng(5)
    V, B = 152064, 3
    x = (rng.standard_normal((B, V)) * 2).astype(np.float32)
    x[1, 77777] = np.nan
    u = rng.random(B).astype(np.float32)
    tok, st, _ = run_batch(gpu, torch, x, u=u, uniform=(0.7, 40, 0.9, 1.0))
    assert list(st) == [0, gpu.GS_ERR_NAN, 0], st
    want = oracle.sample_batch(x[[0, 2]], [(0.7, 40, 0.9, 1.0)] * 2, u[[0, 2]], nthreads=4, fast_topk=True)
    assert tok[0] == want[0] and tok[2] == want[1]
    s = gpu.Sampler(0.7, 40, 0.9, 1.1, seed=42)
    recent = np.array([3, 3, 9, V - 1, 1024], np.uint32)
    d = torch.from_numpy(x[0]).cuda()
    state = 42
    for i in range(5):
        got = s.sample(d, recent)
        r, state = oracle.lcg_draws(state, 1)
        w = oracle.sample(x[0], 0.7, 40, 0.9, 1.1, recent, r=float(r[0]))
        assert got == w, (i, got, w)
    with pytest.raises(gpu.SamplerError):
        s.sample(torch.from_numpy(x[1]).cuda())
