"""Pins the CPU oracle (oracle/sampler_oracle.c) against facts that do not
come from the oracle itself: closed-form LCG vectors, brute-force orderings,
float64 recomputations, numpy's sequential float32 cumsum, hand-built CDFs
and the reference's invariants (src/sampler.rs)."""
import math
import struct

import numpy as np
import pytest


def f32_bits(x):
    return struct.unpack("<I", struct.pack("<f", x))[0]


# --- LCG: src/sampler.rs:3-12 ----------------------------------------------
# KAT for seed 42 (computed with exact u64 arithmetic, independent of the oracle)
LCG42 = [0x00000000, 0x3e91778b, 0x3de6dfe3, 0x3e535f8b, 0x3ea161c4, 0x3eae1e2b]


def test_lcg_kat_seed42(oracle):
    d, _ = oracle.lcg_draws(42, 6)
    assert [f32_bits(float(x)) for x in d] == LCG42


def test_lcg_kat_default_seed(oracle):
    d, _ = oracle.lcg_draws(12345, 1)
    assert float(d[0]) == 0.0  # 12345 >> 33 == 0


def test_lcg_closed_form(oracle):
    # s' = s*a + c mod 2^64; draw = f32(s >> 33) / f32(2^32 - 1) from the pre-update state
    a, c, m = 6364136223846793005, 1442695040888963407, 1 << 64
    s = 0xDEADBEEFCAFEBABE
    d, st = oracle.lcg_draws(s, 50)
    for i in range(50):
        assert float(d[i]) == float(np.float32(np.float32(s >> 33) / np.float32(2.0 ** 32)))
        s = (s * a + c) % m
    assert st == s
    assert float(d.max()) <= 0.5  # r in [0, 0.5]: u32::MAX as f32 == 2^32


def test_lcg_max_draw_is_half(oracle):
    # state with s >> 33 == 2^31 - 1 rounds to 2^31 in f32 -> exactly 0.5
    s = ((1 << 31) - 1) << 33
    d, _ = oracle.lcg_draws(s, 1)
    assert float(d[0]) == 0.5


# --- penalty: src/sampler.rs:23-30 ------------------------------------------
def test_penalty_examples(oracle):
    x = np.array([2.0, -2.0, 0.0, 3.0, 1.0], np.float32)
    _, d = oracle.sample(x, 0.0, 0, 1.0, 2.0, [0, 1, 2, 3, 3, 99], r=0.0, detail=True)
    out = d["logits"]
    assert out[0] == 1.0          # positive: divided
    assert out[1] == -4.0         # negative: multiplied
    assert out[2] == 0.0          # zero is not > 0: multiplied (stays 0)
    assert out[3] == 0.75         # duplicate id: applied twice
    assert out[4] == 1.0          # not in window
    # id 99 >= V is ignored (no crash)


def test_penalty_one_is_identity(oracle):
    x = np.array([np.nan, 1.0, -1.0], np.float32)
    _, d = oracle.sample(x, 0.0, 0, 1.0, 1.0, [0, 1, 2], r=0.0, detail=True)
    # rep == 1.0 returns early, even NaN is untouched (and then greedy panics -> error)
    assert np.isnan(d["logits"][0]) and d["logits"][1] == 1.0


def test_penalty_sign_retest(oracle):
    # with a negative penalty the sign flips between repeated applications
    x = np.array([3.0, 0.0], np.float32)
    _, d = oracle.sample(x, 0.0, 0, 1.0, -2.0, [0, 0], r=0.0, detail=True)
    assert d["logits"][0] == np.float32(np.float32(3.0) / np.float32(-2.0)) * np.float32(-2.0)


# --- greedy: src/sampler.rs:15-19 -------------------------------------------
def test_greedy_last_max(oracle):
    x = np.array([1.0, 5.0, 2.0, 5.0, -1.0], np.float32)
    assert oracle.sample(x, 0.0, 40, 0.9, 1.0, [], r=0.3) == 3
    x = np.array([-0.0, 0.0, -1.0], np.float32)   # -0 == +0 under partial_cmp
    assert oracle.sample(x, -1.0, 40, 0.9, 1.0, [], r=0.3) == 1


def test_greedy_does_not_draw(oracle):
    oracle.set_seed(42)
    oracle.sample(np.array([1.0, 2.0], np.float32), 0.0, 0, 1.0, 1.0, [])
    assert oracle.get_seed() == 42
    oracle.sample(np.array([1.0, 2.0], np.float32), 0.5, 0, 1.0, 1.0, [])
    assert oracle.get_seed() != 42


def test_first_draw_seed42_is_top_candidate(oracle):
    rng = np.random.default_rng(3)
    x = rng.standard_normal(1000).astype(np.float32)
    oracle.set_seed(42)
    assert oracle.sample(x, 0.7, 40, 0.9, 1.0, []) == int(np.argmax(x))


# --- sort / top-k: src/sampler.rs:44-50 -------------------------------------
@pytest.mark.parametrize("seed", range(8))
def test_order_brute_force(oracle, seed):
    rng = np.random.default_rng(seed)
    V = int(rng.integers(1, 9))
    x = rng.integers(-3, 4, size=V).astype(np.float32) / np.float32(2.0)  # many ties
    T = float(rng.choice([0.5, 1.0, 0.7]))
    k = int(rng.integers(0, V + 2))
    _, d = oracle.sample(x, T, k, 1.0, 1.0, [], r=0.1, detail=True)
    y = [float(np.float32(v) / np.float32(T)) for v in x]
    order = sorted(range(V), key=lambda i: (-y[i], i))
    keep = k if 0 < k < V else V
    assert list(d["idx"]) == order[:keep]


def test_topk_fast_equals_full_sort(oracle):
    rng = np.random.default_rng(11)
    for _ in range(20):
        V = 5000
        x = (rng.integers(-50, 50, size=V) / 4).astype(np.float32)  # heavy ties
        k = int(rng.choice([1, 2, 40, 100, 4999]))
        u = float(rng.random())
        rec = rng.integers(0, V, 64)
        full = oracle.sample(x, 0.9, k, 0.9, 1.1, rec, r=u, fast_topk=False)
        fast = oracle.sample(x, 0.9, k, 0.9, 1.1, rec, r=u, fast_topk=True)
        assert full == fast


# --- softmax / nucleus / draw: src/sampler.rs:53-78 -------------------------
@pytest.mark.parametrize("V,k", [(50, 0), (1000, 40), (3000, 0)])
def test_softmax_against_float64(oracle, V, k):
    rng = np.random.default_rng(V)
    x = (rng.standard_normal(V) * 2).astype(np.float32)
    _, d = oracle.sample(x, 0.8, k, 1.0, 1.0, [], r=0.2, detail=True)
    y = (x.astype(np.float32) / np.float32(0.8)).astype(np.float64)
    sel = d["idx"]
    e = np.exp(y[sel] - y[sel].max())
    p64 = e / e.sum()
    np.testing.assert_allclose(d["p"], p64, rtol=1e-5, atol=1e-12)
    # The reference sums sequentially in float32: numpy's float32 cumsum is a
    # sequential running sum (np.sum would be pairwise).
    e32 = np.array([math.exp(v) for v in (y[sel] - y[sel].max())], np.float64)
    # glibc expf is within 1 ulp of the float64 exp rounded to float32
    ours = np.array([np.float32(v) for v in e32], np.float32)
    seq = np.cumsum(ours, dtype=np.float32)[-1]
    assert abs(float(d["sum"]) - float(seq)) <= 4 * np.spacing(np.float32(seq))


def test_nucleus_cut_matches_cumsum(oracle):
    rng = np.random.default_rng(5)
    x = (rng.standard_normal(2000) * 3).astype(np.float32)
    _, d = oracle.sample(x, 1.0, 0, 0.9, 1.0, [], r=0.3, detail=True)
    cum = np.cumsum(d["p"], dtype=np.float32)
    cut = int(np.argmax(cum >= np.float32(0.9))) + 1
    assert d["cut"] == cut
    assert d["s2"] == cum[cut - 1]   # the renormalising sum equals the running sum at the cut


@pytest.mark.parametrize("V", [1, 2, 3, 5, 8])
def test_draw_grid_against_cdf(oracle, V):
    rng = np.random.default_rng(V)
    x = (rng.standard_normal(V) * 1.5).astype(np.float32)
    for top_p in (1.0, 0.7):
        _, d = oracle.sample(x, 1.0, 0, top_p, 1.0, [], r=0.0, detail=True)
        order = d["idx"]
        y = x.astype(np.float64)
        e = np.exp(y[order] - y[order].max())
        p = e / e.sum()
        if top_p < 1.0:
            c = np.cumsum(p)
            n = int(np.argmax(c >= top_p)) + 1 if (c >= top_p).any() else V
            p = p[:n] / p[:n].sum()
            order = order[:n]
        cdf = np.cumsum(p)
        for u in np.linspace(0, 0.999, 211):
            tok = oracle.sample(x, 1.0, 0, top_p, 1.0, [], r=float(u))
            if np.min(np.abs(cdf - u)) < 1e-6:
                continue
            j = int(np.argmax(u < cdf)) if (u < cdf).any() else len(order) - 1
            assert tok == order[j], (u, tok, order[j])


def test_top_p_one_means_no_cut(oracle):
    x = np.array([3.0, 2.0, 1.0, 0.0], np.float32)
    _, d = oracle.sample(x, 1.0, 0, 1.0, 1.0, [], r=0.999, detail=True)
    assert d["cut"] == 4


def test_top_p_zero_keeps_one(oracle):
    x = np.array([1.0, 3.0, 2.0], np.float32)
    for u in (0.0, 0.49, 0.99):
        assert oracle.sample(x, 1.0, 0, 0.0, 1.0, [], r=u) == 1


def test_top_k_one_is_argmax(oracle):
    rng = np.random.default_rng(9)
    for _ in range(20):
        x = rng.standard_normal(300).astype(np.float32)
        assert oracle.sample(x, 0.7, 1, 0.5, 1.0, [], r=float(rng.random())) == int(np.argmax(x))


# --- panics become errors ---------------------------------------------------
def test_errors_and_degenerate(oracle):
    assert oracle.sample(np.array([1.0, np.nan], np.float32), 0.7, 40, 0.9, 1.1, [], r=0.1) == oracle.ERR_NAN
    assert oracle.sample(np.array([1.0, np.nan], np.float32), 0.0, 40, 0.9, 1.1, [], r=0.1) == oracle.ERR_NAN
    assert oracle.sample(np.zeros(0, np.float32), 0.7, 40, 0.9, 1.1, [], r=0.1) == oracle.ERR_EMPTY
    assert oracle.sample(np.zeros(0, np.float32), 0.0, 40, 0.9, 1.1, [], r=0.1) == 0
    assert oracle.sample(np.array([np.nan], np.float32), 0.7, 40, 0.9, 1.1, [], r=0.1) == 0
    # +inf: NaN probabilities; the reference returns the last kept candidate
    x = np.array([1.0, np.inf, 3.0, 2.0], np.float32)
    assert oracle.sample(x, 1.0, 0, 0.9, 1.0, [], r=0.1) == 0
    assert oracle.sample(x, 1.0, 2, 0.9, 1.0, [], r=0.1) == 2
    # -inf entries get probability 0
    x = np.array([-np.inf, 1.0, -np.inf, 1.0], np.float32)
    assert oracle.sample(x, 1.0, 0, 1.0, 1.0, [], r=0.4) == 1
    assert oracle.sample(x, 1.0, 0, 1.0, 1.0, [], r=0.6) == 3


# --- golden fixtures --------------------------------------------------------
def test_golden_fixtures(oracle):
    import json, os
    path = os.path.join(os.path.dirname(__file__), "golden", "sampler_cases.json")
    cases = json.load(open(path))
    assert len(cases) >= 50
    for c in cases:
        x = np.array(c["logits"], np.float32)
        tok = oracle.sample(x, c["T"], c["k"], c["p"], c["rep"], c["recent"], r=c["u"])
        assert tok == c["token"], c["name"]
