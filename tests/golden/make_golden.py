"""Writes tests/golden/sampler_cases.json: small sampler cases whose expected
tokens come from a second, independent restatement of src/sampler.rs:35-79
written here in pure Python with numpy float32 scalars (one IEEE op per step)
and the C library's expf (the function Rust's f32::exp calls).  The oracle in
oracle/ is checked against these vectors by tests/test_oracle.py.

    python tests/golden/make_golden.py
"""
import ctypes
import ctypes.util
import json
import os

import numpy as np

_libm = ctypes.CDLL(ctypes.util.find_library("m"))
_libm.expf.argtypes = [ctypes.c_float]
_libm.expf.restype = ctypes.c_float
F = np.float32


def expf(x):
    return F(_libm.expf(float(x)))


def ref_sample(logits, T, k, p, rep, recent, u):
    l = [F(v) for v in logits]
    if F(rep) != F(1.0):
        for t in recent:
            if t < len(l):
                l[t] = l[t] / F(rep) if l[t] > F(0.0) else l[t] * F(rep)
    if F(T) <= F(0.0):
        best = 0
        for i in range(1, len(l)):
            if l[i] >= l[best]:
                best = i
        return best
    y = [v / F(T) for v in l]
    pairs = sorted(range(len(y)), key=lambda i: (-float(y[i]), i))
    if 0 < k < len(pairs):
        pairs = pairs[:k]
    m = y[pairs[0]]
    e = [expf(y[i] - m) for i in pairs]
    s = F(0.0)
    for v in e:
        s = F(s + v)
    pr = [F(v / s) for v in e]
    if F(p) < F(1.0):
        cum = F(0.0)
        cut = len(pr)
        for i, v in enumerate(pr):
            cum = F(cum + v)
            if cum >= F(p):
                cut = i + 1
                break
        pairs, pr = pairs[:cut], pr[:cut]
        s2 = F(-0.0)
        for v in pr:
            s2 = F(s2 + v)
        pr = [F(v / s2) for v in pr]
    cum = F(0.0)
    for i, v in zip(pairs, pr):
        cum = F(cum + v)
        if F(u) < cum:
            return i
    return pairs[-1]


def main():
    rng = np.random.default_rng(2024)
    cases = []
    for n in range(120):
        V = int(rng.choice([1, 2, 3, 5, 8, 16, 33, 64, 200]))
        kind = n % 4
        if kind == 0:
            x = (rng.standard_normal(V) * 3).astype(np.float32)
        elif kind == 1:
            x = (rng.integers(-4, 5, size=V) / 2).astype(np.float32)  # ties
        elif kind == 2:
            x = (rng.standard_normal(V) * 0.01).astype(np.float32)    # flat
        else:
            x = (rng.standard_normal(V) * 8).astype(np.float32)       # peaked
        T = float(np.float32(rng.choice([0.0, 0.3, 0.7, 1.0, 1.5])))
        k = int(rng.choice([0, 1, 2, 5, 40, V, V + 3]))
        p = float(np.float32(rng.choice([0.0, 0.5, 0.9, 0.95, 1.0])))
        rep = float(np.float32(rng.choice([1.0, 1.1, 1.3, 0.8])))
        recent = [int(v) for v in rng.integers(0, V + 2, size=int(rng.integers(0, 10)))]
        u = float(np.float32(rng.random()))
        tok = ref_sample(x, T, k, p, rep, recent, u)
        cases.append(dict(name="case%03d" % n, logits=[float(v) for v in x], T=T, k=k, p=p,
                          rep=rep, recent=recent, u=u, token=int(tok)))
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "sampler_cases.json")
    with open(out, "w") as f:
        json.dump(cases, f, indent=0)
    print("wrote", out, len(cases))


if __name__ == "__main__":
    main()
