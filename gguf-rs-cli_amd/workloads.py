"""Synthetic inputs of the five sampler configurations (host side, numpy).

Configurations (one logit row = one call of src/sampler.rs:35 in the
reference's decode loop, src/main.rs:280):

  c1  V=32000,  B=1,    256 sequential steps, N(0,3^2) + 5 spikes U(8,12),
      T=0.7 k=40 p=0.9 rep=1.1, window 64, LCG seed 42 (reference stream)
  c2  V=128256, B=64,   N(0,2.5^2) + 10 spikes U(6,10), T=0.8 k=40 p=0.9
      rep=1.1, 128-id window per row, seeded per-row uniforms
  c3  V=152064, B=256,  N(0,2^2), k=0, p=0.95, T=1.0, rep=1.0
  c4  V=256000, B=512,  heterogeneous rows: T~U(0.3,1.5), k in {0,1,20,100},
      p~U(0.5,1), rep~U(1,1.3), 256-id window, N(0,3^2) + 3 spikes U(5,12)
  c5  V=152064, B=1024, 128 device-resident steps, logits from the on-device
      generator (sigma 3), rep=1.3 T=0.7 k=50 p=0.9, 1024-id ring window

Row counts and step counts can be reduced for tests (`B=`, `steps=`); the
per-row shape and distributions stay the configuration's.
"""
import numpy as np

PARAMS_DTYPE = np.dtype([("temperature", "<f4"), ("top_k", "<u4"), ("top_p", "<f4"),
                         ("rep_penalty", "<f4")])

CONFIGS = {
    "c1": dict(V=32000, B=1, steps=256, W=64, sigma=3.0, spikes=5, spike_lo=8.0, spike_hi=12.0,
               T=0.7, k=40, p=0.9, rep=1.1, seed=42),
    "c2": dict(V=128256, B=64, W=128, sigma=2.5, spikes=10, spike_lo=6.0, spike_hi=10.0,
               T=0.8, k=40, p=0.9, rep=1.1),
    "c3": dict(V=152064, B=256, W=0, sigma=2.0, spikes=0, T=1.0, k=0, p=0.95, rep=1.0),
    "c4": dict(V=256000, B=512, W=256, sigma=3.0, spikes=3, spike_lo=5.0, spike_hi=12.0),
    "c5": dict(V=152064, B=1024, steps=128, W=1024, sigma=3.0, T=0.7, k=50, p=0.9, rep=1.3,
               seed=42, synth_seed=0x5eed),
}


def _rows(rng, B, V, sigma, spikes, lo=0.0, hi=0.0):
    x = rng.standard_normal((B, V), dtype=np.float32)
    x *= np.float32(sigma)
    for b in range(B):
        if spikes:
            pos = rng.choice(V, size=spikes, replace=False)
            x[b, pos] += rng.uniform(lo, hi, size=spikes).astype(np.float32)
    return x


def params_rows(rows):
    return np.array([tuple(r) for r in rows], dtype=PARAMS_DTYPE)


def make(name, B=None, steps=None, seed=1234):
    """Return a dict with logits [B, V] (or [steps, V] for c1), params
    (structured [B]), recent [B, W] uint32 (or None), u [B] f32 (or None)."""
    c = dict(CONFIGS[name])
    rng = np.random.default_rng(seed)
    V = c["V"]
    if name == "c1":
        steps = c["steps"] if steps is None else steps
        logits = _rows(rng, steps, V, c["sigma"], c["spikes"], c["spike_lo"], c["spike_hi"])
        init = rng.integers(0, V, size=c["W"], dtype=np.uint32)
        return dict(name=name, V=V, steps=steps, logits=logits, init_recent=init, W=c["W"],
                    T=c["T"], k=c["k"], p=c["p"], rep=c["rep"], seed=c["seed"])
    if name == "c5":
        B = c["B"] if B is None else B
        steps = c["steps"] if steps is None else steps
        window = rng.integers(0, V, size=(B, c["W"]), dtype=np.uint32)
        return dict(name=name, V=V, B=B, steps=steps, W=c["W"], window=window, sigma=c["sigma"],
                    T=c["T"], k=c["k"], p=c["p"], rep=c["rep"], seed=c["seed"],
                    synth_seed=c["synth_seed"])
    B = c["B"] if B is None else B
    if name == "c4":
        logits = _rows(rng, B, V, c["sigma"], c["spikes"], c["spike_lo"], c["spike_hi"])
        T = rng.uniform(0.3, 1.5, size=B).astype(np.float32)
        k = rng.choice(np.array([0, 1, 20, 100], dtype=np.uint32), size=B)
        p = rng.uniform(0.5, 1.0, size=B).astype(np.float32)
        rep = rng.uniform(1.0, 1.3, size=B).astype(np.float32)
        params = params_rows(zip(T, k, p, rep))
    else:
        logits = _rows(rng, B, V, c["sigma"], c["spikes"], c.get("spike_lo", 0.0), c.get("spike_hi", 0.0))
        params = params_rows([(c["T"], c["k"], c["p"], c["rep"])] * B)
    recent = rng.integers(0, V, size=(B, c["W"]), dtype=np.uint32) if c["W"] else None
    u = rng.random(B, dtype=np.float32)
    return dict(name=name, V=V, B=B, W=c["W"], logits=logits, params=params, recent=recent, u=u)


def lcg_stream(seed, n):
    """The reference LCG (src/sampler.rs:7-12): n draws and the next state."""
    a, c, m = 6364136223846793005, 1442695040888963407, (1 << 64) - 1
    s = seed
    out = np.empty(n, np.float32)
    for i in range(n):
        out[i] = np.float32(s >> 33) / np.float32(4294967295.0)
        s = (s * a + c) & m
    return out, s


def algorithmic_bytes_per_row(V, W, hetero=False, window_append=False):
    """One read of the row, the window (if the penalty is active), the draw,
    the token write, per-row params (heterogeneous only), window append."""
    return 4 * V + 4 * W + 4 + 4 + (16 if hetero else 0) + (4 if window_append else 0)


# ---- quantized output matrices (the logits projection) ------------------------
# GGUF block sizes (src/gguf/types.rs:62-71): Q8_0 34 bytes / 32 weights,
# Q4_K 144, Q5_K 176 and Q6_K 210 bytes / 256 weights.
Q4_0, Q4_1, Q8_0, Q3_K, Q4_K, Q5_K, Q6_K = 2, 3, 8, 11, 12, 13, 14
QBLOCK = {Q4_0: (32, 18), Q4_1: (32, 20), Q8_0: (32, 34), Q3_K: (256, 110), Q4_K: (256, 144),
          Q5_K: (256, 176), Q6_K: (256, 210)}


def qmatrix_bytes(qtype, rows, cols):
    w, b = QBLOCK[qtype]
    return rows * (cols // w) * b


def synth_qblocks(qtype, rows, cols, seed=0, dscale=0.002):
    """Seeded random GGUF blocks for a rows x cols matrix: uniform quant bits,
    int8 sub-block scales and small positive f16 block scales (values like a
    trained output matrix's, about 1e-3..1e-2 per weight)."""
    w, nb = QBLOCK[qtype]
    rng = np.random.default_rng(seed)
    n = rows * (cols // w)
    blk = rng.integers(0, 256, size=(n, nb), dtype=np.uint8)
    d = (rng.random(n) * dscale + dscale / 4).astype(np.float16).view(np.uint8).reshape(n, 2)
    if qtype in (Q8_0, Q4_0):
        blk[:, 0:2] = d
    elif qtype == Q4_1:
        blk[:, 0:2] = d                                       # d; m about -8 d (a centred range)
        blk[:, 2:4] = (-(rng.random(n) * 8 + 4) * dscale / 2).astype(np.float16).view(np.uint8).reshape(n, 2)
    elif qtype == Q3_K:
        blk[:, 108:110] = d
    elif qtype in (Q4_K, Q5_K):
        blk[:, 0:2] = d                                       # d; dmin about a tenth of it
        blk[:, 2:4] = (rng.random(n) * dscale / 10).astype(np.float16).view(np.uint8).reshape(n, 2)
    else:
        blk[:, 192:208] = rng.integers(-64, 64, size=(n, 16)).astype(np.int8).view(np.uint8)
        blk[:, 208:210] = d
    return blk.reshape(-1)
