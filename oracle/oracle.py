"""ctypes binding of the CPU oracle (oracle/liboracle.so).

TEST INFRASTRUCTURE ONLY: the parity checker for the HIP sampler.  Imported
by tests/, __graft_entry__.smoke() and the cpu_baseline leg of bench.py;
never by the product path.  The oracle restates gguf-rs-cli src/sampler.rs
(see sampler_oracle.c for the per-function citations) and the Q8_0 / Q6_K
dequantization and matvec of src/tensor/dequant.rs (gemv_oracle.c).
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

ERR_NAN = -3
ERR_EMPTY = -2


class OracleParams(ctypes.Structure):
    _fields_ = [("temperature", ctypes.c_float), ("top_k", ctypes.c_uint32),
                ("top_p", ctypes.c_float), ("rep_penalty", ctypes.c_float)]


class OracleDetail(ctypes.Structure):
    _fields_ = [("idx", ctypes.POINTER(ctypes.c_uint32)), ("p", ctypes.POINTER(ctypes.c_float)),
                ("cap", ctypes.c_size_t), ("n_kept", ctypes.c_size_t), ("cut", ctypes.c_size_t),
                ("sum", ctypes.c_float), ("s2", ctypes.c_float), ("r", ctypes.c_float),
                ("q_last", ctypes.c_float)]


PARAMS_DTYPE = np.dtype([("temperature", "<f4"), ("top_k", "<u4"), ("top_p", "<f4"),
                         ("rep_penalty", "<f4")])

_lib = None


def load(build_if_missing=True):
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH) and build_if_missing:
        subprocess.run(["make", "-s", "-C", HERE, "liboracle.so"], check=True)
    lib = ctypes.CDLL(LIB_PATH)
    P, SZ, F, U64 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_float, ctypes.c_uint64
    lib.oracle_set_seed.argtypes = [U64]
    lib.oracle_get_seed.restype = U64
    lib.oracle_lcg_draw.argtypes = [ctypes.POINTER(U64)]
    lib.oracle_lcg_draw.restype = F
    lib.oracle_sample_ex.argtypes = [P, SZ, F, SZ, F, F, P, SZ, F, P, ctypes.c_int, P]
    lib.oracle_sample_ex.restype = ctypes.c_int64
    lib.oracle_sample.argtypes = [P, SZ, F, SZ, F, F, P, SZ]
    lib.oracle_sample.restype = ctypes.c_int64
    lib.oracle_sample_batch.argtypes = [P, SZ, SZ, SZ, P, P, SZ, P, SZ, P, P, ctypes.c_int, ctypes.c_int]
    lib.oracle_decode_trace.argtypes = [P, SZ, SZ, F, SZ, F, F, SZ, P, SZ, U64, P, ctypes.c_int]
    lib.oracle_generate.argtypes = [P, SZ, SZ, F, SZ, F, F, SZ, P, SZ, P, SZ, SZ, P, P, P, P, P, P, P]
    lib.oracle_synth_logit.argtypes = [U64, U64, F]
    lib.oracle_synth_logit.restype = F
    lib.oracle_synth_logits.argtypes = [P, SZ, U64, U64, F]
    lib.oracle_device_loop.argtypes = [SZ, SZ, SZ, U64, F, P, P, SZ, P, P, ctypes.c_int, ctypes.c_int]
    lib.oracle_now.restype = ctypes.c_double
    lib.oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
    lib.oracle_f16_to_f32.restype = F
    lib.oracle_dequant_q8_0.argtypes = [P, SZ, P]
    lib.oracle_dequant_q6_k.argtypes = [P, SZ, P]
    lib.oracle_dequant_q4_k.argtypes = [P, SZ, P]
    lib.oracle_dequant_q5_k.argtypes = [P, SZ, P]
    lib.oracle_dequant_q4_0.argtypes = [P, SZ, P]
    lib.oracle_dequant_q4_1.argtypes = [P, SZ, P]
    lib.oracle_dequant_q3_k.argtypes = [P, SZ, P]
    lib.oracle_row_dot.argtypes = [ctypes.c_uint32, P, SZ, P]
    lib.oracle_row_dot.restype = F
    lib.oracle_matvec.argtypes = [ctypes.c_uint32, P, SZ, SZ, P, P, P, P, ctypes.c_int]
    _lib = lib
    return lib


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _u32(a):
    return np.ascontiguousarray(a, dtype=np.uint32)


def set_seed(s):
    load().oracle_set_seed(s)


def get_seed():
    return load().oracle_get_seed()


def lcg_draws(seed, n):
    """n draws of the reference LCG from `seed`; returns (draws, final state)."""
    lib = load()
    st = ctypes.c_uint64(seed)
    out = np.empty(n, np.float32)
    for i in range(n):
        out[i] = lib.oracle_lcg_draw(ctypes.byref(st))
    return out, st.value


def sample(logits, temperature, top_k, top_p, rep_penalty, recent=(), r=None, state=None,
           fast_topk=False, detail=False):
    """One reference sample.  `logits` is copied (the reference mutates it;
    the mutated copy is returned in detail['logits']).  Draw: r, or the LCG
    `state` (an int; the advanced state is returned in detail), or the
    oracle's global LCG when both are None."""
    lib = load()
    row = _f32(np.array(logits, dtype=np.float32, copy=True))
    rec = _u32(recent if recent is not None else [])
    det = None
    if detail:
        cap = row.size
        idx = np.zeros(max(cap, 1), np.uint32)
        p = np.zeros(max(cap, 1), np.float32)
        det = OracleDetail(idx.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)),
                           p.ctypes.data_as(ctypes.POINTER(ctypes.c_float)), cap, 0, 0, 0, 0, 0, 0)
    if r is None and state is None:
        tok = lib.oracle_sample(row.ctypes.data, row.size, temperature, top_k, top_p, rep_penalty,
                                rec.ctypes.data if rec.size else None, rec.size)
        st = None
    else:
        stv = ctypes.c_uint64(state if state is not None else 0)
        use_state = state is not None and temperature > 0
        tok = lib.oracle_sample_ex(row.ctypes.data, row.size, temperature, top_k, top_p,
                                   rep_penalty, rec.ctypes.data if rec.size else None, rec.size,
                                   0.0 if r is None else r,
                                   ctypes.addressof(stv) if use_state else None,
                                   1 if fast_topk else 0, ctypes.addressof(det) if det else None)
        st = stv.value if state is not None else None
    if not detail:
        return tok
    n = det.n_kept
    return tok, {"logits": row, "idx": idx[:n].copy(), "p": p[:n].copy(), "cut": det.cut,
                 "sum": det.sum, "s2": det.s2, "r": det.r, "state": st}


def sample_batch(logits, params, u, recent=None, recent_len=None, nthreads=1, fast_topk=False):
    """Reference sample per row with explicit draws.  params: structured array
    (PARAMS_DTYPE) of B rows.  Returns int64 tokens (negative = error)."""
    lib = load()
    lg = _f32(logits)
    B, V = lg.shape
    pr = np.ascontiguousarray(params, dtype=PARAMS_DTYPE)
    uu = _f32(u)
    W = 0
    rec_p, ldr, rl_p = None, 0, None
    if recent is not None:
        rec = _u32(recent)
        W, ldr, rec_p = rec.shape[1], rec.shape[1], rec.ctypes.data
    if recent_len is not None:
        rl = _u32(recent_len)
        rl_p = rl.ctypes.data
    tok = np.empty(B, np.int64)
    st = lib.oracle_sample_batch(lg.ctypes.data, B, V, V, pr.ctypes.data, rec_p, ldr, rl_p, W,
                                 uu.ctypes.data, tok.ctypes.data, nthreads, 1 if fast_topk else 0)
    if st:
        raise RuntimeError("oracle_sample_batch failed: %d" % st)
    return tok


def decode_trace(logits, temperature, top_k, top_p, rep_penalty, window, init_recent, seed,
                 fast_topk=False):
    """Sequential decode loop of src/main.rs:279-311 over given per-step logits."""
    lib = load()
    lg = _f32(logits)
    steps, V = lg.shape
    ir = _u32(init_recent)
    tok = np.empty(steps, np.int64)
    st = lib.oracle_decode_trace(lg.ctypes.data, steps, V, temperature, top_k, top_p, rep_penalty,
                                 window, ir.ctypes.data if ir.size else None, ir.size, seed,
                                 tok.ctypes.data, 1 if fast_topk else 0)
    if st:
        raise RuntimeError("oracle_decode_trace failed: %d" % st)
    return tok


def generate(logits, params, window, init_recent, stops, max_new, seed):
    """generate_collect (src/main.rs:258-313) for one row over per-step
    logits [steps, V].  Returns a dict: sampled (tokens of the steps taken),
    generated, done (0 out of steps, 1 stop, 2 max), state (final LCG state),
    recent (final FIFO, oldest first)."""
    lib = load()
    lg = _f32(logits)
    steps, V = lg.shape
    T, k, p, rep = params
    ir = _u32(init_recent)
    sp = _u32(stops)
    st = ctypes.c_uint64(seed)
    sampled = np.zeros(steps, np.int64)
    n_steps, n_gen, rl = ctypes.c_size_t(), ctypes.c_size_t(), ctypes.c_size_t()
    done = ctypes.c_int()
    rec = np.zeros(max(window, 1), np.uint32)
    rc = lib.oracle_generate(lg.ctypes.data, steps, V, T, k, p, rep, window,
                             ir.ctypes.data if ir.size else None, ir.size,
                             sp.ctypes.data if sp.size else None, sp.size, max_new,
                             ctypes.byref(st), sampled.ctypes.data, ctypes.byref(n_steps),
                             ctypes.byref(n_gen), ctypes.byref(done), rec.ctypes.data, ctypes.byref(rl))
    if rc:
        raise RuntimeError("oracle_generate failed: %d" % rc)
    s = sampled[:n_steps.value]
    return {"sampled": s, "generated": s[:n_gen.value].astype(np.uint32), "done": done.value,
            "state": st.value, "recent": rec[:rl.value].copy()}


def synth_logits(n, seed, counter0, sigma):
    lib = load()
    out = np.empty(n, np.float32)
    lib.oracle_synth_logits(out.ctypes.data, n, seed, counter0, sigma)
    return out


def device_loop(B, V, steps, seed, sigma, params, window, u, nthreads=1, fast_topk=True):
    """Host restatement of the device-resident loop: returns tokens [steps, B]
    and the final window (modified copy)."""
    lib = load()
    p = OracleParams(*params)
    win = _u32(np.array(window, dtype=np.uint32, copy=True))
    uu = _f32(u)
    tok = np.empty(steps * B, np.int64)
    st = lib.oracle_device_loop(B, V, steps, seed, sigma, ctypes.addressof(p), win.ctypes.data,
                                win.shape[1], uu.ctypes.data, tok.ctypes.data, nthreads,
                                1 if fast_topk else 0)
    if st:
        raise RuntimeError("oracle_device_loop failed: %d" % st)
    return tok.reshape(steps, B), win


def now():
    return load().oracle_now()


# ---- quantized matvec (src/tensor/dequant.rs) -------------------------------
QT_Q4_0 = 2
QT_Q4_1 = 3
QT_Q8_0 = 8
QT_Q3_K = 11
QT_Q4_K = 12
QT_Q5_K = 13
QT_Q6_K = 14


def dequant(qtype, blocks, n):
    """dq40 / dq41 / dq80 / dq4k / dq5k / dq6k (src/tensor/dequant.rs:26-54,
    86-94, 141-219) and Q3_K in the GGUF layout: n f32 weights."""
    lib = load()
    b = np.ascontiguousarray(blocks, dtype=np.uint8)
    out = np.empty(n, np.float32)
    f = {QT_Q8_0: lib.oracle_dequant_q8_0, QT_Q4_K: lib.oracle_dequant_q4_k,
         QT_Q5_K: lib.oracle_dequant_q5_k, QT_Q6_K: lib.oracle_dequant_q6_k,
         QT_Q4_0: lib.oracle_dequant_q4_0, QT_Q4_1: lib.oracle_dequant_q4_1,
         QT_Q3_K: lib.oracle_dequant_q3_k}[qtype]
    f(b.ctypes.data, n, out.ctypes.data)
    return out


def row_dot(qtype, row_blocks, cols, x):
    """QuantTensor::row_dot (src/tensor/dequant.rs:277-313), f32 result."""
    lib = load()
    b = np.ascontiguousarray(row_blocks, dtype=np.uint8)
    xx = _f32(x)
    return float(np.float32(lib.oracle_row_dot(qtype, b.ctypes.data, cols, xx.ctypes.data)))


def matvec(qtype, blocks, rows, cols, x, nthreads=1, exact=False):
    """QuantTensor::matvec (src/tensor/dequant.rs:315-318).  Returns the
    reference's f32 outputs, or with exact=True (float64 exact values of the
    reference's weights times x, float64 sums of |w x|)."""
    lib = load()
    b = np.ascontiguousarray(blocks, dtype=np.uint8)
    xx = _f32(x)
    if exact:
        ex = np.empty(rows, np.float64)
        ab = np.empty(rows, np.float64)
        rc = lib.oracle_matvec(qtype, b.ctypes.data, rows, cols, xx.ctypes.data, None,
                               ex.ctypes.data, ab.ctypes.data, nthreads)
        assert rc == 0
        return ex, ab
    out = np.empty(rows, np.float32)
    rc = lib.oracle_matvec(qtype, b.ctypes.data, rows, cols, xx.ctypes.data, out.ctypes.data,
                           None, None, nthreads)
    assert rc == 0
    return out
