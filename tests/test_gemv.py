"""The quantized output projection (the logits producer, src/model/llama.rs:333-334):
CPU pins of the oracle's Q4_0 / Q4_1 / Q8_0 / Q3_K / Q4_K / Q5_K / Q6_K
dequantization and matvec (src/tensor/dequant.rs:26-54, 86-94, 141-219,
277-318), and GPU parity of gs_gemv (include/gs_gemv.h) against it.  Q5_K
follows the GGUF format where the reference cannot (its dq5k indexes past its
32-byte qh slice from the third step on, src/tensor/dequant.rs:177,192), and
Q3_K where the reference's two paths disagree with each other and with the
format (dq3k :120-140, q3k_gemv.glsl): their pins are the format's bit layout,
not reference outputs.

The GPU sums in its own order, so parity is a tolerance: with exact the
float64 value of the reference's f32 weights times x (oracle.matvec exact=True),
|gpu - exact| <= 2^-16 * (sum |w x| + 64 * max|d scale| * sum |x|).  The second
term covers the per-group offset (sum (u - o) x = sum u x - o sum x) the kernel
uses; a wrong weight index or scale moves a row by a whole |w x| term, far
above the bound.
"""
import numpy as np
import pytest

Q4_0, Q4_1, Q8_0, Q3_K, Q4_K, Q5_K, Q6_K = 2, 3, 8, 11, 12, 13, 14


def _f32_bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


# ---- oracle pins (CPU) ------------------------------------------------------
def test_f16_conversion_all_patterns(oracle):
    """half::f16::to_f32 is an exact conversion: every pattern against numpy."""
    lib = oracle.load()
    h = np.arange(65536, dtype=np.uint32)
    want = h.astype(np.uint16).view(np.float16).astype(np.float32)
    got = np.array([lib.oracle_f16_to_f32(int(v)) for v in h], np.float32)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(_f32_bits(got[~nan]), _f32_bits(want[~nan]))


def _q6_block(ql=None, qh=None, sc=None, d=1.0):
    b = np.zeros(210, np.uint8)
    if ql is not None:
        b[0:128] = ql
    if qh is not None:
        b[128:192] = qh
    b[192:208] = np.asarray(sc if sc is not None else np.ones(16), np.int8).view(np.uint8)
    b[208:210] = np.array([d], np.float16).view(np.uint8)
    return b


def test_q6k_zero_block_and_linearity(oracle):
    """All quant bits 0 give q = -32 everywhere; weights scale with d and with
    each sub-block scale (16 weights per scale, in order)."""
    sc = np.arange(1, 17)
    w = oracle.dequant(Q6_K, _q6_block(sc=sc, d=0.5), 256)
    assert np.array_equal(w, (-32.0 * 0.5 * np.repeat(sc, 16)).astype(np.float32))
    w2 = oracle.dequant(Q6_K, _q6_block(sc=-sc, d=0.25), 256)
    assert np.array_equal(w2, (32.0 * 0.25 * np.repeat(sc, 16)).astype(np.float32))


def test_q6k_single_bit_probes(oracle):
    """Each quant bit moves exactly one weight, by the value of that bit times
    d * scale, at the position the GGML Q6_K layout gives it: ql byte 64h + l
    holds weights 128h + l (low nibble) and 128h + l + 64 (high), ql byte
    64h + 32 + l weights 128h + l + 32 and + 96; qh byte 32h + l holds bits
    4-5 of those four weights, two bits each, in that order (0, 32, 64, 96)."""
    base = oracle.dequant(Q6_K, _q6_block(sc=np.full(16, 3), d=2.0), 256)
    for h in range(2):
        for l in (0, 5, 31):
            for nib, off in ((0, 0), (4, 64)):
                for k, (byte, woff) in enumerate(((64 * h + l, 0), (64 * h + 32 + l, 32))):
                    for bit in range(4):
                        ql = np.zeros(128, np.uint8)
                        ql[byte] = 1 << (nib + bit)
                        w = oracle.dequant(Q6_K, _q6_block(ql=ql, sc=np.full(16, 3), d=2.0), 256)
                        diff = np.nonzero(w != base)[0]
                        assert list(diff) == [128 * h + l + woff + off], (h, l, nib, k, bit, diff)
                        assert w[diff[0]] - base[diff[0]] == (1 << bit) * 6.0
            for pair, woff in enumerate((0, 32, 64, 96)):
                for bit in range(2):
                    qh = np.zeros(64, np.uint8)
                    qh[32 * h + l] = 1 << (2 * pair + bit)
                    w = oracle.dequant(Q6_K, _q6_block(qh=qh, sc=np.full(16, 3), d=2.0), 256)
                    diff = np.nonzero(w != base)[0]
                    assert list(diff) == [128 * h + l + woff], (h, l, pair, bit, diff)
                    assert w[diff[0]] - base[diff[0]] == (16 << bit) * 6.0


def _k_block(q5, qs=None, qh=None, scales=None, d=1.0, dmin=0.0):
    b = np.zeros(176 if q5 else 144, np.uint8)
    b[0:2] = np.array([d], np.float16).view(np.uint8)
    b[2:4] = np.array([dmin], np.float16).view(np.uint8)
    if scales is not None:
        b[4:16] = scales
    if q5 and qh is not None:
        b[16:48] = qh
    if qs is not None:
        b[(48 if q5 else 16):] = qs
    return b


# GGML's packing of the eight 6-bit (scale, min) pairs in 12 bytes, bit by
# bit: (byte, bit) -> (sub-block, 0 = scale / 1 = min, bit of the value).
def _k_scale_bits():
    tab = {}
    for j in range(4):
        for bit in range(6):
            tab[(j, bit)] = (j, 0, bit)                 # bytes 0-3: scales 0-3
            tab[(j + 4, bit)] = (j, 1, bit)             # bytes 4-7: mins 0-3
        for bit in (6, 7):
            tab[(j, bit)] = (j + 4, 0, bit - 2)         # top bits of scales 4-7
            tab[(j + 4, bit)] = (j + 4, 1, bit - 2)     # top bits of mins 4-7
        for bit in range(4):
            tab[(j + 8, bit)] = (j + 4, 0, bit)         # bytes 8-11: low nibbles of scales 4-7
            tab[(j + 8, bit + 4)] = (j + 4, 1, bit)     # high nibbles: mins 4-7
    return tab


@pytest.mark.parametrize("qt", [Q4_K, Q5_K])
def test_kquant_scale_min_bit_probes(oracle, qt):
    """Every bit of the 12 scale bytes changes exactly the 32 weights of the
    sub-block GGML's layout gives it, by the bit's value times d (scale) or
    -dmin (min); with all quants 1 (d = 1, dmin = 0.5) a weight is
    sc - 0.5 m."""
    q5 = qt == Q5_K
    qs = np.full(128, 0x11, np.uint8)          # every quant 1
    base = oracle.dequant(qt, _k_block(q5, qs=qs, d=1.0, dmin=0.5), 256)
    assert np.all(base == 0.0)
    for (byte, bit), (sub, kind, vbit) in _k_scale_bits().items():
        sc = np.zeros(12, np.uint8)
        sc[byte] = 1 << bit
        w = oracle.dequant(qt, _k_block(q5, qs=qs, scales=sc, d=1.0, dmin=0.5), 256)
        diff = np.nonzero(w != base)[0]
        assert list(diff) == list(range(32 * sub, 32 * sub + 32)), (byte, bit, diff[:4])
        want = (1 << vbit) * (1.0 if kind == 0 else -0.5)
        assert np.all(w[diff] == np.float32(want)), (byte, bit, w[diff[0]], want)


@pytest.mark.parametrize("qt", [Q4_K, Q5_K])
def test_kquant_quant_bit_probes(oracle, qt):
    """Each quant bit moves one weight by the bit's value times d * sc: qs
    byte 32 s + l holds weight 64 s + l (low nibble) and 64 s + 32 + l (high);
    for Q5_K bit 2 s / 2 s + 1 of qh[l] is the fifth bit (16) of those two.
    Scales 1..8 per sub-block (min 0), d = 0.25."""
    q5 = qt == Q5_K
    sc = np.zeros(12, np.uint8)
    sc[0:4] = [1, 2, 3, 4]
    sc[8:12] = [5, 6, 7, 8]                    # scales 4-7: low nibbles of bytes 8-11
    scale = np.array([1, 2, 3, 4, 5, 6, 7, 8], np.float32)
    base = oracle.dequant(qt, _k_block(q5, scales=sc, d=0.25), 256)
    assert np.all(base == 0.0)
    for s_ in range(4):
        for l in (0, 9, 31):
            for nib in range(2):
                for bit in range(4):
                    qs = np.zeros(128, np.uint8)
                    qs[32 * s_ + l] = 1 << (4 * nib + bit)
                    w = oracle.dequant(qt, _k_block(q5, qs=qs, scales=sc, d=0.25), 256)
                    diff = np.nonzero(w != base)[0]
                    pos = 64 * s_ + 32 * nib + l
                    assert list(diff) == [pos], (s_, l, nib, bit, diff)
                    assert w[pos] == np.float32((1 << bit) * 0.25 * scale[2 * s_ + nib])
            if q5:
                for nib in range(2):
                    qh = np.zeros(32, np.uint8)
                    qh[l] = 1 << (2 * s_ + nib)
                    w = oracle.dequant(qt, _k_block(q5, qh=qh, scales=sc, d=0.25), 256)
                    diff = np.nonzero(w != base)[0]
                    pos = 64 * s_ + 32 * nib + l
                    assert list(diff) == [pos], (s_, l, nib, diff)
                    assert w[pos] == np.float32(16 * 0.25 * scale[2 * s_ + nib])


def test_q8_0_bytes_and_scale(oracle):
    """Q8_0: byte 2 + i is weight i as int8, times the f16 d in bytes 0-1."""
    q = np.arange(-128, 128, 8, dtype=np.int8)[:32]
    b = np.concatenate([np.array([0.125], np.float16).view(np.uint8), q.view(np.uint8)])
    w = oracle.dequant(Q8_0, b, 32)
    assert np.array_equal(w, q.astype(np.float32) * np.float32(0.125))


def test_q4_0_q4_1_nibbles(oracle):
    """dq40 / dq41: byte 2 + l (Q4_1: 4 + l) holds weight l in its low nibble
    and weight l + 16 in its high nibble; Q4_0 w = (q - 8) d, Q4_1 w = q d + m."""
    q = np.arange(32) % 16
    nib = (q[:16] | (q[16:][::-1] << 4)).astype(np.uint8)      # high nibbles reversed
    want_q = np.concatenate([q[:16], q[16:][::-1]]).astype(np.float32)
    d = np.array([0.375], np.float16)
    b0 = np.concatenate([d.view(np.uint8), nib])
    assert np.array_equal(oracle.dequant(Q4_0, b0, 32), (want_q - 8) * np.float32(0.375))
    m = np.array([-2.5], np.float16)
    b1 = np.concatenate([d.view(np.uint8), m.view(np.uint8), nib])
    assert np.array_equal(oracle.dequant(Q4_1, b1, 32), want_q * np.float32(0.375) + np.float32(-2.5))


def _q3_block(hmask=None, qs=None, scales=None, d=1.0):
    b = np.zeros(110, np.uint8)
    if hmask is not None:
        b[0:32] = hmask
    if qs is not None:
        b[32:96] = qs
    if scales is not None:
        b[96:108] = scales
    b[108:110] = np.array([d], np.float16).view(np.uint8)
    return b


# GGUF's packing of the sixteen 6-bit Q3_K scales in 12 bytes, bit by bit:
# (byte, bit) -> (sub-block of 16 weights, bit of the value).
def _q3_scale_bits():
    tab = {}
    for j in range(4):
        for bit in range(4):
            tab[(j, bit)] = (j, bit)                    # bytes 0-3 low nibbles: scales 0-3
            tab[(j, bit + 4)] = (8 + j, bit)            # high nibbles: scales 8-11
            tab[(4 + j, bit)] = (4 + j, bit)            # bytes 4-7: scales 4-7
            tab[(4 + j, bit + 4)] = (12 + j, bit)       # and 12-15
        for k in range(4):
            for hb in range(2):
                tab[(8 + j, 2 * k + hb)] = (4 * k + j, 4 + hb)   # bytes 8-11: top two bits
    return tab


def test_q3k_scale_bit_probes(oracle):
    """Every bit of the 12 scale bytes moves exactly the 16 weights of the
    sub-block GGUF's layout gives it, by the bit's value times d q; all quants
    1 (low bits 01, third bit set), scales 0 (value -32), d = 0.5."""
    hm = np.full(32, 0xFF, np.uint8)
    qs = np.full(64, 0x55, np.uint8)
    base = oracle.dequant(Q3_K, _q3_block(hm, qs, d=0.5), 256)
    assert np.all(base == np.float32(-16.0))
    tab = _q3_scale_bits()
    assert len(tab) == 96
    for (byte, bit), (sub, vbit) in tab.items():
        sc = np.zeros(12, np.uint8)
        sc[byte] = 1 << bit
        w = oracle.dequant(Q3_K, _q3_block(hm, qs, sc, d=0.5), 256)
        diff = np.nonzero(w != base)[0]
        assert list(diff) == list(range(16 * sub, 16 * sub + 16)), (byte, bit, diff[:4])
        assert np.all(w[diff] == np.float32(0.5 * ((1 << vbit) - 32))), (byte, bit, w[diff[0]])


def test_q3k_quant_bit_probes(oracle):
    """Bits 2j, 2j+1 of qs[32 n + l] are the low bits (1, 2) of weight
    128 n + 32 j + l, bit 4 n + j of hmask[l] its third bit (4); with all
    bits clear every weight is q = -4.  Scales 1..16 (bytes give value
    s + 32), d = 0.25."""
    sc_val = np.arange(1, 17)
    raw = sc_val + 32                                   # 6-bit stored values
    sc = np.zeros(12, np.uint8)
    for i, v in enumerate(raw):
        k, j = i >> 2, i & 3
        lo, hi = v & 0xF, v >> 4
        sc[(k & 1) * 4 + j] |= lo << (0 if k < 2 else 4)
        sc[8 + j] |= hi << (2 * k)
    base = oracle.dequant(Q3_K, _q3_block(scales=sc, d=0.25), 256)
    assert np.array_equal(base, (-4.0 * 0.25 * np.repeat(sc_val, 16)).astype(np.float32))
    for n in range(2):
        for j in range(4):
            for l in (0, 5, 16, 31):
                pos = 128 * n + 32 * j + l
                for c in range(2):
                    qs = np.zeros(64, np.uint8)
                    qs[32 * n + l] = 1 << (2 * j + c)
                    w = oracle.dequant(Q3_K, _q3_block(qs=qs, scales=sc, d=0.25), 256)
                    diff = np.nonzero(w != base)[0]
                    assert list(diff) == [pos], (n, j, l, c, diff)
                    assert w[pos] == np.float32(0.25 * sc_val[pos // 16] * ((1 << c) - 4))
                hm = np.zeros(32, np.uint8)
                hm[l] = 1 << (4 * n + j)
                w = oracle.dequant(Q3_K, _q3_block(hmask=hm, scales=sc, d=0.25), 256)
                diff = np.nonzero(w != base)[0]
                assert list(diff) == [pos], (n, j, l, diff)
                assert w[pos] == np.float32(0.0)


def test_q4_0_row_dot_order(oracle):
    """row_dot's Q4_0 arm (dequant.rs:289-298): per block a sequential f32 sum
    over j of (lo_j + hi_j), lo_j = ((q_j - 8) d) x_j, hi_j the same for weight
    j + 16; then a sequential sum of the block sums."""
    import workloads
    rng = np.random.default_rng(11)
    cols = 160
    blocks = workloads.synth_qblocks(Q4_0, 1, cols, seed=12)
    x = rng.standard_normal(cols).astype(np.float32)
    w = oracle.dequant(Q4_0, blocks, cols)
    acc = np.float32(0.0)
    for b in range(cols // 32):
        s = np.float32(0.0)
        for j in range(16):
            s = np.float32(s + np.float32(np.float32(w[32 * b + j] * x[32 * b + j])
                                          + np.float32(w[32 * b + 16 + j] * x[32 * b + 16 + j])))
        acc = np.float32(acc + s)
    assert np.float32(oracle.row_dot(Q4_0, blocks, cols, x)) == acc


def test_row_dot_order_and_unit_vectors(oracle):
    """row_dot: Q6_K sums w * x left to right in f32 (numpy's sequential
    accumulate); Q8_0 sums each block left to right, then the block sums.
    A unit vector picks one weight exactly."""
    import workloads
    rng = np.random.default_rng(3)
    for qt, cols in ((Q6_K, 512), (Q8_0, 96), (Q4_K, 512), (Q5_K, 512), (Q4_1, 96), (Q3_K, 512)):
        blocks = workloads.synth_qblocks(qt, 1, cols, seed=5)
        w = oracle.dequant(qt, blocks, cols)
        x = rng.standard_normal(cols).astype(np.float32)
        got = oracle.row_dot(qt, blocks, cols, x)
        p = (w * x).astype(np.float32) if qt != Q8_0 else None
        if qt != Q8_0:
            want = np.add.accumulate(p, dtype=np.float32)[-1]
        else:
            q = blocks.reshape(-1, 34)[:, 2:].view(np.int8).astype(np.float32)
            d = blocks.reshape(-1, 34)[:, :2].copy().view(np.float16).astype(np.float32)
            pb = (q * d[:, :1]).astype(np.float32) * x.reshape(-1, 32)
            sums = np.array([np.add.accumulate(r, dtype=np.float32)[-1] for r in pb], np.float32)
            want = np.add.accumulate(sums, dtype=np.float32)[-1]
        assert np.float32(got) == want, (qt, got, want)
        for k in (0, 7, cols - 1):
            e = np.zeros(cols, np.float32)
            e[k] = 1.0
            assert np.float32(oracle.row_dot(qt, blocks, cols, e)) == w[k]


def test_matvec_exact_bound(oracle):
    """The reference's sequential f32 sums stay within n * 2^-24 * sum|w x| of
    the exact value; matvec rows equal row_dot."""
    import workloads
    rng = np.random.default_rng(4)
    for qt, rows, cols in ((Q6_K, 20, 1024), (Q8_0, 20, 1024), (Q4_K, 20, 1024), (Q5_K, 20, 1024),
                           (Q4_0, 20, 1024), (Q4_1, 20, 1024), (Q3_K, 20, 1024)):
        blocks = workloads.synth_qblocks(qt, rows, cols, seed=6)
        x = rng.standard_normal(cols).astype(np.float32)
        f32 = oracle.matvec(qt, blocks, rows, cols, x, nthreads=2)
        ex, ab = oracle.matvec(qt, blocks, rows, cols, x, nthreads=2, exact=True)
        assert np.all(np.abs(f32 - ex) <= cols * 2.0 ** -24 * ab)
        rb = workloads.qmatrix_bytes(qt, 1, cols)
        for r in (0, rows - 1):
            assert np.float32(oracle.row_dot(qt, blocks[r * rb:(r + 1) * rb], cols, x)) == f32[r]


# ---- GPU parity ---------------------------------------------------------------
def _gpu_check(gpu, torch, oracle, qt, rows, cols, seed, B=1, x_kind="normal"):
    import workloads
    rng = np.random.default_rng(seed)
    blocks = workloads.synth_qblocks(qt, rows, cols, seed=seed)
    if x_kind == "normal":
        x = rng.standard_normal((B, cols)).astype(np.float32)
    elif x_kind == "spiky":
        x = (rng.standard_normal((B, cols)) * np.exp(rng.standard_normal((B, cols)) * 2)).astype(np.float32)
    else:
        x = np.zeros((B, cols), np.float32)
        x[:, rng.integers(0, cols, 3)] = 1.0
    m = gpu.QMatrix(qt, blocks, rows, cols)
    d_x = torch.from_numpy(x).cuda()
    d_o = torch.full((B, rows), float("nan"), dtype=torch.float32, device="cuda")
    m.gemv(d_x, d_o, B=B)
    torch.cuda.synchronize()
    got = d_o.cpu().numpy()
    m.close()
    if qt == Q6_K:
        smax = np.abs(blocks.reshape(-1, 210)[:, 192:208].view(np.int8)).max() * \
            blocks.reshape(-1, 210)[:, 208:210].copy().view(np.float16).astype(np.float64).max()
    elif qt in (Q4_K, Q5_K):
        # the kernel takes (d sc) sum q x - (dmin m) sum x per 32 weights
        kb = blocks.reshape(-1, 176 if qt == Q5_K else 144)
        dd = kb[:, 0:4].copy().view(np.float16).astype(np.float64)
        smax = 63.0 * (dd[:, 0].max() + dd[:, 1].max())
    elif qt in (Q4_0, Q4_1):
        # d (sum q x - 8 sum x) / d sum q x + m sum x per block
        kb = blocks.reshape(-1, 20 if qt == Q4_1 else 18)
        dd = np.abs(kb[:, 0:4 if qt == Q4_1 else 2].copy().view(np.float16).astype(np.float64))
        smax = 16.0 * dd[:, 0].max() + (dd[:, 1].max() if qt == Q4_1 else 0.0)
    elif qt == Q3_K:
        # (d sc) (sum u x - 4 sum x) per 16 weights, |sc| <= 32
        smax = 32.0 * blocks.reshape(-1, 110)[:, 108:110].copy().view(np.float16).astype(np.float64).max()
    else:
        smax = blocks.reshape(-1, 34)[:, :2].copy().view(np.float16).astype(np.float64).max()
    for b in range(B):
        ex, ab = oracle.matvec(qt, blocks, rows, cols, x[b], nthreads=8, exact=True)
        tol = 2.0 ** -16 * (ab + 64 * smax * np.abs(x[b]).astype(np.float64).sum())
        err = np.abs(got[b].astype(np.float64) - ex)
        bad = np.nonzero(~(err <= tol))[0]
        assert bad.size == 0, (qt, rows, cols, b, bad[:5], got[b][bad[:5]], ex[bad[:5]], tol[bad[:5]])


@pytest.mark.gpu
@pytest.mark.parametrize("qt,rows,cols", [
    (Q6_K, 1000, 3584),      # Qwen2.5-7B hidden size (register path, 56 of 64 lanes)
    (Q6_K, 517, 4096),       # Llama hidden size (all 64 lanes)
    (Q6_K, 37, 256),         # one block per row
    (Q6_K, 300, 8192),       # LDS path
    (Q6_K, 9, 16384),        # largest row
    (Q8_0, 1000, 4096),      # Llama-2 hidden size (4 half blocks per lane)
    (Q8_0, 333, 3584),
    (Q8_0, 77, 32),          # one block per row
    (Q8_0, 200, 8192),       # LDS path
    (Q4_K, 1000, 3584),      # register path, 56 of 64 lanes
    (Q4_K, 517, 4096),
    (Q4_K, 37, 256),
    (Q4_K, 300, 8192),       # LDS path
    (Q5_K, 1000, 3584),
    (Q5_K, 517, 4096),
    (Q5_K, 37, 256),
    (Q5_K, 300, 8192),
    (Q4_0, 1000, 3584),      # register path: 112 blocks, 2 per lane
    (Q4_0, 517, 4096),
    (Q4_0, 77, 32),          # one block per row
    (Q4_0, 200, 8192),       # LDS path
    (Q4_1, 1000, 3584),
    (Q4_1, 77, 32),
    (Q4_1, 200, 8192),
    (Q3_K, 1000, 3584),      # register path, 56 of 64 lanes
    (Q3_K, 517, 4096),
    (Q3_K, 37, 256),
    (Q3_K, 300, 8192),       # LDS path
])
def test_gemv_parity(gpu, torch, oracle, qt, rows, cols):
    _gpu_check(gpu, torch, oracle, qt, rows, cols, seed=rows + cols)


@pytest.mark.gpu
def test_gemv_inputs(gpu, torch, oracle):
    """Heavy-tailed and sparse x, several vectors per call, a row count below
    the number of waves and one far above it."""
    _gpu_check(gpu, torch, oracle, Q6_K, 2000, 3584, seed=1, x_kind="spiky")
    _gpu_check(gpu, torch, oracle, Q8_0, 2000, 4096, seed=2, x_kind="sparse")
    _gpu_check(gpu, torch, oracle, Q6_K, 64, 3584, seed=3, B=3)
    _gpu_check(gpu, torch, oracle, Q6_K, 5, 1024, seed=4)
    _gpu_check(gpu, torch, oracle, Q8_0, 40000, 1024, seed=5)
    _gpu_check(gpu, torch, oracle, Q4_K, 2000, 3584, seed=6, x_kind="spiky")
    _gpu_check(gpu, torch, oracle, Q5_K, 64, 3584, seed=7, B=3)
    _gpu_check(gpu, torch, oracle, Q4_0, 2000, 3584, seed=8, x_kind="spiky")
    _gpu_check(gpu, torch, oracle, Q4_1, 64, 3584, seed=9, B=3)
    _gpu_check(gpu, torch, oracle, Q3_K, 2000, 3584, seed=10, x_kind="sparse")


@pytest.mark.gpu
@pytest.mark.parametrize("qt,rows,cols", [
    (Q6_K, 152064, 3584),    # Qwen2.5-7B lm_head (the bench's GEMV)
    (Q4_K, 152064, 3584),
    (Q8_0, 128256, 4096),    # Llama-3-8B lm_head shape
    (Q4_0, 152064, 3584),
    (Q3_K, 152064, 3584),
])
def test_gemv_full_lm_head(gpu, torch, oracle, qt, rows, cols):
    """Full output-projection shapes, every row against the oracle."""
    print("gemv full", qt, rows, cols, flush=True)
    _gpu_check(gpu, torch, oracle, qt, rows, cols, seed=rows % 1000 + qt)
