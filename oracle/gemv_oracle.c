/* gemv_oracle.c -- CPU restatement of gguf-rs-cli's quantized matrix-vector
 * product for the Q4_0, Q4_1, Q8_0, Q3_K, Q4_K, Q5_K and Q6_K block types
 * (the logits projection,
 * src/model/llama.rs:405-407 on the CPU path).
 * TEST INFRASTRUCTURE ONLY (parity checker); never linked into the product.
 *
 * Follows src/tensor/dequant.rs:
 *   dq40      :26-41   Q4_0 dequantization, w = ((q - 8) as f32) * d
 *   dq41      :42-54   Q4_1 dequantization, w = (q as f32) * d + m
 *   dq80      :86-94   Q8_0 dequantization, w = (q as f32) * d
 *   Q3_K      the GGUF format (see oracle_dequant_q3_k: the reference's
 *             dq3k :120-140 decodes another layout), w = (d * sc) * q
 *   dq6k      :197-219 Q6_K dequantization, w = (d * (scale as f32)) * q
 *   get_scale_min_k4 :141-148, dq4k :149-170, dq5k :171-196
 *                      Q4_K / Q5_K, w = (d * sc) * q - dmin * m
 *   row_dot   :277-313 Q8_0: per block a sequential f32 sum of (q * d) * x,
 *                      then a sequential sum of the block sums; Q4_0: per
 *                      block a sequential sum over j of (lo_j + hi_j), lo_j =
 *                      ((q_j - 8) * d) * x_j, hi_j the same for weight j + 16;
 *                      other types (K-quants): dequantize the row, then a
 *                      sequential f32 sum of w * x
 *   matvec    :315-318 out[i] = row_dot(i, x), rows in parallel
 * f16 -> f32 is the `half` crate's (2.7.1, Cargo.lock:219) to_f32, an exact
 * conversion.  Rust's f32 Iterator::sum is a left fold, restated as a loop.
 * Built with -ffp-contract=off: every f32 op is one IEEE op, as in Rust. */
#include <math.h>
#include <pthread.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define QT_Q4_0 2u
#define QT_Q4_1 3u
#define QT_Q8_0 8u
#define QT_Q3_K 11u
#define QT_Q4_K 12u
#define QT_Q5_K 13u
#define QT_Q6_K 14u

/* IEEE binary16 -> binary32, exact (every f16 is an f32). */
float oracle_f16_to_f32(uint16_t h)
{
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t ex = (h >> 10) & 0x1fu, man = h & 0x3ffu;
    uint32_t bits;
    if (ex == 0x1fu) {
        bits = sign | 0x7f800000u | (man << 13);           /* inf / nan (payload kept) */
    } else if (ex != 0) {
        bits = sign | ((ex + 112u) << 23) | (man << 13);   /* normal: rebias 15 -> 127 */
    } else if (man == 0) {
        bits = sign;                                       /* +-0 */
    } else {
        /* subnormal: man * 2^-24, renormalised */
        int e = -1;
        uint32_t m = man;
        do { m <<= 1; e++; } while (!(m & 0x400u));
        bits = sign | ((uint32_t)(112 - e) << 23) | ((m & 0x3ffu) << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* dq80 (dequant.rs:86-94): n weights from n/32 blocks of 34 bytes. */
void oracle_dequant_q8_0(const uint8_t *data, size_t n, float *o)
{
    for (size_t b = 0; b < n / 32; b++) {
        const uint8_t *d = data + b * 34;
        const float sc = oracle_f16_to_f32(rd16(d));
        for (int i = 0; i < 32; i++) o[b * 32 + i] = (float)(int8_t)d[2 + i] * sc;
    }
}

/* dq40 (dequant.rs:26-41): n weights from n/32 blocks of 18 bytes; byte
 * 2 + j holds weight j (low nibble) and weight j + 16 (high). */
void oracle_dequant_q4_0(const uint8_t *data, size_t n, float *o)
{
    for (size_t b = 0; b < n / 32; b++) {
        const uint8_t *d = data + b * 18;
        const float sc = oracle_f16_to_f32(rd16(d));
        for (int j = 0; j < 16; j++) {
            o[b * 32 + j] = (float)((int)(d[2 + j] & 0xF) - 8) * sc;
            o[b * 32 + j + 16] = (float)((int)(d[2 + j] >> 4) - 8) * sc;
        }
    }
}

/* dq41 (dequant.rs:42-54): n/32 blocks of 20 bytes (f16 d, f16 m, 16 bytes
 * of nibbles as Q4_0), w = q * d + m. */
void oracle_dequant_q4_1(const uint8_t *data, size_t n, float *o)
{
    for (size_t b = 0; b < n / 32; b++) {
        const uint8_t *d = data + b * 20;
        const float sc = oracle_f16_to_f32(rd16(d)), mn = oracle_f16_to_f32(rd16(d + 2));
        for (int j = 0; j < 16; j++) {
            o[b * 32 + j] = (float)(d[4 + j] & 0xF) * sc + mn;
            o[b * 32 + j + 16] = (float)(d[4 + j] >> 4) * sc + mn;
        }
    }
}

/* The 6-bit scale of sub-block is (0..15) of a Q3_K block, as GGUF packs
 * them in 12 bytes: bytes 0-7 hold the low nibbles (scales 0-7 low, 8-15
 * high nibbles), bytes 8-11 the top two bits (bits 2k..2k+1 of byte 8 + j
 * for scale 4k + j).  Returns the signed scale, value - 32. */
static int q3k_scale(const uint8_t *s, int is)
{
    const int k = is >> 2, j = is & 3;
    const int low = k == 0 ? (s[j] & 0xF) : k == 1 ? (s[4 + j] & 0xF) : k == 2 ? (s[j] >> 4) : (s[4 + j] >> 4);
    const int high = (s[8 + j] >> (2 * k)) & 3;
    return (low | (high << 4)) - 32;
}

/* Q3_K: n/256 blocks of 110 bytes (hmask[32], qs[64], scales[12], f16 d), in
 * the GGUF format: weight i = 128 n + 32 j + l (n < 2, j < 4, l < 32) has the
 * low two bits (qs[32 n + l] >> 2 j) & 3, the third bit (hmask[l] >> (4 n +
 * j)) & 1, value q = bits - 4, and sub-block scale i / 16.  w = (d * sc) * q
 * as the reference's dq3k evaluates it (dequant.rs:136).
 * Deviation: the reference's dq3k reads the low bits of weight i from
 * qs[i / 4] >> 2 (i % 4) (:134), and scale j < 4 as the low six bits of
 * byte j, scale 8 + j as those of byte 8 + j, the others from nibble pairs
 * (:126-131); its GPU shader (q3k_gemv.glsl) decodes the scales another way
 * again.  The GGUF layout is the one files carry, so Q3_K is pinned to the
 * format by bit probes, not to either reference path. */
void oracle_dequant_q3_k(const uint8_t *data, size_t n, float *o)
{
    for (size_t b = 0; b < n / 256; b++) {
        const uint8_t *d = data + b * 110;
        const uint8_t *hm = d, *qs = d + 32, *sc = d + 96;
        const float df = oracle_f16_to_f32(rd16(d + 108));
        for (int i = 0; i < 256; i++) {
            const int nn = i >> 7, j = (i >> 5) & 3, l = i & 31;
            const int lo = (qs[32 * nn + l] >> (2 * j)) & 3;
            const int hi = (hm[l] >> (4 * nn + j)) & 1;
            const int q = (lo | (hi << 2)) - 4;
            o[b * 256 + i] = df * (float)q3k_scale(sc, i >> 4) * (float)q;
        }
    }
}

/* dq6k (dequant.rs:197-219): n weights from n/256 blocks of 210 bytes. */
void oracle_dequant_q6_k(const uint8_t *data, size_t n, float *o)
{
    for (size_t b = 0; b < n / 256; b++) {
        const uint8_t *d = data + b * 210;
        const uint8_t *ql = d, *qh = d + 128;
        const int8_t *sc = (const int8_t *)(d + 192);
        const float df = oracle_f16_to_f32(rd16(d + 208));
        size_t y = b * 256, qlo = 0, qhi = 0, si = 0;
        for (int half = 0; half < 2; half++) {
            for (int l = 0; l < 32; l++) {
                const int q1 = ((ql[qlo + l] & 0xF) | (((qh[qhi + l] >> 0) & 3) * 16)) - 32;
                const int q2 = ((ql[qlo + l + 32] & 0xF) | (((qh[qhi + l] >> 2) & 3) * 16)) - 32;
                const int q3 = ((ql[qlo + l] >> 4) | (((qh[qhi + l] >> 4) & 3) * 16)) - 32;
                const int q4 = ((ql[qlo + l + 32] >> 4) | (((qh[qhi + l] >> 6) & 3) * 16)) - 32;
                const int is = l / 16;
                o[y + l] = df * (float)sc[si + is] * (float)q1;
                o[y + l + 32] = df * (float)sc[si + is + 2] * (float)q2;
                o[y + l + 64] = df * (float)sc[si + is + 4] * (float)q3;
                o[y + l + 96] = df * (float)sc[si + is + 6] * (float)q4;
            }
            y += 128; qlo += 64; qhi += 32; si += 8;
        }
    }
}

/* get_scale_min_k4 (dequant.rs:141-148): the 6-bit scale and min of
 * sub-block j from the 12 packed bytes q. */
static void scale_min_k4(int j, const uint8_t *q, float *d, float *m)
{
    uint8_t a, b;
    if (j < 4) {
        a = q[j] & 63;
        b = q[j + 4] & 63;
    } else {
        a = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        b = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
    *d = (float)a;
    *m = (float)b;
}

/* dq4k (dequant.rs:149-170): n weights from n/256 blocks of 144 bytes,
 * w = (df * sc) * q - dmin * m. */
void oracle_dequant_q4_k(const uint8_t *data, size_t n, float *o)
{
    for (size_t b = 0; b < n / 256; b++) {
        const uint8_t *d = data + b * 144;
        const float df = oracle_f16_to_f32(rd16(d)), dmin = oracle_f16_to_f32(rd16(d + 2));
        const uint8_t *scales = d + 4, *qs = d + 16;
        size_t is = 0, qoff = 0, y = b * 256;
        for (int it = 0; it < 4; it++) {
            float sc1, m1, sc2, m2;
            scale_min_k4((int)is, scales, &sc1, &m1);
            scale_min_k4((int)is + 1, scales, &sc2, &m2);
            const float d1 = df * sc1, mb1 = dmin * m1, d2 = df * sc2, mb2 = dmin * m2;
            for (int l = 0; l < 32; l++) {
                o[y + l] = d1 * (float)(qs[qoff + l] & 0xF) - mb1;
                o[y + l + 32] = d2 * (float)(qs[qoff + l] >> 4) - mb2;
            }
            is += 2; qoff += 32; y += 64;
        }
    }
}

/* dq5k (dequant.rs:171-196): n weights from n/256 blocks of 176 bytes; the
 * fifth bit of the two sub-blocks of step j is bit 2j / 2j+1 of qh[l].
 * One deviation, from the GGUF format: the reference advances its qh offset
 * by 32 after step 1 (:192), so step 2 indexes qh[32 + l] in the 32-byte qh
 * slice (:177) and the Rust code panics on every Q5_K block; here qh[l]
 * serves all four steps, as the format defines (the masks already select
 * the step's bits).  Parity for Q5_K is therefore pinned to the format by
 * bit probes, not to the reference. */
void oracle_dequant_q5_k(const uint8_t *data, size_t n, float *o)
{
    for (size_t b = 0; b < n / 256; b++) {
        const uint8_t *d = data + b * 176;
        const float df = oracle_f16_to_f32(rd16(d)), dmin = oracle_f16_to_f32(rd16(d + 2));
        const uint8_t *scales = d + 4, *qh = d + 16, *qs = d + 48;
        size_t is = 0, qoff = 0, y = b * 256;
        const size_t qhoff = 0;
        for (int j = 0; j < 4; j++) {
            const uint8_t hm1 = (uint8_t)(1u << (j * 2)), hm2 = (uint8_t)(1u << (j * 2 + 1));
            float sc1, m1, sc2, m2;
            scale_min_k4((int)is, scales, &sc1, &m1);
            scale_min_k4((int)is + 1, scales, &sc2, &m2);
            const float d1 = df * sc1, mb1 = dmin * m1, d2 = df * sc2, mb2 = dmin * m2;
            for (int l = 0; l < 32; l++) {
                const float v1 = (float)(qs[qoff + l] & 0xF) + ((qh[qhoff + l] & hm1) ? 16.0f : 0.0f);
                const float v2 = (float)(qs[qoff + l] >> 4) + ((qh[qhoff + l] & hm2) ? 16.0f : 0.0f);
                o[y + l] = d1 * v1 - mb1;
                o[y + l + 32] = d2 * v2 - mb2;
            }
            is += 2; qoff += 32; y += 64;
        }
    }
}

static size_t row_bytes(uint32_t qt, size_t cols)
{
    switch (qt) {
    case QT_Q4_0: return cols / 32 * 18;
    case QT_Q4_1: return cols / 32 * 20;
    case QT_Q3_K: return cols / 256 * 110;
    case QT_Q8_0: return cols / 32 * 34;
    case QT_Q4_K: return cols / 256 * 144;
    case QT_Q5_K: return cols / 256 * 176;
    default: return cols / 256 * 210;
    }
}

static void dequant(uint32_t qt, const uint8_t *d, size_t n, float *w)
{
    switch (qt) {
    case QT_Q4_0: oracle_dequant_q4_0(d, n, w); break;
    case QT_Q4_1: oracle_dequant_q4_1(d, n, w); break;
    case QT_Q3_K: oracle_dequant_q3_k(d, n, w); break;
    case QT_Q8_0: oracle_dequant_q8_0(d, n, w); break;
    case QT_Q4_K: oracle_dequant_q4_k(d, n, w); break;
    case QT_Q5_K: oracle_dequant_q5_k(d, n, w); break;
    default: oracle_dequant_q6_k(d, n, w); break;
    }
}

/* row_dot (dequant.rs:277-313) for one row's blocks.  `w` is scratch for
 * `cols` floats (the Q6_K dequantized row). */
static float row_dot(uint32_t qt, const uint8_t *d, size_t cols, const float *x, float *w)
{
    if (qt == QT_Q8_0) {
        float acc = 0.0f;
        for (size_t blk = 0; blk < cols / 32; blk++) {
            const uint8_t *db = d + blk * 34;
            const float sc = oracle_f16_to_f32(rd16(db));
            float s = 0.0f;
            for (int i = 0; i < 32; i++) s += (float)(int8_t)db[2 + i] * sc * x[blk * 32 + i];
            acc += s;
        }
        return acc;
    }
    if (qt == QT_Q4_0) {
        float acc = 0.0f;
        for (size_t blk = 0; blk < cols / 32; blk++) {
            const uint8_t *db = d + blk * 18;
            const float sc = oracle_f16_to_f32(rd16(db));
            float s = 0.0f;
            for (int j = 0; j < 16; j++) {
                const float lo = (float)((int)(db[2 + j] & 0xF) - 8) * sc * x[blk * 32 + j];
                const float hi = (float)((int)(db[2 + j] >> 4) - 8) * sc * x[blk * 32 + j + 16];
                s += lo + hi;
            }
            acc += s;
        }
        return acc;
    }
    dequant(qt, d, cols, w);      /* the others: the row dequantized, then one sequential sum */
    float acc = 0.0f;
    for (size_t i = 0; i < cols; i++) acc += w[i] * x[i];
    return acc;
}

float oracle_row_dot(uint32_t qtype, const uint8_t *row_blocks, size_t cols, const float *x)
{
    float *w = (float *)malloc(sizeof(float) * (cols ? cols : 1));
    if (!w) return NAN;
    const float r = row_dot(qtype, row_blocks, cols, x, w);
    free(w);
    return r;
}

/* The exact value of the same product: the reference's f32 weights times x,
 * summed in double (each product w*x of two f32 is exact in double, and a
 * double sum of a few thousand of them carries a relative error below 2^-40),
 * and the sum of |w * x| for tolerances. */
static double row_exact(uint32_t qt, const uint8_t *d, size_t cols, const float *x, float *w, double *abs_sum)
{
    dequant(qt, d, cols, w);
    double s = 0.0, a = 0.0;
    for (size_t i = 0; i < cols; i++) {
        const double p = (double)w[i] * (double)x[i];
        s += p;
        a += fabs(p);
    }
    *abs_sum = a;
    return s;
}

typedef struct {
    uint32_t qt; const uint8_t *blocks; size_t rows, cols; const float *x;
    float *out; double *exact; double *abs_sum; size_t r0, r1;
} job_t;

static void *run_rows(void *arg)
{
    job_t *j = (job_t *)arg;
    float *w = (float *)malloc(sizeof(float) * (j->cols ? j->cols : 1));
    if (!w) return NULL;
    const size_t rb = row_bytes(j->qt, j->cols);
    for (size_t r = j->r0; r < j->r1; r++) {
        const uint8_t *d = j->blocks + r * rb;
        if (j->out) j->out[r] = row_dot(j->qt, d, j->cols, j->x, w);
        if (j->exact) j->exact[r] = row_exact(j->qt, d, j->cols, j->x, w, &j->abs_sum[r]);
    }
    free(w);
    return NULL;
}

/* matvec (dequant.rs:315-318) over `nthreads` threads (the reference uses
 * rayon's pool; every row is computed the same way on any thread).  Either
 * output may be NULL: `out` gets the reference's f32 results, `exact` and
 * `abs_sum` the double values above.  Returns 0, or -1 for a bad type. */
int oracle_matvec(uint32_t qtype, const uint8_t *blocks, size_t rows, size_t cols, const float *x,
                  float *out, double *exact, double *abs_sum, int nthreads)
{
    if (qtype != QT_Q8_0 && qtype != QT_Q6_K && qtype != QT_Q4_K && qtype != QT_Q5_K && qtype != QT_Q4_0 &&
        qtype != QT_Q4_1 && qtype != QT_Q3_K)
        return -1;
    if (nthreads < 1) nthreads = 1;
    if ((size_t)nthreads > rows) nthreads = rows ? (int)rows : 1;
    pthread_t th[64];
    job_t jobs[64];
    if (nthreads > 64) nthreads = 64;
    for (int i = 0; i < nthreads; i++) {
        jobs[i] = (job_t){qtype, blocks, rows, cols, x, out, exact, abs_sum,
                          rows * (size_t)i / (size_t)nthreads, rows * (size_t)(i + 1) / (size_t)nthreads};
        if (nthreads == 1) run_rows(&jobs[i]);
        else pthread_create(&th[i], NULL, run_rows, &jobs[i]);
    }
    if (nthreads > 1)
        for (int i = 0; i < nthreads; i++) pthread_join(th[i], NULL);
    return 0;
}
