/*
 * sampler_oracle.c -- CPU restatement of gguf-rs-cli's token sampler.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the parity checker for the HIP
 * sampler in gguf-rs-cli_amd/.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load it; the product path never calls it.
 *
 * It restates /root/reference/src/sampler.rs operation for operation:
 *   - rand_f32 / set_seed      : src/sampler.rs:3-12   (global u64 LCG)
 *   - greedy                   : src/sampler.rs:15-19  (last maximal index)
 *   - apply_rep_penalty        : src/sampler.rs:23-30
 *   - sample                   : src/sampler.rs:35-79
 *   - decode-loop recent FIFO  : src/main.rs:98, 280-281, 302-303
 *   - generate_collect step    : src/main.rs:279-304 (stop / max checks)
 * Build with -O2 -ffp-contract=off and no fast-math, so that every f32
 * operation is one IEEE op in the same order as the Rust code.  f32::exp
 * lowers to the platform libm expf (glibc on linux-gnu), which is what this
 * file calls.
 *
 * Tie order.  Rust's sort_unstable_by leaves equal keys in an unspecified
 * order.  This oracle (and the GPU path) defines the order as: scaled logit
 * descending, then token index ascending.  That choice is "parity unpinned"
 * against the Rust binary: only a run of the Rust build could pin it.
 *
 * Pinning of each function (see tests/test_oracle.py):
 *   lcg          : closed-form KAT vectors (exact u64 arithmetic in Python)
 *   penalty      : single IEEE ops, cross-checked against numpy float32
 *   sort/top-k   : brute force + numpy lexsort on tiny and medium V
 *   softmax/top-p: float64 recomputation within 1e-5 relative; sequential
 *                  f32 sums cross-checked against numpy.cumsum(float32)
 *   draw         : grid over u against a hand-built CDF on V <= 8
 *   invariants   : top_k=1 => argmax, rep=1 => identity, top_p>=1 => no cut,
 *                  T<=0 => greedy and no RNG advance.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <pthread.h>
#include <time.h>

#include "sampler_oracle.h"

/* ---- RNG: src/sampler.rs:3-12 ---------------------------------------- */

static uint64_t g_seed = 12345u; /* src/sampler.rs:3 */

void oracle_set_seed(uint64_t s) { g_seed = s; } /* src/sampler.rs:5 */
uint64_t oracle_get_seed(void) { return g_seed; }

/* fetch_update returns the PRE-update state; the draw is made from it. */
float oracle_lcg_draw(uint64_t *state)
{
    uint64_t s = *state;
    *state = s * 6364136223846793005ull + 1442695040888963407ull;
    /* (s >> 33) as f32 / u32::MAX as f32 ; u32::MAX as f32 == 2^32 */
    return (float)(s >> 33) / (float)4294967295u;
}


/* ---- greedy: src/sampler.rs:15-19 ------------------------------------- */
/* Iterator::max_by keeps the LAST of equal maxima. */
static size_t greedy(const float *l, size_t n)
{
    size_t best = 0;
    for (size_t i = 1; i < n; i++)
        if (!(l[i] < l[best])) best = i; /* l[i] >= l[best] (no NaN here) */
    return best;
}

/* ---- penalty: src/sampler.rs:23-30 ------------------------------------- */
void oracle_apply_rep_penalty(float *l, size_t n, const uint32_t *recent,
                              size_t w, float penalty)
{
    if (penalty == 1.0f) return;
    for (size_t j = 0; j < w; j++) {
        uint32_t t = recent[j];
        if ((size_t)t < n) {
            if (l[t] > 0.0f) l[t] /= penalty;
            else l[t] *= penalty;
        }
    }
}

/* ---- sort order: value descending, index ascending ------------------- */
typedef struct { uint32_t idx; float v; } pair_t;

static int cmp_pair(const void *a, const void *b)
{
    const pair_t *x = (const pair_t *)a, *y = (const pair_t *)b;
    if (x->v > y->v) return -1;
    if (x->v < y->v) return 1;
    return (x->idx > y->idx) - (x->idx < y->idx);
}

static int pair_before(const pair_t *x, const pair_t *y) { return cmp_pair(x, y) < 0; }

/* Top-k prefix of the total order by a bounded min-heap (root = worst kept).
 * Same set and order as sort+truncate because the order is total. */
static void heap_sift_down(pair_t *h, size_t n, size_t i)
{
    for (;;) {
        size_t l = 2 * i + 1, r = l + 1, w = i;
        if (l < n && pair_before(&h[w], &h[l])) w = l;
        if (r < n && pair_before(&h[w], &h[r])) w = r;
        if (w == i) return;
        pair_t t = h[i]; h[i] = h[w]; h[w] = t; i = w;
    }
}

static size_t topk_prefix(const float *v, size_t n, size_t k, pair_t *out)
{
    /* out has room for k; builds a heap where the root is the worst kept */
    size_t m = 0;
    for (size_t i = 0; i < n; i++) {
        pair_t p = { (uint32_t)i, v[i] };
        if (m < k) {
            out[m++] = p;
            if (m == k)
                for (size_t j = k / 2 + 1; j-- > 0;) heap_sift_down(out, k, j);
        } else if (pair_before(&p, &out[0])) {
            out[0] = p;
            heap_sift_down(out, k, 0);
        }
    }
    qsort(out, m, sizeof(pair_t), cmp_pair);
    return m;
}

/* ---- sample: src/sampler.rs:35-79 --------------------------------------
 * logits is mutated exactly as the reference mutates it (penalized, and
 * divided by T when T > 0).  `r` is the uniform draw; if draw_state is not
 * NULL the draw comes from that LCG state instead (advanced only if T > 0).
 * fast_topk != 0 selects the top-k prefix with a heap instead of a full sort
 * (identical result, used to keep big test cases fast).
 * Returns the token, or a negative status where Rust would panic. */
int64_t oracle_sample_ex(float *logits, size_t V, float temperature,
                         size_t top_k, float top_p, float rep_penalty,
                         const uint32_t *recent, size_t W, float r,
                         uint64_t *draw_state, int fast_topk,
                         oracle_detail *det)
{
    if (det) { det->n_kept = 0; det->cut = 0; det->r = 0.0f; }
    oracle_apply_rep_penalty(logits, V, recent, W, rep_penalty);

    if (temperature <= 0.0f) {
        if (V == 0) return 0; /* unwrap_or(0) */
        if (V > 1)
            for (size_t i = 0; i < V; i++)
                if (isnan(logits[i])) return ORACLE_ERR_NAN; /* partial_cmp().unwrap() */
        return (int64_t)greedy(logits, V);
    }

    for (size_t i = 0; i < V; i++) logits[i] /= temperature;

    if (V == 0) return ORACLE_ERR_EMPTY; /* pairs[0] panics */
    if (V > 1)
        for (size_t i = 0; i < V; i++)
            if (isnan(logits[i])) return ORACLE_ERR_NAN;

    size_t keep = (top_k > 0 && top_k < V) ? top_k : V;
    pair_t *pairs = (pair_t *)malloc(sizeof(pair_t) * (fast_topk ? keep : V));
    if (!pairs) return ORACLE_ERR_NOMEM;
    if (fast_topk && keep < V) {
        topk_prefix(logits, V, keep, pairs);
    } else {
        for (size_t i = 0; i < V; i++) { pairs[i].idx = (uint32_t)i; pairs[i].v = logits[i]; }
        qsort(pairs, V, sizeof(pair_t), cmp_pair);
    }
    size_t n = keep; /* truncate(top_k) */

    /* softmax over survivors: sequential f32 sum in sorted order */
    float mx = pairs[0].v;
    float sum = 0.0f;
    for (size_t i = 0; i < n; i++) { pairs[i].v = expf(pairs[i].v - mx); sum += pairs[i].v; }
    for (size_t i = 0; i < n; i++) pairs[i].v /= sum;
    if (det) {
        det->sum = sum;
        for (size_t i = 0; i < n && i < det->cap; i++) { det->idx[i] = pairs[i].idx; det->p[i] = pairs[i].v; }
    }

    /* nucleus */
    if (top_p < 1.0f) {
        float cum = 0.0f;
        size_t cut = n;
        for (size_t i = 0; i < n; i++) {
            cum += pairs[i].v;
            if (cum >= top_p) { cut = i + 1; break; }
        }
        n = cut;
        float s = -0.0f; /* Iterator::sum for f32 folds from -0.0 (or 0.0: same for p > 0) */
        for (size_t i = 0; i < n; i++) s += pairs[i].v;
        for (size_t i = 0; i < n; i++) pairs[i].v /= s;
        if (det) det->s2 = s;
    } else if (det) {
        det->s2 = 1.0f;
    }
    if (det) det->cut = n;

    if (draw_state) r = oracle_lcg_draw(draw_state);
    if (det) det->r = r;
    float cum = 0.0f;
    int64_t tok = -1;
    for (size_t i = 0; i < n; i++) {
        cum += pairs[i].v;
        if (r < cum) { tok = pairs[i].idx; break; }
    }
    if (tok < 0) tok = n ? pairs[n - 1].idx : 0;
    if (det) { det->n_kept = keep; det->q_last = n ? pairs[n - 1].v : 0.0f; }
    free(pairs);
    return tok;
}

/* The reference entry point with the process-global LCG. */
int64_t oracle_sample(float *logits, size_t V, float temperature, size_t top_k,
                      float top_p, float rep_penalty, const uint32_t *recent,
                      size_t W)
{
    return oracle_sample_ex(logits, V, temperature, top_k, top_p, rep_penalty,
                            recent, W, 0.0f, temperature > 0.0f ? &g_seed : NULL,
                            0, NULL);
}

/* ---- batch over B rows (explicit per-row u), optional threads ---------- */
typedef struct {
    const float *logits; size_t B, V, ld;
    const oracle_params *params; const uint32_t *recent; size_t ld_recent;
    const uint32_t *recent_len; size_t W; const float *u; int64_t *tokens;
    int fast_topk; size_t row0, row1; int status;
} batch_job;

static void *batch_worker(void *arg)
{
    batch_job *j = (batch_job *)arg;
    float *row = (float *)malloc(sizeof(float) * (j->V ? j->V : 1));
    if (!row) { j->status = ORACLE_ERR_NOMEM; return NULL; }
    for (size_t b = j->row0; b < j->row1; b++) {
        memcpy(row, j->logits + b * j->ld, sizeof(float) * j->V);
        const oracle_params *p = &j->params[b];
        size_t w = j->recent_len ? j->recent_len[b] : j->W;
        const uint32_t *rc = j->recent ? j->recent + b * j->ld_recent : NULL;
        j->tokens[b] = oracle_sample_ex(row, j->V, p->temperature, p->top_k, p->top_p,
                                        p->rep_penalty, rc, rc ? w : 0, j->u[b], NULL,
                                        j->fast_topk, NULL);
    }
    free(row);
    return NULL;
}

int oracle_sample_batch(const float *logits, size_t B, size_t V, size_t ld,
                        const oracle_params *params, const uint32_t *recent,
                        size_t ld_recent, const uint32_t *recent_len, size_t W,
                        const float *u, int64_t *tokens, int nthreads,
                        int fast_topk)
{
    if (nthreads < 1) nthreads = 1;
    if ((size_t)nthreads > B) nthreads = (int)(B ? B : 1);
    batch_job jobs[256];
    pthread_t th[256];
    if (nthreads > 256) nthreads = 256;
    for (int t = 0; t < nthreads; t++) {
        batch_job *j = &jobs[t];
        j->logits = logits; j->B = B; j->V = V; j->ld = ld; j->params = params;
        j->recent = recent; j->ld_recent = ld_recent; j->recent_len = recent_len;
        j->W = W; j->u = u; j->tokens = tokens; j->fast_topk = fast_topk;
        j->row0 = B * (size_t)t / (size_t)nthreads;
        j->row1 = B * (size_t)(t + 1) / (size_t)nthreads;
        j->status = 0;
    }
    if (nthreads == 1) batch_worker(&jobs[0]);
    else {
        for (int t = 0; t < nthreads; t++) pthread_create(&th[t], NULL, batch_worker, &jobs[t]);
        for (int t = 0; t < nthreads; t++) pthread_join(th[t], NULL);
    }
    for (int t = 0; t < nthreads; t++) if (jobs[t].status) return jobs[t].status;
    return 0;
}

/* ---- decode loop semantics: src/main.rs:98, 280-281, 302-303 ----------
 * One row, `steps` sequential draws from the global-LCG stream; logits for
 * step t are logits + t*V (unmodified input; a private copy is mutated).
 * `recent` is a FIFO of at most `window` ids: it starts as the last
 * `window` entries of init_recent (empty in the reference's first turn,
 * src/main.rs:98) and every generated id is pushed (src/main.rs:302-303). */
int oracle_decode_trace(const float *logits, size_t steps, size_t V,
                        float temperature, size_t top_k, float top_p,
                        float rep_penalty, size_t window, const uint32_t *init_recent,
                        size_t init_len, uint64_t seed, int64_t *tokens, int fast_topk)
{
    float *row = (float *)malloc(sizeof(float) * (V ? V : 1));
    uint32_t *recent = (uint32_t *)malloc(sizeof(uint32_t) * (window + 1));
    if (!row || !recent) { free(row); free(recent); return ORACLE_ERR_NOMEM; }
    size_t w = init_len < window ? init_len : window;
    if (w) memcpy(recent, init_recent + (init_len - w), sizeof(uint32_t) * w);
    uint64_t st = seed;
    for (size_t t = 0; t < steps; t++) {
        memcpy(row, logits + t * V, sizeof(float) * V);
        int64_t tok = oracle_sample_ex(row, V, temperature, top_k, top_p, rep_penalty,
                                       recent, w, 0.0f,
                                       temperature > 0.0f ? &st : NULL, fast_topk, NULL);
        tokens[t] = tok;
        if (tok < 0) { free(row); free(recent); return (int)tok; }
        recent[w++] = (uint32_t)tok;                 /* recent.push(next) */
        if (w > window) { memmove(recent, recent + 1, sizeof(uint32_t) * window); w = window; } /* remove(0) */
    }
    free(row); free(recent);
    return 0;
}

/* generate_collect (src/main.rs:258-313) for one row over given per-step
 * logits: sample (:280), stop check (:281), max check (:282), recent FIFO
 * push of the last `window` ids (:302-303), generated push (:304).  The
 * smart-context branch (:284-296) is not part of it.  logits[t*V..] are the
 * logits the row sees at step t; `steps` bounds the loop.  Outputs: sampled[t]
 * for every step taken, *n_steps, *n_gen, *done (0 = ran out of steps, 1 =
 * stop token, 2 = max), the LCG state after the loop in *state (in: the seed)
 * and the final FIFO in recent_out[0..*recent_len), oldest first. */
int oracle_generate(const float *logits, size_t steps, size_t V, float temperature,
                    size_t top_k, float top_p, float rep_penalty, size_t window,
                    const uint32_t *init_recent, size_t init_len, const uint32_t *stops,
                    size_t n_stop, size_t max_new, uint64_t *state, int64_t *sampled,
                    size_t *n_steps, size_t *n_gen, int *done, uint32_t *recent_out,
                    size_t *recent_len)
{
    float *row = (float *)malloc(sizeof(float) * (V ? V : 1));
    uint32_t *recent = (uint32_t *)malloc(sizeof(uint32_t) * (window + 1));
    if (!row || !recent) { free(row); free(recent); return ORACLE_ERR_NOMEM; }
    size_t w = init_len < window ? init_len : window;
    if (w) memcpy(recent, init_recent + (init_len - w), sizeof(uint32_t) * w);
    size_t gen = 0, t = 0;
    int why = 0;
    for (; t < steps; t++) {
        memcpy(row, logits + t * V, sizeof(float) * V);
        const int64_t tok = oracle_sample_ex(row, V, temperature, top_k, top_p, rep_penalty,
                                             recent, w, 0.0f, temperature > 0.0f ? state : NULL, 0, NULL);
        sampled[t] = tok;
        if (tok < 0) { free(row); free(recent); return (int)tok; }
        int is_stop = 0;
        for (size_t i = 0; i < n_stop; i++) is_stop |= stops[i] == (uint32_t)tok;
        if (is_stop) { why = 1; t++; break; }
        if (gen >= max_new) { why = 2; t++; break; }
        if (window) {
            recent[w++] = (uint32_t)tok;
            if (w > window) { memmove(recent, recent + 1, sizeof(uint32_t) * window); w = window; }
        }
        gen++;
    }
    *n_steps = t;
    *n_gen = gen;
    *done = why;
    if (recent_out && w) memcpy(recent_out, recent, sizeof(uint32_t) * w);
    *recent_len = w;
    free(row); free(recent);
    return 0;
}

/* ---- synthetic on-device generator, restated for the host -------------
 * Must equal the device function gs_synth_logit() bit for bit: integer
 * hashing, one exact int->f32 conversion, then two IEEE f32 multiplies. */
static uint64_t splitmix64(uint64_t x)
{
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

float oracle_synth_logit(uint64_t seed, uint64_t counter, float sigma)
{
    uint64_t h = splitmix64(seed ^ splitmix64(counter));
    int32_t s = (int32_t)(h & 0xFFFF) + (int32_t)((h >> 16) & 0xFFFF) +
                (int32_t)((h >> 32) & 0xFFFF) + (int32_t)((h >> 48) & 0xFFFF);
    /* Irwin-Hall(4): mean 4*32767.5, sd sqrt(4/12)*65536 = 37837.227 */
    float z = (float)(2 * s - 262140) * 0x1.bb67bp-17f /* RN(1/75674.453) */;
    return z * sigma;
}

void oracle_synth_logits(float *out, size_t n, uint64_t seed, uint64_t counter0, float sigma)
{
    for (size_t i = 0; i < n; i++) out[i] = oracle_synth_logit(seed, counter0 + i, sigma);
}

/* ---- device-resident decode loop (batch, ring window) -----------------
 * B rows, `steps` steps.  Step t logits of row b are synthesized from
 * counter (t*B + b)*V + col.  Each row keeps a ring window of W ids
 * (initial contents given); the sampled token overwrites slot t % W.
 * Draw for (t, b) is u[t*B + b]. */
/* Rows [row0, row1) of one step's synthetic logits, for the threads of
 * oracle_device_loop. */
struct synth_job { float *out; size_t n; uint64_t seed, c0; float sigma; };
static void *synth_worker(void *arg)
{
    struct synth_job *j = (struct synth_job *)arg;
    oracle_synth_logits(j->out, j->n, j->seed, j->c0, j->sigma);
    return NULL;
}

static void synth_rows(float *lg, size_t B, size_t V, uint64_t seed, uint64_t c0, float sigma, int nthreads)
{
    if (nthreads < 1) nthreads = 1;
    if (nthreads > 256) nthreads = 256;
    if ((size_t)nthreads > B) nthreads = (int)(B ? B : 1);
    pthread_t th[256];
    struct synth_job jobs[256];
    for (int t = 0; t < nthreads; t++) {
        const size_t r0 = B * (size_t)t / (size_t)nthreads, r1 = B * (size_t)(t + 1) / (size_t)nthreads;
        jobs[t].out = lg + r0 * V;
        jobs[t].n = (r1 - r0) * V;
        jobs[t].seed = seed;
        jobs[t].c0 = c0 + r0 * V;
        jobs[t].sigma = sigma;
    }
    if (nthreads == 1) { synth_worker(&jobs[0]); return; }
    for (int t = 0; t < nthreads; t++) pthread_create(&th[t], NULL, synth_worker, &jobs[t]);
    for (int t = 0; t < nthreads; t++) pthread_join(th[t], NULL);
}

int oracle_device_loop(size_t B, size_t V, size_t steps, uint64_t seed, float sigma,
                       const oracle_params *p, uint32_t *window, size_t W,
                       const float *u, int64_t *tokens, int nthreads, int fast_topk)
{
    float *lg = (float *)malloc(sizeof(float) * B * V);
    oracle_params *pp = (oracle_params *)malloc(sizeof(oracle_params) * B);
    if (!lg || !pp) { free(lg); free(pp); return ORACLE_ERR_NOMEM; }
    for (size_t b = 0; b < B; b++) pp[b] = *p;
    int st = 0;
    for (size_t t = 0; t < steps && !st; t++) {
        synth_rows(lg, B, V, seed, (uint64_t)t * B * V, sigma, nthreads);
        st = oracle_sample_batch(lg, B, V, V, pp, window, W, NULL, W, u + t * B,
                                 tokens + t * B, nthreads, fast_topk);
        for (size_t b = 0; b < B && !st; b++) {
            if (tokens[t * B + b] < 0) { st = (int)tokens[t * B + b]; break; }
            window[b * W + (t % W)] = (uint32_t)tokens[t * B + b];
        }
    }
    free(lg); free(pp);
    return st;
}

/* ---- wall clock for the CPU baseline ---------------------------------- */
double oracle_now(void)
{
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}
