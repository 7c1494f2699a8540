/*
 * gs_sampler.h -- C ABI of the MI355X (gfx950) token sampler.
 *
 * Drop-in for gguf-rs-cli's sampler (src/sampler.rs).  The reference API is a
 * crate-internal Rust free function plus a process-global LCG:
 *
 *   pub fn set_seed(s: u64)                                  src/sampler.rs:5
 *   pub fn sample(logits: &mut Vec<f32>, temperature: f32,
 *                 top_k: usize, top_p: f32, rep_penalty: f32,
 *                 recent: &[u32]) -> usize                   src/sampler.rs:35-36
 *
 * Its one caller is the decode loop, src/main.rs:280 (seed set at :54).
 * Every entry point returns an int status: GS_OK (0) or a negative GS_ERR_*.
 * The statuses stand in for the reference's panics: NaN logits
 * (src/sampler.rs:17,45 partial_cmp().unwrap()) and empty logits with T > 0
 * (src/sampler.rs:53 pairs[0]).
 *
 * Buffers are caller-owned.  Batched calls are asynchronous and ordered on
 * the given HIP stream (NULL = the default stream).  No torch types appear in
 * this interface.
 */
#ifndef GS_SAMPLER_H
#define GS_SAMPLER_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GS_OK               0
#define GS_ERR_INVALID    (-1)  /* bad argument (null pointer, size out of range) */
#define GS_ERR_EMPTY      (-2)  /* V == 0 with T > 0: reference panics at pairs[0] */
#define GS_ERR_NAN        (-3)  /* NaN logit with V > 1: reference panics in partial_cmp */
#define GS_ERR_HIP        (-5)  /* a HIP runtime call failed */
#define GS_ERR_NOMEM      (-6)  /* device allocation failed */
#define GS_ERR_UNSUPPORTED (-7) /* request outside the implemented limits */

/* Sampler parameters: the four scalars of src/sampler.rs:35-36 (16 bytes).
 * Defaults of the reference CLI (src/main.rs:24-31): T 0.7, k 40, p 0.9, rep 1.1. */
typedef struct gs_params {
    float temperature;  /* <= 0: greedy (src/sampler.rs:39) */
    uint32_t top_k;     /* 0 or >= V: no truncation (src/sampler.rs:48-50) */
    float top_p;        /* >= 1: no nucleus cut (src/sampler.rs:59) */
    float rep_penalty;  /* == 1: no penalty (src/sampler.rs:24) */
} gs_params;

typedef struct gs_sampler gs_sampler;

/* Library limits (also returned by gs_limits). */
#define GS_MAX_VOCAB   (1u << 22)  /* 4,194,304 logits per row */
#define GS_MAX_WINDOW  1024u       /* recent-window length per row */

/* ---- sampler object: "Sampler construction" of the drop-in -------------
 * Replaces set_seed (src/sampler.rs:5) plus the four scalars the caller
 * passes on every call (src/main.rs:280).  `seed` initialises the sampler's
 * own copy of the reference LCG (src/sampler.rs:3-12).  The sampler binds to
 * the HIP device current at creation.  Creation allocates the sampler's
 * streams, its pinned host words and 8 KB of device counters (the chunked
 * top-k path's), and synchronises once. */
int gs_sampler_create(const gs_params *params, uint64_t seed, gs_sampler **out);
int gs_sampler_destroy(gs_sampler *s);
int gs_sampler_set_params(gs_sampler *s, const gs_params *params);
int gs_sampler_get_params(const gs_sampler *s, gs_params *params);
/* Diagnostic, no counterpart in the reference: how many rows of this
 * sampler's last sampling call on the full-vocabulary path (top_k = 0 or
 * beyond the small-k limit) were not finished by the increment-histogram
 * path but by its fallbacks (the first binned form, then the sort; same
 * tokens, slower).  Waits for `stream`, the stream that call ran on; 0 if
 * the last call did not use that path. */
int gs_sampler_fallback_rows(gs_sampler *s, void *stream, size_t *n);
/* set_seed (src/sampler.rs:5) for this sampler's stream. */
int gs_sampler_set_seed(gs_sampler *s, uint64_t seed);
/* Raw LCG state, so a decode trace can be checkpointed and resumed. */
int gs_sampler_get_state(const gs_sampler *s, uint64_t *state);
int gs_sampler_set_state(gs_sampler *s, uint64_t state);

/* Pre-allocate the full-vocabulary scratch (16*V bytes per row) for batches
 * of up to B rows, and for V > 32768 the virtual rows of the split and
 * chunked top-k paths (256 KB per row for up to 32 rows, or
 * ceil(V / 32768) KB per row for B rows, whichever is larger), e.g. before
 * capturing gs_sample_batch into a HIP graph (the batch call otherwise
 * allocates on first use; under capture, rows whose buffers are missing
 * take the one-workgroup-per-row path instead). */
int gs_sampler_reserve(gs_sampler *s, size_t B, size_t V);

/* ---- single row: sample(logits, recent) -> token -------------------------
 * Replaces sampler::sample (src/sampler.rs:35-79) at its call site
 * src/main.rs:280.  `logits` and `recent` may be host or device pointers.
 * One LCG draw is consumed iff temperature > 0, as in the reference.
 * Synchronous: returns after the token is in *out_token.
 * `logits` is not modified (the reference leaves it penalized and divided
 * by T; its only caller discards it, src/main.rs:305): gs_sample_mut is the
 * variant that leaves it as the reference does. */
int gs_sample(gs_sampler *s, const float *logits, size_t V,
              const uint32_t *recent, size_t W, uint32_t *out_token);

/* sample(&mut logits, ...) exactly as src/sampler.rs:35-41 takes it: the
 * token of gs_sample, and on return `logits` (host or device) holds what the
 * reference leaves in the caller's Vec: every id of `recent` penalized once
 * per occurrence (:37, apply_rep_penalty :23-30), then every logit divided
 * by T when T > 0 (:41; a row with T <= 0 returns before the division, :39).
 * `logits` is written only when the call returns GS_OK. */
int gs_sample_mut(gs_sampler *s, float *logits, size_t V,
                  const uint32_t *recent, size_t W, uint32_t *out_token);

/* ---- batched: B independent rows (new; no reference counterpart beyond
 * calling src/sampler.rs:35 once per row) ----------------------------------
 * d_logits   : device, row b at d_logits + b*ld (ld >= V), f32.
 * d_params   : device, B gs_params (heterogeneous rows), or NULL = the
 *              sampler's params for every row.
 * d_recent   : device, row b's window at d_recent + b*ld_recent, or NULL.
 * d_recent_len: device, B lengths (<= W), or NULL = W for every row.
 * d_u        : device, B uniform draws in [0,1), or NULL = the sampler's LCG
 *              stream (row b gets the b-th next draw; the host state advances
 *              by B if T > 0, by 0 if T <= 0).  NULL requires d_params NULL.
 * d_tokens   : device, B uint32 outputs.
 * d_status   : device, B int32 per-row statuses (GS_OK/GS_ERR_NAN/...), or NULL.
 * stream     : hipStream_t (NULL = default stream).
 * Scratch for rows that need the full-vocabulary path is owned by the
 * sampler and grows on demand (allocation happens outside kernels, before
 * the launch).
 * One sampler serves one stream at a time: its scratch and the chunked
 * top-k path's per-row counters are shared by all its calls, so its batched
 * calls must be stream-ordered one after the other, graph replays included
 * (two streams, or a replay beside an eager call, may race: a row's finish
 * can then be missed and its token left unwritten).
 * HIP graph capture: call gs_sampler_reserve(s, B, V) before capturing (a
 * call that would have to allocate under capture returns
 * GS_ERR_UNSUPPORTED), and pass d_u (a captured call with d_u == NULL and
 * T > 0 returns GS_ERR_UNSUPPORTED: the host LCG state would be frozen into
 * the graph and every replay would repeat the same draws).  Once a call has
 * been captured, buffers the sampler replaces later are kept until
 * gs_sampler_destroy, so earlier graphs never touch freed memory. */
int gs_sample_batch(gs_sampler *s, const float *d_logits, size_t B, size_t V,
                    size_t ld, const gs_params *d_params,
                    const uint32_t *d_recent, size_t ld_recent,
                    const uint32_t *d_recent_len, size_t W, const float *d_u,
                    uint32_t *d_tokens, int32_t *d_status, void *stream);

/* ---- batched, allocation-free --------------------------------------------
 * No counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  Same arguments, semantics and results as
 * gs_sample_batch, but every scratch buffer (per-row fallback flags, the
 * split top-k path's virtual rows, the full-vocabulary path's scratch) lives
 * in one statically sized device array of GS_NOALLOC_SCRATCH_BYTES per GPU,
 * part of the library's code object and held until the process ends.  The
 * call makes no hipMalloc/hipFree and no allocating library call.
 * Limit: the buffers of the paths the call can take must fit, otherwise
 * GS_ERR_UNSUPPORTED:
 *   fallback flags, 4 B per row rounded up to 256 B;
 *   + for V > 32768, the larger of the split top-k buffers (uniform params
 *     with 0 < top_k <= 128 and at most 32 rows: 8 B * (V/1024) *
 *     round_up(top_k, 4) per row) and the chunked top-k buffers (fewer
 *     rows than CUs: 8 B * ceil(V/32768) * 128 per row), rounded up to 256 B;
 *   + when d_params is given or the sampler's params need the
 *     full-vocabulary path (T > 0 and top_k == 0, top_k >= V or
 *     top_k > 1024): B rows of full-vocabulary scratch, about 25 B per
 *     vocabulary entry (3.8 MB per row at V = 152064, so at most 16 rows).
 * Top-k-only batches need no full-vocabulary scratch: C5's 1024 rows of
 * V = 152064, top_k = 50 fit.
 * Every call on one GPU shares that GPU's array (whichever sampler makes
 * it) and the array keeps the last call's contents: calls that overlap on
 * one GPU (two streams, or two threads) race and must be serialised by the
 * caller.  gs_sampler_fallback_rows reads its flags from the array, so it
 * reports the last allocation-free call on the GPU, whichever sampler made
 * it.  Nothing in the array needs to start at zero.  The chunked top-k
 * path's per-row counters (8 KB) are the sampler's own, allocated and
 * cleared by gs_sampler_create, and each call leaves them at zero. */
#define GS_NOALLOC_SCRATCH_BYTES (64u << 20)
int gs_sample_batch_noalloc(gs_sampler *s, const float *d_logits, size_t B, size_t V,
                            size_t ld, const gs_params *d_params,
                            const uint32_t *d_recent, size_t ld_recent,
                            const uint32_t *d_recent_len, size_t W, const float *d_u,
                            uint32_t *d_tokens, int32_t *d_status, void *stream);

/* ---- diagnostic: the reference's intermediate results -------------------
 * No counterpart in the reference's API: it exposes what src/sampler.rs:44-78
 * computes on the way to the token, for parity checks.  Per row b (device
 * buffers, any may be NULL):
 *   ids[b*cap + j], p[b*cap + j]  for j < min(n_kept, cap): the candidates
 *       after truncate(top_k) in the reference's order (scaled logit
 *       descending, equal values by index) and their post-softmax
 *       probabilities a_j / S (:55-56);
 *   n_kept[b]  candidates after truncate(top_k) (:48-50); 0 for a greedy
 *              row (T <= 0, :39) or a failed row;
 *   cut[b]     candidates after the nucleus cut (:59-66); n_kept if
 *              top_p >= 1;
 *   sums[2b], sums[2b+1]  S (:54) and s2 (:67; 1 if top_p >= 1);
 *   ties[b]    bit 0: two equal scaled logits meet at rank k (the
 *              truncation boundary), inside the kept prefix or at the
 *              nucleus cut; bit 1: the drawn element's value is shared by
 *              another element, so the token depends on the order the
 *              reference's sort_unstable_by gives equal keys (index
 *              ascending here).  Equal summands commute, so S, s2 and the
 *              cumulative sums never depend on that order. */
typedef struct {
    uint32_t *ids;
    float *p;
    size_t cap;
    uint32_t *n_kept;
    uint32_t *cut;
    float *sums;
    uint32_t *ties;
} gs_detail;

/* gs_sample_batch's arguments and tokens, plus `det`.  Every row with
 * T > 0 takes a sort-based kernel (slow: a diagnostic, not a sampling
 * path); tokens are the same as gs_sample_batch's. */
int gs_sample_detail(gs_sampler *s, const float *d_logits, size_t B, size_t V,
                     size_t ld, const gs_params *d_params,
                     const uint32_t *d_recent, size_t ld_recent,
                     const uint32_t *d_recent_len, size_t W, const float *d_u,
                     uint32_t *d_tokens, int32_t *d_status, const gs_detail *det,
                     void *stream);

/* ---- batched write-back of the reference's mutation ----------------------
 * Leaves rows [0, B) of d_logits as src/sampler.rs:37,41 leave each row it
 * samples: penalized per window occurrence (the row's window as
 * gs_sample_batch reads it: d_recent, d_recent_len, W), then divided by the
 * row's T when T > 0.  Stream-ordered on `stream`; call it after
 * gs_sample_batch on the same rows (the sampler reads the unmodified
 * logits).  Same argument meaning as gs_sample_batch; d_params NULL = this
 * sampler's params. */
int gs_logits_writeback(gs_sampler *s, float *d_logits, size_t B, size_t V, size_t ld,
                        const gs_params *d_params, const uint32_t *d_recent, size_t ld_recent,
                        const uint32_t *d_recent_len, size_t W, void *stream);

/* ---- device-resident decode helpers (decode loop, src/main.rs:279-311) ---
 * Append each row's token to its ring window: window[b*ld + (pos % W)] =
 * tokens[b].  The penalty only depends on how often each id occurs in the
 * window, so a ring is equivalent to the reference's FIFO (src/main.rs:302-303)
 * once the window is full. */
int gs_window_push(uint32_t *d_window, size_t B, size_t ld, size_t W, size_t pos,
                   const uint32_t *d_tokens, void *stream);

/* Synthetic logits for device-resident benchmarks and tests:
 * out[b*ld + c] = sigma * IrwinHall4(splitmix64(seed ^ splitmix64(counter0 + b*V + c))).
 * Deterministic and reproducible on the host. */
int gs_synth_logits(float *d_out, size_t B, size_t V, size_t ld, uint64_t seed,
                    uint64_t counter0, float sigma, void *stream);

/* Library limits and build identification. */
int gs_limits(uint32_t *max_vocab, uint32_t *max_window);
const char *gs_version(void);

#ifdef __cplusplus
}
#endif
#endif /* GS_SAMPLER_H */
