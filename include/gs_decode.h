/*
 * gs_decode.h -- C ABI of the device-resident decode step: the logits stay in
 * HBM, and the decode loop's per-row state lives on the device, so many steps
 * can run (or be captured in one HIP graph) with no host round trip.
 *
 * It restates the body of gguf-rs-cli's generate_collect (src/main.rs:258-313),
 * one iteration per call, for B independent rows:
 *
 *   let next = sampler::sample(last, T, top_k, top_p, rep, recent);  src/main.rs:280
 *   if stops.contains(&(next as u32)) { break; }                     src/main.rs:281
 *   if generated.len() >= max         { break; }                     src/main.rs:282
 *   recent.push(next as u32);                                        src/main.rs:302
 *   if recent.len() > 64 { recent.remove(0); }                       src/main.rs:303
 *   generated.push(next as u32);                                     src/main.rs:304
 *   *last = model.forward_gpu(next, *pos, g);                        src/main.rs:306-309
 *
 * where the reference reads the logits back to the host every token
 * (Gpu::read_logits, src/gpu/mod.rs:364-381) and samples on the CPU.  Here the
 * logits come from gs_gemv (include/gs_gemv.h) into a device buffer and the
 * sampler reads them there; only the 4-byte token of each row is produced.
 * The forward pass before the output projection (the next row of x) is the
 * caller's.  The smart-context rebuild (src/main.rs:284-296) is the caller's
 * too: pass max_new no larger than the positions left in its context.
 *
 * Row state: each row carries its own copy of the reference LCG
 * (src/sampler.rs:3-12), seeded like set_seed (src/sampler.rs:5).  A row
 * with B = 1 and the CLI's seed reproduces the reference's token stream
 * exactly (one draw per step iff T > 0; the step that samples a stop token
 * consumes its draw, as at src/main.rs:280-281).  Each step's draw is made
 * ahead of it: by gs_decode_init for the first step, then by the commit of
 * the step before, for rows that go on (ctx->u holds it).  So a finished
 * row's rng is the reference's final state; a running row's is one draw
 * ahead of the steps it has taken.
 *
 * The window is a ring of W slots per row (W = 64 in the reference): the
 * penalty depends only on how often each id occurs in it, so the ring equals
 * the reference's FIFO.  Same status codes as gs_sampler.h.
 */
#ifndef GS_DECODE_H
#define GS_DECODE_H

#include <stddef.h>
#include <stdint.h>

#include "gs_gemv.h"
#include "gs_sampler.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Why a row stopped (gs_decode_row.done). */
#define GS_DONE_RUNNING 0u
#define GS_DONE_STOP    1u   /* sampled a stop token (src/main.rs:281) */
#define GS_DONE_MAX     2u   /* generated max_new tokens (src/main.rs:282) */
#define GS_DONE_ERROR   3u   /* the sampler failed on the row (a NaN logit: the reference panics) */

/* Most stop ids one call accepts (the reference's set is the EOS ids plus a
 * template's extras, src/tokenizer/chat.rs:57-72). */
#define GS_MAX_STOP 256u

/* Per-row decode state, device memory, 24 bytes. */
typedef struct gs_decode_row {
    uint64_t rng;    /* LCG state; a fresh row holds its seed (src/sampler.rs:5) */
    uint32_t n_gen;  /* generated.len() */
    uint32_t wpos;   /* ids written to the window so far, initial fill included */
    uint32_t done;   /* GS_DONE_* */
    uint32_t last;   /* the last sampled token (the stop token once done == GS_DONE_STOP) */
} gs_decode_row;

/* The device buffers of a batch of B decoding rows.  All pointers are device
 * memory the caller owns.  The struct is read at call time (its values are
 * what a captured graph replays). */
typedef struct gs_decode_ctx {
    size_t B;
    gs_decode_row *rows;        /* [B] */
    uint32_t *window;           /* [B][ld_window] ring of the last W ids, or NULL (W = 0) */
    size_t ld_window;
    size_t W;                   /* <= GS_MAX_WINDOW */
    uint32_t *window_len;       /* [B] min(wpos, W), kept by the commit; the sampler reads it */
    const uint32_t *stop;       /* [n_stop] stop ids, or NULL */
    size_t n_stop;              /* <= GS_MAX_STOP */
    uint32_t max_new;           /* `max` of src/main.rs:282 */
    uint32_t *generated;        /* [B][ld_generated] generated ids, or NULL */
    size_t ld_generated;        /* ids past ld_generated are not stored */
    uint32_t *next;             /* [B] the token each running row feeds to its next forward, or NULL */
    float *u;                   /* [B] the next step's draws */
    uint32_t *tokens;           /* [B] scratch: this step's sampled tokens */
    int32_t *status;            /* [B] per-row sampler statuses, or NULL */
    uint32_t *n_active;         /* [1] rows still running (set by init, decremented as rows end), or NULL */
} gs_decode_ctx;

/* Reset B rows: rng = seeds[b] (host array), n_gen = 0, done = running,
 * wpos = window_len[b] = init_len[b] (host array or NULL = 0; the caller has
 * written those ids to window slots 0..init_len-1, the reference's `recent`
 * at the start of a turn, oldest first, src/main.rs:98, 198), *n_active = B;
 * then the first step's draws: u[b] = rand_f32() of row b's LCG
 * (src/sampler.rs:7-12) iff the row's temperature (d_params[b], or the
 * sampler's when d_params is NULL) is > 0.  Synchronous. */
int gs_decode_init(gs_sampler *s, const gs_params *d_params, const gs_decode_ctx *ctx, const uint64_t *seeds,
                   const uint32_t *init_len, void *stream);

/* Commit this step's tokens (ctx->tokens, statuses ctx->status or all OK)
 * for every running row, in the reference's order: a failed sample ends the
 * row (GS_DONE_ERROR); a stop token ends it (GS_DONE_STOP); else a row with
 * n_gen >= max_new ends (GS_DONE_MAX); else the token goes to the window
 * ring, to generated[n_gen] and to next[b], n_gen grows by one, and the
 * next step's u[b] is drawn (T > 0).  For callers that sample on their own;
 * gs_decode_step does this inside the sampler's last kernel. */
int gs_decode_commit(gs_sampler *s, const gs_params *d_params, const gs_decode_ctx *ctx, void *stream);

/* One whole decode step, stream-ordered and free of host synchronisation
 * and allocation (call gs_sampler_reserve(s, B, V) first when the rows take
 * the full-vocabulary or split paths):
 *   lm_head != NULL: d_logits[b*V + r] = gs_gemv(lm_head, d_x)   (V = rows of lm_head, ld = V;
 *                    one pass over the matrix per row b: for small B, see gs_gemv)
 *   lm_head == NULL: the caller's logits are already in d_logits (row stride ld)
 *   then gs_sample_batch with the ring window and ctx->u, whose last kernel
 *   commits each row as gs_decode_commit does.
 * Rows that have finished are still sampled (their tokens are discarded);
 * a serving loop compacts its batch instead. */
int gs_decode_step(gs_sampler *s, const gs_qmatrix *lm_head, const float *d_x,
                   float *d_logits, size_t V, size_t ld, const gs_params *d_params,
                   const gs_decode_ctx *ctx, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* GS_DECODE_H */
