// gs_decode_dev.hpp -- one row's decode-loop commit (src/main.rs:280-304),
// shared by the commit kernel and the sampler's last kernel of a step.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/gs_decode.h"
#include "gs_lcg.hpp"

namespace gs {

// The decode state a kernel commits into (the fields of gs_decode_ctx plus
// the per-row temperatures for the next draw).  rows == nullptr: no commit.
struct DecodeHook {
    gs_decode_row *rows;
    const uint32_t *stop;
    int n_stop;
    uint32_t max_new;
    uint32_t *window;
    size_t ld_window;
    uint32_t W;
    uint32_t *window_len;
    uint32_t *generated;
    size_t ld_generated;
    uint32_t *next;
    float *u;
    uint32_t *n_active;
    const gs_params *params;     // per row, or null: T_all
    float T_all;
};

// Commit row b's token: one thread.  Order of src/main.rs:280-304; a failed
// sample (the reference's panic) ends the row too.  A row that goes on draws
// the next step's u now (src/sampler.rs:7-12, iff T > 0).
__device__ __forceinline__ void decode_commit_row(const DecodeHook &h, int b, uint32_t tok, int status)
{
    gs_decode_row r = h.rows[b];
    if (r.done != GS_DONE_RUNNING) return;
    r.last = tok;
    bool is_stop = false;
    for (int i = 0; i < h.n_stop; i++) is_stop |= h.stop[i] == tok;
    if (status != GS_OK) {
        r.done = GS_DONE_ERROR;
    } else if (is_stop) {
        r.done = GS_DONE_STOP;
    } else if (r.n_gen >= h.max_new) {
        r.done = GS_DONE_MAX;
    } else {
        if (h.W) {
            h.window[(size_t)b * h.ld_window + r.wpos % h.W] = tok;
            r.wpos++;
            h.window_len[b] = r.wpos < h.W ? r.wpos : h.W;
        }
        if (h.generated && r.n_gen < h.ld_generated) h.generated[(size_t)b * h.ld_generated + r.n_gen] = tok;
        if (h.next) h.next[b] = tok;
        r.n_gen++;
        const float T = h.params ? h.params[b].temperature : h.T_all;
        if (T > 0.0f) {
            h.u[b] = lcg_value(r.rng);
            r.rng = lcg_jump(r.rng, 1);
        }
    }
    if (r.done != GS_DONE_RUNNING && h.n_active) atomicSub(h.n_active, 1u);
    h.rows[b] = r;
}

} // namespace gs
