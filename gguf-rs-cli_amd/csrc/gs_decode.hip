// gs_decode.hip -- device-resident decode step (declared in include/gs_decode.h).
//
// The body of gguf-rs-cli's generate_collect (src/main.rs:279-311) for B
// independent rows, with the loop state on the device: a per-row copy of the
// reference LCG (src/sampler.rs:3-12), the recent-id ring, the stop check and
// the generated ids.  A step is GEMV (logits in HBM) -> draw -> sample ->
// commit, four stream-ordered launches with no host synchronisation, so a
// caller can capture many steps in one HIP graph.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include <vector>

#include "../../include/gs_decode.h"
#include "gs_lcg.hpp"

namespace gs {

static_assert(sizeof(gs_decode_row) == 24, "gs_decode_row layout");

constexpr int kCommitThreads = 1024;

// One thread per row: u = rand_f32() (src/sampler.rs:7-12) for running rows
// whose temperature is > 0; the state then moves one step.  The reference
// draws only past its greedy return (src/sampler.rs:39, 72).
__global__ void decode_draw_kernel(gs_decode_row *rows, int B, const gs_params *params, float T_all, float *u)
{
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= B) return;
    gs_decode_row r = rows[b];
    float v = 0.0f;
    const float T = params ? params[b].temperature : T_all;
    if (r.done == GS_DONE_RUNNING && T > 0.0f) {
        v = lcg_value(r.rng);
        rows[b].rng = lcg_jump(r.rng, 1);
    }
    u[b] = v;
}

struct CommitArgs {
    gs_decode_row *rows;
    int B;
    const uint32_t *tokens;
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
    uint32_t *n_active;
};

// One workgroup over all rows (a few hundred bytes of state per step).  The
// order of the checks is src/main.rs:281, 282, 302-304.
__global__ void __launch_bounds__(kCommitThreads) decode_commit_kernel(CommitArgs a)
{
    __shared__ uint32_t stop[GS_MAX_STOP];
    __shared__ uint32_t active[kCommitThreads / 64];
    const int t = threadIdx.x;
    for (int i = t; i < a.n_stop; i += kCommitThreads) stop[i] = a.stop[i];
    __syncthreads();
    uint32_t running = 0;
    for (int b = t; b < a.B; b += kCommitThreads) {
        gs_decode_row r = a.rows[b];
        if (r.done != GS_DONE_RUNNING) continue;
        const uint32_t tok = a.tokens[b];
        r.last = tok;
        bool is_stop = false;
        for (int i = 0; i < a.n_stop; i++) is_stop |= stop[i] == tok;
        if (is_stop) {
            r.done = GS_DONE_STOP;
        } else if (r.n_gen >= a.max_new) {
            r.done = GS_DONE_MAX;
        } else {
            if (a.W) {
                a.window[(size_t)b * a.ld_window + r.wpos % a.W] = tok;
                r.wpos++;
                a.window_len[b] = r.wpos < a.W ? r.wpos : a.W;
            }
            if (a.generated && r.n_gen < a.ld_generated) a.generated[(size_t)b * a.ld_generated + r.n_gen] = tok;
            if (a.next) a.next[b] = tok;
            r.n_gen++;
            running++;
        }
        a.rows[b] = r;
    }
    if (a.n_active) {
        for (int off = 32; off > 0; off >>= 1) running += __shfl_xor(running, off);
        if ((t & 63) == 0) active[t >> 6] = running;
        __syncthreads();
        if (t == 0) {
            uint32_t n = 0;
            for (int w = 0; w < kCommitThreads / 64; w++) n += active[w];
            *a.n_active = n;
        }
    }
}

} // namespace gs

namespace {

int check_ctx(const gs_decode_ctx *c)
{
    if (!c || !c->rows || !c->u || !c->tokens || c->B > 0x7fffffff) return GS_ERR_INVALID;
    if (c->W && (!c->window || !c->window_len || c->ld_window < c->W)) return GS_ERR_INVALID;
    if (c->W > GS_MAX_WINDOW || c->n_stop > GS_MAX_STOP) return GS_ERR_UNSUPPORTED;
    if (c->n_stop && !c->stop) return GS_ERR_INVALID;
    if (c->generated && c->ld_generated == 0) return GS_ERR_INVALID;
    return GS_OK;
}

} // namespace

extern "C" {

int gs_decode_init(const gs_decode_ctx *ctx, const uint64_t *seeds, const uint32_t *init_len, void *stream)
{
    int rc = check_ctx(ctx);
    if (rc) return rc;
    if (!seeds && ctx->B) return GS_ERR_INVALID;
    const size_t B = ctx->B;
    if (B == 0) return GS_OK;
    std::vector<gs_decode_row> rows(B);
    std::vector<uint32_t> wl(B);
    for (size_t b = 0; b < B; b++) {
        const uint32_t n = init_len ? init_len[b] : 0;
        if (n > ctx->W) return GS_ERR_INVALID;
        rows[b] = gs_decode_row{seeds[b], 0, n, GS_DONE_RUNNING, 0};
        wl[b] = n;
    }
    hipStream_t st = (hipStream_t)stream;
    if (hipMemcpyAsync(ctx->rows, rows.data(), B * sizeof(gs_decode_row), hipMemcpyHostToDevice, st) != hipSuccess)
        return GS_ERR_HIP;
    if (ctx->W && hipMemcpyAsync(ctx->window_len, wl.data(), B * sizeof(uint32_t), hipMemcpyHostToDevice, st) != hipSuccess)
        return GS_ERR_HIP;
    return hipStreamSynchronize(st) == hipSuccess ? GS_OK : GS_ERR_HIP;
}

int gs_decode_draw(gs_sampler *s, const gs_params *d_params, const gs_decode_ctx *ctx, void *stream)
{
    int rc = check_ctx(ctx);
    if (rc) return rc;
    gs_params p;
    if (!s || gs_sampler_get_params(s, &p) != GS_OK) return GS_ERR_INVALID;
    if (ctx->B == 0) return GS_OK;
    const int B = (int)ctx->B;
    hipLaunchKernelGGL(gs::decode_draw_kernel, dim3((B + 255) / 256), dim3(256), 0, (hipStream_t)stream,
                       ctx->rows, B, d_params, p.temperature, ctx->u);
    return hipGetLastError() == hipSuccess ? GS_OK : GS_ERR_HIP;
}

int gs_decode_commit(const gs_decode_ctx *ctx, void *stream)
{
    int rc = check_ctx(ctx);
    if (rc) return rc;
    if (ctx->B == 0) return GS_OK;
    gs::CommitArgs a;
    a.rows = ctx->rows;
    a.B = (int)ctx->B;
    a.tokens = ctx->tokens;
    a.stop = ctx->stop;
    a.n_stop = (int)ctx->n_stop;
    a.max_new = ctx->max_new;
    a.window = ctx->window;
    a.ld_window = ctx->ld_window;
    a.W = (uint32_t)ctx->W;
    a.window_len = ctx->window_len;
    a.generated = ctx->generated;
    a.ld_generated = ctx->ld_generated;
    a.next = ctx->next;
    a.n_active = ctx->n_active;
    hipLaunchKernelGGL(gs::decode_commit_kernel, dim3(1), dim3(gs::kCommitThreads), 0, (hipStream_t)stream, a);
    return hipGetLastError() == hipSuccess ? GS_OK : GS_ERR_HIP;
}

int gs_decode_step(gs_sampler *s, const gs_qmatrix *lm_head, const float *d_x, float *d_logits, size_t V,
                   size_t ld, const gs_params *d_params, const gs_decode_ctx *ctx, void *stream)
{
    int rc = check_ctx(ctx);
    if (rc) return rc;
    if (!s || !d_logits) return GS_ERR_INVALID;
    if (lm_head) {
        uint32_t qt;
        size_t rows, cols;
        if ((rc = gs_qmatrix_shape(lm_head, &qt, &rows, &cols))) return rc;
        if (rows != V || ld != V || !d_x) return GS_ERR_INVALID;
        if ((rc = gs_gemv(lm_head, d_x, ctx->B, d_logits, stream))) return rc;
    }
    if ((rc = gs_decode_draw(s, d_params, ctx, stream))) return rc;
    if ((rc = gs_sample_batch(s, d_logits, ctx->B, V, ld, d_params, ctx->W ? ctx->window : nullptr,
                              ctx->ld_window, ctx->W ? ctx->window_len : nullptr, ctx->W, ctx->u,
                              ctx->tokens, ctx->status, stream)))
        return rc;
    return gs_decode_commit(ctx, stream);
}

} // extern "C"
