// gs_decode.hip -- device-resident decode step (declared in include/gs_decode.h).
//
// The body of gguf-rs-cli's generate_collect (src/main.rs:279-311) for B
// independent rows, with the loop state on the device: a per-row copy of the
// reference LCG (src/sampler.rs:3-12), the recent-id ring, the stop check and
// the generated ids.  A step is the GEMV (logits in HBM), then the sampler,
// whose last kernel commits each row and draws its next u: stream-ordered
// launches with no host synchronisation, so a caller can capture many steps
// in one HIP graph.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include <vector>

#include "../../include/gs_decode.h"
#include "gs_kernels.hpp"
#include "gs_lcg.hpp"

namespace gs {

static_assert(sizeof(gs_decode_row) == 24, "gs_decode_row layout");

// The first step's draws (gs_decode_init): u = rand_f32() (src/sampler.rs:7-12)
// for rows whose temperature is > 0; the state then moves one step.  The
// reference draws only past its greedy return (src/sampler.rs:39, 72).
__global__ void decode_first_draw_kernel(gs_decode_row *rows, int B, const gs_params *params, float T_all, float *u)
{
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= B) return;
    const float T = params ? params[b].temperature : T_all;
    if (T > 0.0f) {
        const uint64_t s = rows[b].rng;
        u[b] = lcg_value(s);
        rows[b].rng = lcg_jump(s, 1);
    }
}

// Commit every row's token, one thread per row (decode_commit_row).
__global__ void decode_commit_kernel(DecodeHook h, int B, const uint32_t *tokens, const int32_t *status)
{
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b < B) decode_commit_row(h, b, tokens[b], status ? status[b] : GS_OK);
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

int make_hook(gs_sampler *s, const gs_params *d_params, const gs_decode_ctx *c, gs::DecodeHook *h)
{
    gs_params p;
    if (!s || gs_sampler_get_params(s, &p) != GS_OK) return GS_ERR_INVALID;
    h->rows = c->rows;
    h->stop = c->stop;
    h->n_stop = (int)c->n_stop;
    h->max_new = c->max_new;
    h->window = c->W ? c->window : nullptr;
    h->ld_window = c->ld_window;
    h->W = (uint32_t)c->W;
    h->window_len = c->W ? c->window_len : nullptr;
    h->generated = c->generated;
    h->ld_generated = c->ld_generated;
    h->next = c->next;
    h->u = c->u;
    h->n_active = c->n_active;
    h->params = d_params;
    h->T_all = p.temperature;
    return GS_OK;
}

} // namespace

extern "C" {

int gs_decode_init(gs_sampler *s, const gs_params *d_params, const gs_decode_ctx *ctx, const uint64_t *seeds,
                   const uint32_t *init_len, void *stream)
{
    int rc = check_ctx(ctx);
    if (rc) return rc;
    gs_params p;
    if (!s || gs_sampler_get_params(s, &p) != GS_OK) return GS_ERR_INVALID;
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
    const uint32_t nb = (uint32_t)B;
    hipStream_t st = (hipStream_t)stream;
    if (hipMemcpyAsync(ctx->rows, rows.data(), B * sizeof(gs_decode_row), hipMemcpyHostToDevice, st) != hipSuccess)
        return GS_ERR_HIP;
    if (ctx->W && hipMemcpyAsync(ctx->window_len, wl.data(), B * sizeof(uint32_t), hipMemcpyHostToDevice, st) != hipSuccess)
        return GS_ERR_HIP;
    if (ctx->n_active && hipMemcpyAsync(ctx->n_active, &nb, sizeof(nb), hipMemcpyHostToDevice, st) != hipSuccess)
        return GS_ERR_HIP;
    hipLaunchKernelGGL(gs::decode_first_draw_kernel, dim3((unsigned)((B + 255) / 256)), dim3(256), 0, st,
                       ctx->rows, (int)B, d_params, p.temperature, ctx->u);
    if (hipGetLastError() != hipSuccess) return GS_ERR_HIP;
    return hipStreamSynchronize(st) == hipSuccess ? GS_OK : GS_ERR_HIP;
}

int gs_decode_commit(gs_sampler *s, const gs_params *d_params, const gs_decode_ctx *ctx, void *stream)
{
    int rc = check_ctx(ctx);
    if (rc) return rc;
    gs::DecodeHook h;
    if ((rc = make_hook(s, d_params, ctx, &h))) return rc;
    if (ctx->B == 0) return GS_OK;
    const int B = (int)ctx->B;
    hipLaunchKernelGGL(gs::decode_commit_kernel, dim3((B + 255) / 256), dim3(256), 0, (hipStream_t)stream, h, B,
                       (const uint32_t *)ctx->tokens, (const int32_t *)ctx->status);
    return hipGetLastError() == hipSuccess ? GS_OK : GS_ERR_HIP;
}

int gs_decode_step(gs_sampler *s, const gs_qmatrix *lm_head, const float *d_x, float *d_logits, size_t V,
                   size_t ld, const gs_params *d_params, const gs_decode_ctx *ctx, void *stream)
{
    int rc = check_ctx(ctx);
    if (rc) return rc;
    if (!d_logits) return GS_ERR_INVALID;
    gs::DecodeHook h;
    if ((rc = make_hook(s, d_params, ctx, &h))) return rc;
    if (lm_head) {
        uint32_t qt;
        size_t rows, cols;
        if ((rc = gs_qmatrix_shape(lm_head, &qt, &rows, &cols))) return rc;
        if (rows != V || ld != V || !d_x) return GS_ERR_INVALID;
        if ((rc = gs_gemv(lm_head, d_x, ctx->B, d_logits, stream))) return rc;
    }
    return gs::sample_batch(s, d_logits, ctx->B, V, ld, d_params, ctx->W ? ctx->window : nullptr, ctx->ld_window,
                            ctx->W ? ctx->window_len : nullptr, ctx->W, ctx->u, ctx->tokens, ctx->status, &h,
                            stream);
}

} // extern "C"
