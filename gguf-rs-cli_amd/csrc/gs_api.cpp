// gs_api.cpp -- C ABI of the gfx950 token sampler (declared in include/gs_sampler.h).
//
// Host side of the drop-in for gguf-rs-cli src/sampler.rs.  Owns the
// sampler's LCG state (src/sampler.rs:3-12), device staging for the
// single-row call and the scratch of the full-vocabulary path.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include <mutex>
#include <new>
#include <vector>

#include "../../include/gs_sampler.h"
#include "gs_kernels.hpp"
#include "gs_lcg.hpp"

struct gs_sampler {
    gs_params params;
    uint64_t state;              // LCG state (pre-update value of the next draw)
    int device;
    hipStream_t stream;          // stream of the synchronous single-row call
    float *d_row;                // staging for host logits
    size_t row_cap;
    uint32_t *h_rec;             // pinned, mapped: a host window is copied here and read
    uint32_t *d_rec_map;         // by the kernel through this alias (no copy command)
    uint32_t *h_tok;             // pinned, mapped, coherent: kernel writes the token here
    int32_t *h_status;
    uint64_t *h_done;            // single-row calls: (sequence << 32) | (status & 0xff) << 24 | token
    uint32_t *d_tok_map;         // device aliases of h_tok / h_status / h_done
    int32_t *d_status_map;
    uint64_t *d_done_map;
    uint32_t seq;
    const char *dev_lo, *dev_hi; // last device allocation seen by is_device_ptr
    uint32_t *scratch;           // full-vocabulary path
    size_t scratch_elems;
    int32_t *fb;                 // per-row fallback flags of the full-vocabulary path
    size_t fb_cap;
    size_t fb_rows;              // rows of the last call that launched that path (0: none)
    void *split;                 // split top-k path: virtual rows (f32), then their ids (u32)
    size_t split_cap;
    const int32_t *fb_last;      // fallback flags of the last call (own buffer or the static scratch)
    bool captured;               // a call was recorded into a graph: buffers are never freed before destroy
    void **retired;              // buffers replaced after a capture, freed by gs_sampler_destroy
    size_t n_retired, cap_retired;
    int n_cus;                   // compute units of the device (0: not queried yet)
    hipStream_t side;            // batches with per-row params: small rows beside the full rows
    hipEvent_t ev_fork, ev_join;
    uint32_t *csync;             // chunked top-k path: per-row chunk counters, zero between calls
};

namespace gs { int init_static_scratch(int device); }

namespace {
// Is `stream` being captured into a HIP graph?
int capturing(hipStream_t stream, bool *cap)
{
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cs) != hipSuccess) { (void)hipGetLastError(); return GS_ERR_HIP; }
    *cap = cs != hipStreamCaptureStatusNone;
    return GS_OK;
}
} // namespace

namespace {

// Device pointer test with a one-allocation cache: consecutive rows of one
// device tensor skip the runtime query.
bool is_device_ptr(gs_sampler *s, const void *p)
{
    const char *c = (const char *)p;
    if (c >= s->dev_lo && c < s->dev_hi) return true;
    hipPointerAttribute_t at;
    if (hipPointerGetAttributes(&at, p) != hipSuccess) { (void)hipGetLastError(); return false; }
    const bool dev = at.type == hipMemoryTypeDevice || at.type == hipMemoryTypeManaged;
    if (dev) {
        hipDeviceptr_t base = nullptr;
        size_t size = 0;
        if (hipMemGetAddressRange(&base, &size, (hipDeviceptr_t)p) == hipSuccess && base) {
            s->dev_lo = (const char *)base;
            s->dev_hi = (const char *)base + size;
        } else {
            (void)hipGetLastError();
        }
    }
    return dev;
}

// Grow a sampler-owned device buffer.  Once a call of this sampler has been
// captured into a HIP graph the old buffer may still be referenced by that
// graph, so it is kept (freed by gs_sampler_destroy) instead of freed.
int grow(gs_sampler *s, void **buf, size_t *cap, size_t need_bytes)
{
    if (*cap >= need_bytes) return GS_OK;
    if (*buf && s->captured) {
        if (s->n_retired == s->cap_retired) {
            const size_t nc = s->cap_retired ? 2 * s->cap_retired : 8;
            void **r = (void **)realloc(s->retired, nc * sizeof(void *));
            if (!r) return GS_ERR_NOMEM;
            s->retired = r;
            s->cap_retired = nc;
        }
        s->retired[s->n_retired++] = *buf;
        *buf = nullptr;
        *cap = 0;
    }
    if (*buf) { (void)hipFree(*buf); *buf = nullptr; *cap = 0; }
    if (hipMalloc(buf, need_bytes) != hipSuccess) { (void)hipGetLastError(); *buf = nullptr; return GS_ERR_NOMEM; }
    *cap = need_bytes;
    return GS_OK;
}

// Compute units of the sampler's device (queried once).
int num_cus(gs_sampler *s)
{
    if (!s->n_cus) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, s->device) != hipSuccess || n <= 0) {
            (void)hipGetLastError();
            n = 256;
        }
        s->n_cus = n;
    }
    return s->n_cus;
}

bool needs_full_path(const gs_params &p, size_t V)
{
    if (!(p.temperature > 0.0f) || V <= 1) return false;
    size_t keep = (p.top_k > 0 && p.top_k < V) ? p.top_k : V;
    return keep >= V || keep > (size_t)gs::kMaxTopK;
}

// Buffer of the split top-k path for `rows` rows of width `width`: the
// virtual rows' values, then their ids.
size_t split_bytes(size_t rows, size_t width) { return rows * width * 8; }
// Buffer of the chunked top-k path (virtual rows of stride chunk_stride).
size_t chunk_bytes(size_t B, size_t V) { return split_bytes(B, gs::chunk_stride(V)); }

int reserve_split(gs_sampler *s, size_t rows, size_t width)
{
    return grow(s, &s->split, &s->split_cap, split_bytes(rows, width));
}

hipError_t launch_split_rows(void *buf, const gs::RowArgs &a, size_t B, size_t width, hipStream_t st)
{
    float *vrow = (float *)buf;
    return gs::launch_split(a, (int)B, vrow, (uint32_t *)(vrow + B * width), st);
}

int reserve_scratch(gs_sampler *s, size_t rows, size_t V)
{
    void *f = s->fb;
    int rcf = grow(s, &f, &s->fb_cap, (rows ? rows : 1) * sizeof(int32_t));
    s->fb = (int32_t *)f;
    if (rcf) return rcf;
    size_t elems = rows * gs::scratch_u32_per_row(V);
    size_t cap = s->scratch_elems * sizeof(uint32_t);
    void *p = s->scratch;
    int rc = grow(s, &p, &cap, elems * sizeof(uint32_t));
    s->scratch = (uint32_t *)p;
    s->scratch_elems = cap / sizeof(uint32_t);
    return rc;
}

} // namespace

extern "C" {

int gs_sampler_create(const gs_params *params, uint64_t seed, gs_sampler **out)
{
    if (!params || !out) return GS_ERR_INVALID;
    *out = nullptr;
    gs_sampler *s = new (std::nothrow) gs_sampler();
    if (!s) return GS_ERR_NOMEM;
    memset(s, 0, sizeof(*s));
    s->params = *params;
    s->state = seed;
    if (hipGetDevice(&s->device) != hipSuccess) { delete s; return GS_ERR_HIP; }
    if (hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking) != hipSuccess) { delete s; return GS_ERR_HIP; }
    if (hipStreamCreateWithFlags(&s->side, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreateWithFlags(&s->ev_fork, hipEventDisableTiming) != hipSuccess ||
        hipEventCreateWithFlags(&s->ev_join, hipEventDisableTiming) != hipSuccess) {
        gs_sampler_destroy(s);
        return GS_ERR_HIP;
    }
    if (hipMalloc((void **)&s->csync, 2 * sizeof(uint32_t) * gs::kCSyncRows) != hipSuccess ||
        hipMemsetAsync(s->csync, 0, 2 * sizeof(uint32_t) * gs::kCSyncRows, s->stream) != hipSuccess ||
        hipStreamSynchronize(s->stream) != hipSuccess) {
        gs_sampler_destroy(s);
        return GS_ERR_HIP;
    }
    // set-up of gs_sample_batch_noalloc's scratch on this device (once per device)
    if (gs::init_static_scratch(s->device) != GS_OK) { gs_sampler_destroy(s); return GS_ERR_HIP; }
    if (hipHostMalloc((void **)&s->h_tok, 64, hipHostMallocMapped | hipHostMallocCoherent) != hipSuccess ||
        hipHostGetDevicePointer((void **)&s->d_tok_map, s->h_tok, 0) != hipSuccess) {
        gs_sampler_destroy(s);
        return GS_ERR_HIP;
    }
    s->h_status = (int32_t *)(s->h_tok + 4);
    s->d_status_map = (int32_t *)(s->d_tok_map + 4);
    if (hipHostMalloc((void **)&s->h_rec, sizeof(uint32_t) * gs::kMaxWindow,
                      hipHostMallocMapped | hipHostMallocCoherent) != hipSuccess ||
        hipHostGetDevicePointer((void **)&s->d_rec_map, s->h_rec, 0) != hipSuccess) {
        gs_sampler_destroy(s);
        return GS_ERR_HIP;
    }
    s->h_done = reinterpret_cast<uint64_t *>(s->h_tok + 8);        // 32 bytes in: 8-byte aligned
    s->d_done_map = reinterpret_cast<uint64_t *>(s->d_tok_map + 8);
    *(volatile uint64_t *)s->h_done = 0u;
    *out = s;
    return GS_OK;
}

int gs_sampler_destroy(gs_sampler *s)
{
    if (!s) return GS_ERR_INVALID;
    int dev;
    (void)hipGetDevice(&dev);
    (void)hipSetDevice(s->device);
    if (s->stream) (void)hipStreamSynchronize(s->stream);
    if (s->d_row) (void)hipFree(s->d_row);
    if (s->h_rec) (void)hipHostFree(s->h_rec);
    if (s->scratch) (void)hipFree(s->scratch);
    if (s->fb) (void)hipFree(s->fb);
    if (s->split) (void)hipFree(s->split);
    if (s->csync) (void)hipFree(s->csync);
    for (size_t i = 0; i < s->n_retired; i++) (void)hipFree(s->retired[i]);
    free(s->retired);
    if (s->h_tok) (void)hipHostFree(s->h_tok);
    if (s->side) (void)hipStreamSynchronize(s->side);
    if (s->ev_fork) (void)hipEventDestroy(s->ev_fork);
    if (s->ev_join) (void)hipEventDestroy(s->ev_join);
    if (s->side) (void)hipStreamDestroy(s->side);
    if (s->stream) (void)hipStreamDestroy(s->stream);
    (void)hipSetDevice(dev);
    delete s;
    return GS_OK;
}

int gs_sampler_set_params(gs_sampler *s, const gs_params *params)
{
    if (!s || !params) return GS_ERR_INVALID;
    s->params = *params;
    return GS_OK;
}

int gs_sampler_get_params(const gs_sampler *s, gs_params *params)
{
    if (!s || !params) return GS_ERR_INVALID;
    *params = s->params;
    return GS_OK;
}

int gs_sampler_set_seed(gs_sampler *s, uint64_t seed)
{
    if (!s) return GS_ERR_INVALID;
    s->state = seed;
    return GS_OK;
}

int gs_sampler_fallback_rows(gs_sampler *s, void *stream, size_t *n)
{
    if (!s || !n) return GS_ERR_INVALID;
    *n = 0;
    if (!s->fb_rows) return GS_OK;
    std::vector<int32_t> h(s->fb_rows);
    hipStream_t st = (hipStream_t)stream;
    if (hipMemcpyAsync(h.data(), s->fb_last, h.size() * sizeof(int32_t), hipMemcpyDeviceToHost, st) != hipSuccess ||
        hipStreamSynchronize(st) != hipSuccess)
        return GS_ERR_HIP;
    for (int32_t f : h) *n += f != 0;
    return GS_OK;
}

int gs_sampler_get_state(const gs_sampler *s, uint64_t *state)
{
    if (!s || !state) return GS_ERR_INVALID;
    *state = s->state;
    return GS_OK;
}

int gs_sampler_set_state(gs_sampler *s, uint64_t state)
{
    if (!s) return GS_ERR_INVALID;
    s->state = state;
    return GS_OK;
}

int gs_sampler_reserve(gs_sampler *s, size_t B, size_t V)
{
    if (!s || V > GS_MAX_VOCAB) return GS_ERR_INVALID;
    if (V > gs::kRegMaxV) {               // rows the split or chunked top-k paths may take, any k
        const size_t rows = B < (size_t)gs::kSplitMaxRows ? B : (size_t)gs::kSplitMaxRows;
        size_t need = split_bytes(rows ? rows : 1, gs::kSplitMaxWidth);
        if (gs::chunk_path_ok(V) && chunk_bytes(B, V) > need) need = chunk_bytes(B, V);
        int rc = grow(s, &s->split, &s->split_cap, need);
        if (rc) return rc;
    }
    return reserve_scratch(s, B, V);
}

int gs_sample(gs_sampler *s, const float *logits, size_t V, const uint32_t *recent, size_t W,
              uint32_t *out_token)
{
    if (!s || !out_token || (V > 0 && !logits) || (W > 0 && !recent)) return GS_ERR_INVALID;
    s->fb_rows = 0;
    if (V > GS_MAX_VOCAB) return GS_ERR_UNSUPPORTED;
    if (W > (size_t)gs::kMaxWindow) return GS_ERR_UNSUPPORTED;
    int rc;
    const float *d_logits = logits;
    if (V > 0 && !is_device_ptr(s, logits)) {
        void *p = s->d_row;
        rc = grow(s, &p, &s->row_cap, V * sizeof(float));
        s->d_row = (float *)p;
        if (rc) return rc;
        if (hipMemcpyAsync(s->d_row, logits, V * sizeof(float), hipMemcpyHostToDevice, s->stream) != hipSuccess)
            return GS_ERR_HIP;
        d_logits = s->d_row;
    }
    // A host window (the reference's &[u32]) is copied into mapped pinned
    // memory; the kernel reads it there.  The previous call's kernel has
    // finished (every call waits for its result), so the buffer is free.
    const uint32_t *d_rec = recent;
    const bool host_win = W > 0 && !is_device_ptr(s, recent);
    if (host_win) {
        memcpy(s->h_rec, recent, W * sizeof(uint32_t));
        d_rec = s->d_rec_map;
    }
    if (needs_full_path(s->params, V) && (rc = reserve_scratch(s, 1, V))) return rc;
    gs::RowArgs a;
    memset(&a, 0, sizeof(a));
    a.logits = d_logits ? d_logits : s->d_row;
    a.ld = V;
    a.V = (int)V;
    a.params = nullptr;
    a.uparams = s->params;
    a.recent = W ? d_rec : nullptr;
    a.ld_recent = W;
    a.recent_len = nullptr;
    a.W = (int)W;
    a.u = nullptr;
    a.lcg_state = s->state;
    a.tokens = s->d_tok_map;
    a.status = s->d_status_map;
    a.scratch = s->scratch;
    a.scratch_stride = gs::scratch_u32_per_row(V);
    a.fb = s->fb;
    if (host_win && W <= (size_t)gs::kKernWin) {
        // a short host window also travels in the kernel arguments: the
        // register path reads it there instead of across the bus
        memcpy(a.kwin, recent, W * sizeof(uint32_t));
        a.kwin_n = (int)W;
    }
    const bool full = needs_full_path(s->params, V);
    int st;
    uint32_t tok;
    if (full) {
        // the full-vocabulary path (several kernels) synchronises the stream
        s->fb_rows = 1;
        s->fb_last = s->fb;
        if (gs::launch_sample_rows(a, 1, s->stream) != hipSuccess) return GS_ERR_HIP;
        if (hipStreamSynchronize(s->stream) != hipSuccess) return GS_ERR_HIP;
        st = *(volatile int32_t *)s->h_status;
        tok = *(volatile uint32_t *)s->h_tok;
    } else {
        // One small-path kernel signals completion through the mapped word,
        // which the host polls instead of synchronising the stream.  Rows
        // that fit in registers take the dedicated kernel; the rare row it
        // cannot finish is run again by the general one.
        a.done = s->d_done_map;
        bool reg = gs::reg_row_fits(s->params, V, a.logits);
        const bool split = !reg && gs::split_fits(s->params, V) &&
                           reserve_split(s, 1, gs::split_width(s->params, V)) == GS_OK;
        for (;;) {
            a.done_val = ++s->seq;
            const hipError_t le = reg     ? gs::launch_reg_row(a, s->stream)
                                  : split ? launch_split_rows(s->split, a, 1, gs::split_width(s->params, V), s->stream)
                                          : gs::launch_sample_rows(a, 1, s->stream);
            if (le != hipSuccess) return GS_ERR_HIP;
            volatile uint64_t *f = s->h_done;
            uint64_t w = *f;
            for (uint32_t spins = 0; (uint32_t)(w >> 32) != s->seq; spins++) {
                if (spins > (1u << 22)) {           // slow call: wait through the runtime
                    if (hipStreamSynchronize(s->stream) != hipSuccess) return GS_ERR_HIP;
                    w = *f;
                    if ((uint32_t)(w >> 32) != s->seq) return GS_ERR_HIP;
                    break;
                }
                __builtin_ia32_pause();
                w = *f;
            }
            st = (int)(int8_t)(uint8_t)(w >> 24);
            tok = (uint32_t)w & 0xffffffu;
            if (!(reg && st == gs::kStatusRetryHost)) break;
            reg = false;
        }
    }
    if (s->params.temperature > 0.0f) s->state = gs::lcg_jump(s->state, 1);   // one draw iff T > 0
    if (st != GS_OK) return st;
    *out_token = tok;
    return GS_OK;
}

int gs_sample_mut(gs_sampler *s, float *logits, size_t V, const uint32_t *recent, size_t W, uint32_t *out_token)
{
    int rc = gs_sample(s, logits, V, recent, W, out_token);
    if (rc != GS_OK || V == 0) return rc;
    // gs_sample left the row on the device (the caller's buffer or the
    // staging copy) and a host window in the mapped buffer
    const bool dev_row = is_device_ptr(s, logits);
    float *d_row = dev_row ? logits : s->d_row;
    const uint32_t *d_rec = (W > 0 && !is_device_ptr(s, recent)) ? s->d_rec_map : recent;
    if (gs::launch_writeback(d_row, 1, (int)V, V, nullptr, s->params, W ? d_rec : nullptr, W, nullptr, (int)W,
                             s->stream) != hipSuccess)
        return GS_ERR_HIP;
    if (!dev_row &&
        hipMemcpyAsync(logits, d_row, V * sizeof(float), hipMemcpyDeviceToHost, s->stream) != hipSuccess)
        return GS_ERR_HIP;
    return hipStreamSynchronize(s->stream) == hipSuccess ? GS_OK : GS_ERR_HIP;
}

int gs_sample_detail(gs_sampler *s, const float *d_logits, size_t B, size_t V, size_t ld, const gs_params *d_params,
                     const uint32_t *d_recent, size_t ld_recent, const uint32_t *d_recent_len, size_t W,
                     const float *d_u, uint32_t *d_tokens, int32_t *d_status, const gs_detail *det, void *stream)
{
    if (!s || !d_tokens || !det || (B > 0 && V > 0 && !d_logits) || ld < V) return GS_ERR_INVALID;
    if (d_recent && ld_recent < W) return GS_ERR_INVALID;
    if (!d_u && d_params) return GS_ERR_INVALID;
    if ((det->ids || det->p) && det->cap == 0) return GS_ERR_INVALID;
    if (V > GS_MAX_VOCAB || B > 0x7fffffff) return GS_ERR_UNSUPPORTED;
    if (d_recent && W > (size_t)gs::kMaxWindow) return GS_ERR_UNSUPPORTED;
    s->fb_rows = 0;
    if (B == 0) return GS_OK;
    int rc;
    bool cap = false;
    if ((rc = capturing((hipStream_t)stream, &cap))) return rc;
    if (cap) return GS_ERR_UNSUPPORTED;   // a diagnostic: not for graphs
    if ((rc = reserve_scratch(s, B, V))) return rc;
    gs::RowArgs a;
    memset(&a, 0, sizeof(a));
    a.logits = d_logits;
    a.ld = ld;
    a.V = (int)V;
    a.params = d_params;
    a.uparams = s->params;
    a.recent = d_recent;
    a.ld_recent = ld_recent;
    a.recent_len = d_recent_len;
    a.W = d_recent ? (int)W : 0;
    a.u = d_u;
    a.lcg_state = s->state;
    a.tokens = d_tokens;
    a.status = d_status;
    a.scratch = s->scratch;
    a.scratch_stride = gs::scratch_u32_per_row(V);
    a.det = *det;
    if (gs::launch_detail_rows(a, (int)B, (hipStream_t)stream) != hipSuccess) return GS_ERR_HIP;
    if (!d_u && s->params.temperature > 0.0f) s->state = gs::lcg_jump(s->state, B);
    return GS_OK;
}

int gs_logits_writeback(gs_sampler *s, float *d_logits, size_t B, size_t V, size_t ld, const gs_params *d_params,
                        const uint32_t *d_recent, size_t ld_recent, const uint32_t *d_recent_len, size_t W,
                        void *stream)
{
    if (!s || (B > 0 && V > 0 && !d_logits) || ld < V) return GS_ERR_INVALID;
    if (d_recent && ld_recent < W) return GS_ERR_INVALID;
    if (V > GS_MAX_VOCAB || B > 65535) return GS_ERR_UNSUPPORTED;
    if (B == 0 || V == 0) return GS_OK;
    return gs::launch_writeback(d_logits, (int)B, (int)V, ld, d_params, s->params, d_recent, ld_recent,
                                d_recent_len, d_recent ? (int)W : 0, (hipStream_t)stream) == hipSuccess
               ? GS_OK : GS_ERR_HIP;
}

int gs_sample_batch(gs_sampler *s, const float *d_logits, size_t B, size_t V, size_t ld,
                    const gs_params *d_params, const uint32_t *d_recent, size_t ld_recent,
                    const uint32_t *d_recent_len, size_t W, const float *d_u,
                    uint32_t *d_tokens, int32_t *d_status, void *stream)
{
    return gs::sample_batch(s, d_logits, B, V, ld, d_params, d_recent, ld_recent, d_recent_len, W, d_u, d_tokens,
                            d_status, nullptr, stream);
}

} // extern "C"

namespace gs {

namespace {

// Device buffers of one batched call.  `fixed` buffers come from the caller
// (the static scratch of gs_sample_batch_noalloc) and never grow.
struct CallBufs {
    bool fixed;
    uint32_t *scratch;           // full-vocabulary path, B * scratch_u32_per_row(V) words
    int32_t *fb;                 // B fallback flags
    void *split;                 // split top-k path
    size_t split_cap;            // bytes
};

} // namespace

int sample_batch_bufs(gs_sampler *s, const float *d_logits, size_t B, size_t V, size_t ld, const gs_params *d_params,
                      const uint32_t *d_recent, size_t ld_recent, const uint32_t *d_recent_len, size_t W,
                      const float *d_u, uint32_t *d_tokens, int32_t *d_status, const DecodeHook *hook,
                      void *stream, const CallBufs *fixed)
{
    if (!s || !d_tokens || (B > 0 && V > 0 && !d_logits) || ld < V) return GS_ERR_INVALID;
    s->fb_rows = 0;
    if (d_recent && ld_recent < W) return GS_ERR_INVALID;
    if (!d_u && d_params) return GS_ERR_INVALID;   // LCG draws need host-known T per row
    if (V > GS_MAX_VOCAB || B > 0x7fffffff) return GS_ERR_UNSUPPORTED;
    if (d_recent && W > (size_t)gs::kMaxWindow) return GS_ERR_UNSUPPORTED;
    if (B == 0) return GS_OK;
    int rc;
    bool cap = false;
    if ((rc = capturing((hipStream_t)stream, &cap))) return rc;
    // The sampler's own LCG is host state: a graph would replay the draws it
    // held at capture time, so under capture the draws must come from d_u.
    if (cap && !d_u && s->params.temperature > 0.0f) return GS_ERR_UNSUPPORTED;
    if (cap) s->captured = true;
    const bool full = d_params || needs_full_path(s->params, V);
    CallBufs bf;
    if (fixed) {
        bf = *fixed;
    } else {
        if (full && (s->fb_cap < B * sizeof(int32_t) ||
                     s->scratch_elems < B * gs::scratch_u32_per_row(V))) {
            if (cap) return GS_ERR_UNSUPPORTED;      // no allocation under capture: reserve first
            if ((rc = reserve_scratch(s, B, V))) return rc;
        }
        bf = CallBufs{false, s->scratch, s->fb, s->split, s->split_cap};
    }
    gs::RowArgs a;
    memset(&a, 0, sizeof(a));
    a.logits = d_logits;
    a.ld = ld;
    a.V = (int)V;
    a.params = d_params;
    a.uparams = s->params;
    a.recent = d_recent;
    a.ld_recent = ld_recent;
    a.recent_len = d_recent_len;
    a.W = d_recent ? (int)W : 0;
    a.u = d_u;
    a.lcg_state = s->state;
    a.tokens = d_tokens;
    a.status = d_status;
    a.scratch = bf.scratch;
    a.scratch_stride = gs::scratch_u32_per_row(V);
    a.fb = bf.fb;
    if (hook) a.hook = *hook;
    // top-k rows of a large vocabulary in a batch with fewer rows than CUs:
    // chunks of up to 32768 logits, one workgroup each (per-row params: the
    // kernels pick the rows).  With B >= #CUs one workgroup per row already
    // fills the chip, and leaves the CUs that a batch's full-vocabulary rows
    // do not use to its top-k rows.  Float4-aligned rows take the one-launch
    // form (measured on MI355X faster than the split path at every B).
    const bool chunk_ok = gs::chunk_path_ok(V) && B < (size_t)num_cus(s) &&
                          (d_params || gs::chunk_fits(s->params, V));
    const bool self = chunk_ok && B <= (size_t)gs::kCSyncRows && (V & 3) == 0 && (ld & 3) == 0 &&
                      ((uintptr_t)d_logits & 15u) == 0 && gs::chunk_stride(V) <= gs::kChunkSelfMaxN;
    // otherwise, measured on MI355X: the split path (1024-logit chunks)
    // beats the two-launch chunked path up to about 2000 chunks per call
    // (V = 152064: B <= 8; V = 128256: B <= 16; V = 256000: B <= 4)
    bool split = !self && !d_params && B <= (size_t)gs::kSplitMaxRows &&
                 B * (V / gs::kSplitL) <= gs::kSplitMaxChunks && gs::split_fits(s->params, V);
    const size_t wd = split ? gs::split_width(s->params, V) : 0;
    if (split && bf.split_cap < split_bytes(B, wd)) {
        // the buffers must grow: not with fixed buffers or under stream
        // capture (no allocation there); the rows then take the
        // one-workgroup-per-row path instead
        if (bf.fixed || cap) split = false;
        else if ((rc = reserve_split(s, B, wd))) return rc;
        else bf.split = s->split;
    }
    bool chunked = !split && chunk_ok;
    if (chunked && bf.split_cap < chunk_bytes(B, V)) {
        if (bf.fixed || cap) chunked = false;
        else if ((rc = grow(s, &s->split, &s->split_cap, chunk_bytes(B, V)))) return rc;
        else { bf.split = s->split; bf.split_cap = s->split_cap; }
    }
    if (split) {
        // a few rows of a large vocabulary: spread each row over the chip
        if (launch_split_rows(bf.split, a, B, wd, (hipStream_t)stream) != hipSuccess) return GS_ERR_HIP;
    } else {
        if (full) { s->fb_rows = B; s->fb_last = bf.fb; }
        else a.fb = nullptr;            // no full-vocabulary row: the flags are not written
        const hipStream_t st = (hipStream_t)stream;
        const hipError_t le =
            chunked ? gs::launch_chunked(a, (int)B, (float *)bf.split,
                                         (uint32_t *)((float *)bf.split + B * gs::chunk_stride(V)),
                                         self ? s->csync : nullptr, st)
            : d_params ? gs::launch_sample_rows_forked(a, (int)B, st, s->side, s->ev_fork, s->ev_join)
                       : gs::launch_sample_rows(a, (int)B, st);
        if (le != hipSuccess) return GS_ERR_HIP;
    }
    if (!d_u && s->params.temperature > 0.0f) s->state = gs::lcg_jump(s->state, B);
    return GS_OK;
}

int sample_batch(gs_sampler *s, const float *d_logits, size_t B, size_t V, size_t ld, const gs_params *d_params,
                 const uint32_t *d_recent, size_t ld_recent, const uint32_t *d_recent_len, size_t W,
                 const float *d_u, uint32_t *d_tokens, int32_t *d_status, const DecodeHook *hook, void *stream)
{
    return sample_batch_bufs(s, d_logits, B, V, ld, d_params, d_recent, ld_recent, d_recent_len, W, d_u, d_tokens,
                             d_status, hook, stream, nullptr);
}

// ---- the scratch of gs_sample_batch_noalloc --------------------------------
// One array per GPU, in the code object: the library holds it until the
// process ends.  Host code never uses the symbol's name as an address (that
// is a host-side stand-in); it uses the device address resolved per device
// by hipGetSymbolAddress.
constexpr size_t kStaticScratchBytes = (size_t)GS_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint32_t scratch[kStaticScratchBytes / sizeof(uint32_t)];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices];

// The device address of `scratch` on `device` (made current by the caller).
int static_scratch(int device, void **out)
{
    if (device < 0 || device >= kMaxDevices) return GS_ERR_UNSUPPORTED;
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    if (!g_scratch_ptr[device]) {
        void *ptr = nullptr;
        if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) != hipSuccess || !ptr) {
            (void)hipGetLastError();
            return GS_ERR_HIP;
        }
        g_scratch_ptr[device] = ptr;
    }
    *out = g_scratch_ptr[device];
    return GS_OK;
}

size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }
} // namespace

// Resolve the static scratch of the current device (sampler set-up).
int init_static_scratch(int device)
{
    void *p;
    return static_scratch(device, &p);
}

} // namespace gs

extern "C" {

int gs_sample_batch_noalloc(gs_sampler *s, const float *d_logits, size_t B, size_t V, size_t ld,
                            const gs_params *d_params, const uint32_t *d_recent, size_t ld_recent,
                            const uint32_t *d_recent_len, size_t W, const float *d_u,
                            uint32_t *d_tokens, int32_t *d_status, void *stream)
{
    if (!s) return GS_ERR_INVALID;
    if (V > GS_MAX_VOCAB || B > 0x7fffffff) return GS_ERR_UNSUPPORTED;
    void *base = nullptr;
    int rc = gs::static_scratch(s->device, &base);
    if (rc) return rc;
    // layout: B fallback flags | split top-k buffers (any k, up to
    // kSplitMaxRows rows) | full-vocabulary scratch
    // Only the buffers of the paths this call can take are counted: the
    // full-vocabulary scratch when some row may take that path, the chunked
    // top-k buffers when the batch has fewer rows than CUs, the split
    // buffers for a few rows with uniform params.  (A path whose buffer is
    // not given is not taken: sample_batch_bufs falls back to one workgroup
    // per row for top-k rows.)
    const bool full = d_params || needs_full_path(s->params, V);
    const size_t fb_bytes = gs::align256((B ? B : 1) * sizeof(int32_t));
    size_t sp_need = 0;
    if (V > gs::kRegMaxV) {
        if (!d_params && B <= (size_t)gs::kSplitMaxRows && gs::split_fits(s->params, V))
            sp_need = split_bytes(B, gs::split_width(s->params, V));
        if (gs::chunk_path_ok(V) && B < (size_t)num_cus(s) && chunk_bytes(B, V) > sp_need)
            sp_need = chunk_bytes(B, V);
    }
    const size_t sp_bytes = gs::align256(sp_need);
    const size_t full_bytes = full ? B * gs::scratch_u32_per_row(V) * sizeof(uint32_t) : 0;
    if (fb_bytes + sp_bytes + full_bytes > gs::kStaticScratchBytes) return GS_ERR_UNSUPPORTED;
    char *p = (char *)base;
    gs::CallBufs bf{true, full_bytes ? (uint32_t *)(p + fb_bytes + sp_bytes) : nullptr, (int32_t *)p,
                    sp_bytes ? p + fb_bytes : nullptr, sp_bytes};
    return gs::sample_batch_bufs(s, d_logits, B, V, ld, d_params, d_recent, ld_recent, d_recent_len, W, d_u,
                                 d_tokens, d_status, nullptr, stream, &bf);
}

int gs_window_push(uint32_t *d_window, size_t B, size_t ld, size_t W, size_t pos,
                   const uint32_t *d_tokens, void *stream)
{
    if (!d_window || !d_tokens || W == 0 || ld < W || B > 0x7fffffff) return GS_ERR_INVALID;
    if (B == 0) return GS_OK;
    return gs::launch_window_push(d_window, (int)B, ld, (int)W, pos, d_tokens, (hipStream_t)stream) == hipSuccess
               ? GS_OK : GS_ERR_HIP;
}

int gs_synth_logits(float *d_out, size_t B, size_t V, size_t ld, uint64_t seed, uint64_t counter0,
                    float sigma, void *stream)
{
    if (!d_out || ld < V || B > 0x7fffffff || V > 0x7fffffff) return GS_ERR_INVALID;
    if (B == 0 || V == 0) return GS_OK;
    return gs::launch_synth(d_out, (int)B, (int)V, ld, seed, counter0, sigma, (hipStream_t)stream) == hipSuccess
               ? GS_OK : GS_ERR_HIP;
}

int gs_limits(uint32_t *max_vocab, uint32_t *max_window)
{
    if (max_vocab) *max_vocab = GS_MAX_VOCAB;
    if (max_window) *max_window = (uint32_t)gs::kMaxWindow;
    return GS_OK;
}

const char *gs_version(void) { return "gs_sampler 0.1 gfx950"; }

} // extern "C"
