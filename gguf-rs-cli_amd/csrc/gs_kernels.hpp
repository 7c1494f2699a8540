// gs_kernels.hpp -- launch interface between the C ABI and the kernels.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "../../include/gs_sampler.h"
#include "gs_decode_dev.hpp"

namespace gs {

constexpr int kMaxWindow = 1024;   // unique penalized ids held in the LDS hash
constexpr int kMaxTopK = 1024;     // largest k served by the LDS top-k path
constexpr int kKernWin = 64;       // host windows up to this length travel in the kernel arguments

struct RowArgs {
    const float *logits;
    size_t ld;
    int V;
    const gs_params *params;       // per row, or null
    gs_params uparams;             // used when params == null
    const uint32_t *recent;
    size_t ld_recent;
    const uint32_t *recent_len;
    int W;
    const float *u;                // per-row draws, or null
    uint64_t lcg_state;            // used when u == null: row b draws jump(state, b)
    uint32_t *tokens;
    int32_t *status;
    int32_t *fb;                   // per row: 1 = the increment histogram failed, a fallback form finished the row
    uint32_t *scratch;             // full-vocabulary paths: scratch_stride u32 per row
    size_t scratch_stride;         // u32 elements per row
    uint64_t *done;                // optional (single-row calls, B = 1): receives
    uint32_t done_val;             // (done_val << 32) | (status & 0xff) << 24 | token in one store,
                                   // instead of tokens/status, for host polling
    DecodeHook hook;               // decode step: the kernel that stores a row's token commits it
    int kwin_n;                    // single-row calls: a host window of W <= kKernWin ids passed
    uint32_t kwin[kKernWin];       // by value here (used instead of `recent` when kwin_n != 0)
    gs_detail det;                 // diagnostic outputs of the detail kernel (gs_sample_detail)
    int chunked;                   // rows with chunk_row() true are sampled by the chunked top-k path
                                   // (kChunkedX / kChunkedSelf / kChunkedY):
    const float *cvrow;            // its virtual rows (values, ids), stride cvld, cnch chunks
    const uint32_t *cvidx;
    size_t cvld;
    int cnch;
    uint32_t *csync;               // kChunkedSelf: per row, chunks done and a fallback flag (zero
                                   // between calls: the finishing block clears them)
};

// How the row kernels treat rows with chunk_row() true.
constexpr int kChunkedX = 1;       // sample the virtual row of penalized logits (chunk_topk_kernel)
constexpr int kChunkedSelf = 2;    // skip: chunk_rows_kernel samples them
constexpr int kChunkedY = 3;       // sample the virtual row of scaled logits (chunk_rows_kernel)
constexpr int kCSyncRows = 1024;   // rows of the csync buffer (2 words each)
constexpr size_t kChunkSelfMaxN = 2048;   // widest virtual row (chunk_stride) of the one-launch path

// Per-row scratch (u32 units) of the full-vocabulary paths: the sort path
// needs 4V; the exact path its element list and walk items (each V plus
// room for the overflow, the bins and penalized values, in u64) and its
// deferred ids.
// The increment-histogram path (gs_full3.hpp) lists at most f3_list_cap(V)
// entries per pass; its scratch (u64 words): the unsorted list, the two
// sorted lists, their summands (two f32 arrays), the ambiguous and deferred
// entries and two per-bin tables.
constexpr size_t kF3AmbCap = 4096;
constexpr size_t kF3DefCap = 8192;
__host__ __device__ inline size_t f3_list_cap(size_t V) { return ((V < 65536 ? V : 65536) + 256 + 2 * 2048 + 1) & ~(size_t)1; }
__host__ __device__ inline size_t f3_scratch_u64(size_t V) { return 4 * f3_list_cap(V) + kF3AmbCap + kF3DefCap + 4096; }
inline size_t scratch_u32_per_row(size_t V)
{
    const size_t v2 = 6 * V + 2 * (3 * 256 + 2 * 4096 + 6 * 2048) + 16384;
    const size_t v3 = 2 * f3_scratch_u64(V);
    return v2 > v3 ? v2 : v3;
}

// The row kernels of a batch: the small-path rows (and, when a.chunked is
// set, the chunked rows' virtual rows), then the full-vocabulary rows by the
// increment-histogram path and, for rows whose checks failed, by its
// fallback forms in the same workgroup.
hipError_t launch_sample_rows(const RowArgs &a, int B, hipStream_t st);
// The same for a batch with per-row params (rows of both kinds): the small
// rows run on `side` beside the full-vocabulary rows on st (fork / join by
// the two events, so graph capture records the same dependencies).
hipError_t launch_sample_rows_forked(const RowArgs &a, int B, hipStream_t st, hipStream_t side, hipEvent_t fork,
                                    hipEvent_t join);
// Every row sorted (diagnostic; fills a.det); scratch as the sort path.
hipError_t launch_detail_rows(const RowArgs &a, int B, hipStream_t st);
// Single-row register path (B = 1); rows it cannot finish report kStatusRetryHost.
constexpr int kStatusRetryHost = 0x7f;
bool reg_row_fits(const gs_params &p, size_t V, const void *row);
hipError_t launch_reg_row(const RowArgs &a, hipStream_t st);
// Split top-k path for a few rows of a large vocabulary: pass 1 spreads each
// row over V / kSplitL workgroups, each keeping its chunk's best kp =
// round_up(k, 4) elements (penalized) in index order in a virtual row of
// split_width(p, V) entries; pass 2 samples the virtual rows and maps the
// token back.
constexpr size_t kRegMaxV = 32768;   // widest row the register kernel holds (1024 threads x 8 float4)
constexpr int kSplitL = 1024;          // elements per chunk; the last chunk takes the rest (< 2 kSplitL)
constexpr int kSplitMaxKp = 128;
constexpr int kSplitMaxRows = 32;      // more rows fill the chip one workgroup per row
constexpr size_t kSplitMaxChunks = 2000; // B * V / kSplitL above this: the chunked path is faster
constexpr size_t kSplitMaxWidth = 32768;
bool split_fits(const gs_params &p, size_t V);
// Chunked top-k path for batches: rows with V > kRegMaxV, finite T > 0 and
// 0 < k <= kChunkMaxK (checked per row on the device, so per-row params
// work) are cut into nch = chunk_count(V) balanced chunks of at most
// kChunkL logits; each chunk keeps its best kp = round_up(k, 4) in a virtual
// row of stride chunk_stride(V), one 1024-thread workgroup per chunk.  With
// csync (rows of V % 4 == 0, 16-byte aligned) that launch also samples the
// row -- its last chunk to finish does -- and with per-row params the row
// kernels then take the batch's other rows; without it (chunk_topk_kernel)
// one launch of the row kernels samples the virtual rows and every other
// row of the batch.
constexpr int kChunkL = 32768;
constexpr uint32_t kChunkMaxK = 128;
inline int chunk_count(size_t V) { return (int)((V + kChunkL - 1) / kChunkL); }
inline size_t chunk_stride(size_t V) { return (size_t)chunk_count(V) * kChunkMaxK; }
inline bool chunk_path_ok(size_t V) { return V > kRegMaxV && chunk_stride(V) <= kSplitMaxWidth; }
hipError_t launch_chunked(RowArgs a, int B, float *vrow, uint32_t *vidx, uint32_t *csync, hipStream_t st);
inline bool chunk_fits(const gs_params &p, size_t V)
{
    return p.temperature > 0.0f && p.temperature < INFINITY && p.top_k > 0 && (size_t)p.top_k < V &&
           p.top_k <= kChunkMaxK;
}
size_t split_width(const gs_params &p, size_t V);
hipError_t launch_split(const RowArgs &a, int B, float *vrow, uint32_t *vidx, hipStream_t st);
// gs_sample_batch with an optional decode hook (the sampler's last kernel
// commits each row into it).
int sample_batch(gs_sampler *s, const float *d_logits, size_t B, size_t V, size_t ld, const gs_params *d_params,
                 const uint32_t *d_recent, size_t ld_recent, const uint32_t *d_recent_len, size_t W,
                 const float *d_u, uint32_t *d_tokens, int32_t *d_status, const DecodeHook *hook, void *stream);
hipError_t launch_window_push(uint32_t *win, int B, size_t ld, int W, size_t pos,
                              const uint32_t *tok, hipStream_t st);
// The caller-visible mutation of src/sampler.rs:37,41 (penalty, then / T when T > 0).
hipError_t launch_writeback(float *logits, int B, int V, size_t ld, const gs_params *params, const gs_params &up,
                           const uint32_t *recent, size_t ld_recent, const uint32_t *recent_len, int W,
                           hipStream_t st);
hipError_t launch_synth(float *out, int B, int V, size_t ld, uint64_t seed, uint64_t c0,
                        float sigma, hipStream_t st);

} // namespace gs
