// gs_kernels.hip -- gfx950 kernels of the token sampler.
//
// One workgroup (1024 threads, 16 wave64) owns one logit row.  Per row:
//   1. penalty table  : the recent window folded into an LDS hash of
//                       (id -> penalized logit), src/sampler.rs:23-30
//   2. T <= 0         : greedy argmax, last maximal index (src/sampler.rs:15-19)
//   3. 0 < k < V, k <= kMaxTopK : radix select of the top-k keys with LDS
//                       histograms, bitonic sort of the survivors in LDS, then
//                       softmax / nucleus / draw (src/sampler.rs:44-78)
//   4. otherwise      : exact full-vocabulary path: stable LSD radix sort of
//                       (key, index) in per-row scratch, then the same
//                       softmax / nucleus / draw over the sorted row.
// All sequential f32 sums of the reference are evaluated exactly by
// block_seqsum (see gs_block.hpp).
#include <type_traits>

#include "gs_block.hpp"
#include "gs_kernels.hpp"
#include "gs_full_smem.hpp"
#include "gs_select.hpp"

namespace gs {

#ifdef GS_TIMING
// Stage timestamps of row 0 (development builds only).
__device__ uint64_t g_stamp[32];
__device__ int g_fails[1280];
__constant__ unsigned g_row;   // scalar loads: a stamp adds no memory wait
__device__ uint32_t g_stages[256 * 32];   // per row: realtime at each stamp (mode 1)
#define GS_STAMP(i) do { if (threadIdx.x == 0) { const uint64_t _t = __builtin_amdgcn_s_memrealtime(); if (blockIdx.x == g_row) g_stamp[i] = _t; if (blockIdx.x < 256 && (i) >= 8 && (i) < 24) g_stages[blockIdx.x * 32 + (i)] = (uint32_t)_t; } } while (0)
#define GS_DIAG(i, v) do { if (blockIdx.x == g_row && threadIdx.x == 0) g_stamp[i] = (uint64_t)(v); } while (0)
#define GS_SUB0(i) do { if (threadIdx.x == 0 && blockIdx.x == g_row) g_stamp[16 + (i)] = __builtin_amdgcn_s_memrealtime(); } while (0)
#define GS_SUB(i) do { if (blockIdx.x == g_row && threadIdx.x == 0 && g_fails[899] < 1) g_fails[900 + (i)] = (int)__builtin_amdgcn_s_memrealtime(); } while (0)
#else
#define GS_STAMP(i) do { } while (0)
#define GS_DIAG(i, v) do { } while (0)
#define GS_SUB(i) do { } while (0)
#define GS_SUB0(i) do { } while (0)
#endif

constexpr int kHashSlots = 2 * kMaxWindow;     // open addressing, load <= 1/2
constexpr int kHistBins = 4096;                 // 12-bit radix digits
constexpr int kCandCap = 2048;                  // LDS candidate capacity
constexpr uint32_t kEmpty = 0xffffffffu;
constexpr int kPenBitsWords = 8192;             // bitmap of ids < 262144 (the register and streamed rows)
constexpr int kPenBitsTable = 1024;             // the part build_penalty keeps (ids < 32768)

struct TopkSmem {
    union alignas(16) {
        uint32_t hist[kHistBins];
        uint32_t wcnt[kWaves * 256];            // radix sort: per-wave digit counts
        float ev[kHistBins];
    } u;
    alignas(16) uint64_t cand[kCandCap];        // (key << 32) | ~idx, sorted descending
    uint32_t base[256];
    uint32_t hraw[kHashSlots];                  // raw logit of each penalized id (table build only)
    uint32_t pbits[kPenBitsWords];              // penalized-id bitmap, ids < 32 * kPenBitsWords
};

struct RowSmem {
    uint32_t hkey[kHashSlots];                  // penalized ids
    uint32_t hval[kHashSlots];                  // occurrence count, then f32 bits of the penalized logit
    SeqSmem seq;
    int ncand;
    int nuniq;
    int flag_nan;
    uint32_t sel_prefix;
    uint32_t sel_above;
    uint32_t red_u32[kWaves];
    float red_f32[kWaves];
    int red_i32[kWaves];
    double red_f64[kWaves];
    double red_f64b[kWaves];      // a second buffer for scans that run back to back
    alignas(16) float fin[256];                 // finish_wave: the values being accumulated
    int tok;
    int flag_snan;                              // a NaN in the streamed part of a row (topk_row_reg)
    uint32_t reg_sel;                           // topk_row_reg: the bound's histogram bin
    union {
        TopkSmem tk;
        FullSmem fs;
        Full3Smem f3;
    } x;
    int clast;                                  // chunk_rows_kernel: this block finishes the row
};

// --------------------------------------------------------------------------
__device__ __forceinline__ uint32_t hash_slot(uint32_t id) { return (id * 2654435761u) >> (32 - 11); }
static_assert(kHashSlots == 2048, "hash_slot assumes 2048 slots");

// Returns the slot of id, or -1.
__device__ __forceinline__ int hash_find(const RowSmem &sm, uint32_t id)
{
    uint32_t h = hash_slot(id);
    for (int n = 0; n < kHashSlots; n++) {
        uint32_t k = sm.hkey[h];
        if (k == id) return (int)h;
        if (k == kEmpty) return -1;
        h = (h + 1) & (kHashSlots - 1);
    }
    return -1;
}

// The recent window's loads, issued before the penalty table is built so
// that both dependent loads overlap the row loads: thread j takes recent[j]
// (W <= kMaxWindow == kThreads) and the raw logit of that id.  Ids outside
// [0, V) are skipped, as logits.get_mut does at src/sampler.rs:26.
struct PenLoad { uint32_t id; float raw; };
static_assert(kMaxWindow <= kThreads, "one window entry per thread");
__device__ __forceinline__ PenLoad pen_load(const float *row, int V, const uint32_t *rec, int W, bool with_raw)
{
    PenLoad p{kEmpty, 0.0f};
    const int t = threadIdx.x;
    if (t < W) {
        const uint32_t id = ldg(rec + t);
        if (id < (uint32_t)V) { p.id = id; if (with_raw) p.raw = ldg(row + id); }
    }
    return p;
}

// Build the penalty table for this row (src/sampler.rs:23-30): an LDS hash of
// id -> penalized logit, the occurrence count applied one op at a time, and
// a bitmap of the penalized ids below 32 * kPenBitsTable.  sm.nuniq receives
// the number of distinct ids.
__device__ void build_penalty(RowSmem &sm, PenLoad pl, float T, float pen)
{
    const int t = threadIdx.x;
    for (int i = t; i < kHashSlots; i += kThreads) { sm.hkey[i] = kEmpty; sm.hval[i] = 0; }
    for (int i = t; i < kPenBitsTable; i += kThreads) sm.x.tk.pbits[i] = 0u;
    if (t == 0) sm.nuniq = 0;
    __syncthreads();
    if (pl.id != kEmpty) {
        const uint32_t id = pl.id;
        uint32_t h = hash_slot(id);
        for (;;) {
            const uint32_t prev = atomicCAS(&sm.hkey[h], kEmpty, id);
            if (prev == kEmpty || prev == id) {
                if (prev == kEmpty) atomicAdd(&sm.nuniq, 1);
                atomicAdd(&sm.hval[h], 1u);
                sm.x.tk.hraw[h] = __float_as_uint(pl.raw);   // every writer stores the same value
                break;
            }
            h = (h + 1) & (kHashSlots - 1);
        }
        if (id < 32u * kPenBitsTable) atomicOr(&sm.x.tk.pbits[id >> 5], 1u << (id & 31u));
    }
    __syncthreads();
    for (int i = t; i < kHashSlots; i += kThreads) {
        const uint32_t id = sm.hkey[i];
        if (id != kEmpty) {
            const float l = penalize(__uint_as_float(sm.x.tk.hraw[i]), sm.hval[i], pen);
            sm.hval[i] = __float_as_uint(l);
            if (isnan(l / T)) sm.flag_nan = 1;
        }
    }
    __syncthreads();
}

// Effective scaled logit of element i given its raw value.
__device__ __forceinline__ float eff_scaled(const RowSmem &sm, bool has_pen, uint32_t i, float x, float T)
{
    if (has_pen) {
        int s = hash_find(sm, i);
        if (s >= 0) x = __uint_as_float(sm.hval[s]);
    }
    return x / T;
}

// --------------------------------------------------------------------------
// Block reductions.
__device__ int block_or(int v, RowSmem &sm)
{
    v = __any(v) ? 1 : 0;
    if (lane_id() == 0) sm.red_i32[wave_id()] = v;
    __syncthreads();
    int r = 0;
    for (int i = 0; i < kWaves; i++) r |= sm.red_i32[i];
    __syncthreads();
    return r;
}

// --------------------------------------------------------------------------
// Visit every element of a row once, f(index, value).  With a 16-byte
// aligned row the loads are float4 and kUnroll of them are in flight per
// thread before any is consumed (a row is 1024*16*kUnroll bytes per round).
constexpr int kUnroll = 4;
template <bool NT = false, class F>
__device__ __forceinline__ void row_for_each(const float *row, int V, bool aligned, F f)
{
    const int t = threadIdx.x;
    if (aligned) {
        const float4 *r4 = reinterpret_cast<const float4 *>(row);
        const int n4 = V >> 2;
        for (int base = 0; base < n4; base += kThreads * kUnroll) {
            float4 v[kUnroll];
#pragma unroll
            for (int u = 0; u < kUnroll; u++)
                v[u] = NT ? ldg_nt(r4 + min(base + u * kThreads + t, n4 - 1))
                          : ldg(r4 + min(base + u * kThreads + t, n4 - 1));   // unconditional: no wait between loads
#pragma unroll
            for (int u = 0; u < kUnroll; u++) {
                int q = base + u * kThreads + t;
                if (q < n4) {
                    f(4 * q + 0, v[u].x);
                    f(4 * q + 1, v[u].y);
                    f(4 * q + 2, v[u].z);
                    f(4 * q + 3, v[u].w);
                }
            }
        }
        for (int i = (n4 << 2) + t; i < V; i += kThreads) f(i, ldg(row + i));
    } else {
        for (int base = 0; base < V; base += kThreads * kUnroll) {
            float v[kUnroll];
#pragma unroll
            for (int u = 0; u < kUnroll; u++) v[u] = ldg(row + min(base + u * kThreads + t, V - 1));
#pragma unroll
            for (int u = 0; u < kUnroll; u++) {
                int i = base + u * kThreads + t;
                if (i < V) f(i, v[u]);
            }
        }
    }
}

// f(i, row[i]) for every element of a row that is only 4-byte aligned: the
// first h < 4 elements (up to the next 16-byte boundary) one per thread, the
// body as float4, the last (V - h) % 4 one per thread.
template <bool NT = false, class F>
__device__ __forceinline__ void row_for_each_any(const float *row, int V, F f)
{
    const int h = min(V, (int)(((16u - ((uint32_t)reinterpret_cast<uintptr_t>(row) & 15u)) & 15u) >> 2));
    if ((int)threadIdx.x < h) f((int)threadIdx.x, ldg(row + threadIdx.x));
    row_for_each<NT>(row + h, V - h, true, [&](int i, float x) { f(i + h, x); });
}

// Two-phase visit of a 16-byte aligned row: for each float4, cls(y) is
// evaluated for the four values first (pure, so their LDS reads issue
// together), then act(i, y, c) performs the side effects in index order.
// xf maps the raw logit to the value that is classified.
template <class X, class C, class A>
__device__ __forceinline__ void row_for_each_cls(const float *row, int V, X xf, C cls, A act)
{
    const int t = threadIdx.x;
    const float4 *r4 = reinterpret_cast<const float4 *>(row);
    const int n4 = V >> 2;
    for (int base = 0; base < n4; base += kThreads * kUnroll) {
        float4 v[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; u++)
            v[u] = ldg(r4 + min(base + u * kThreads + t, n4 - 1));   // unconditional: no wait between loads
#pragma unroll
        for (int u = 0; u < kUnroll; u++) {
            const int q = base + u * kThreads + t;
            if (q < n4) {
                const float y0 = xf(v[u].x), y1 = xf(v[u].y), y2 = xf(v[u].z), y3 = xf(v[u].w);
                const auto c0 = cls(y0), c1 = cls(y1), c2 = cls(y2), c3 = cls(y3);
                act(4 * q + 0, y0, c0);
                act(4 * q + 1, y1, c1);
                act(4 * q + 2, y2, c2);
                act(4 * q + 3, y3, c3);
            }
        }
    }
    for (int i = (n4 << 2) + t; i < V; i += kThreads) {
        const float y = xf(ldg(row + i));
        act(i, y, cls(y));
    }
}

// --------------------------------------------------------------------------
// Greedy (T <= 0): argmax over penalized logits, last index among equals.
__device__ void greedy_row(RowSmem &sm, const float *row, int V, bool has_pen, int *tok, int *status)
{
    float bv = -INFINITY;
    int bi = -1;
    int nan = 0;
    for (int i = threadIdx.x; i < V; i += kThreads) {
        float x = row[i];
        nan |= isnan(x);
        if (x > bv || (x == bv && i > bi)) {
            if (!has_pen || hash_find(sm, (uint32_t)i) < 0) { bv = x; bi = i; }
        }
    }
    if (has_pen) {
        for (int s = threadIdx.x; s < kHashSlots; s += kThreads) {
            uint32_t id = sm.hkey[s];
            if (id == kEmpty) continue;
            float x = __uint_as_float(sm.hval[s]);
            nan |= isnan(x);
            if (x > bv || (x == bv && (int)id > bi)) { bv = x; bi = (int)id; }
        }
    }
    // wave reduce
    for (int d = 32; d > 0; d >>= 1) {
        float ov = __shfl_xor(bv, d, 64);
        int oi = __shfl_xor(bi, d, 64);
        if (ov > bv || (ov == bv && oi > bi)) { bv = ov; bi = oi; }
    }
    if (lane_id() == 0) { sm.red_f32[wave_id()] = bv; sm.red_i32[wave_id()] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        float v = sm.red_f32[0]; int ix = sm.red_i32[0];
        for (int w = 1; w < kWaves; w++) {
            float ov = sm.red_f32[w]; int oi = sm.red_i32[w];
            if (ov > v || (ov == v && oi > ix)) { v = ov; ix = oi; }
        }
        sm.tok = ix < 0 ? 0 : ix;
    }
    __syncthreads();
    int anynan = block_or(nan, sm);
    *tok = sm.tok;
    *status = (anynan && V > 1) ? GS_ERR_NAN : GS_OK;
}

// --------------------------------------------------------------------------
// Wave-level softmax / nucleus / draw for n <= 256 survivors.  Every lane of
// the wave runs the reference's sequential loops (src/sampler.rs:53-78) in
// lockstep, reading the element of step j with v_readlane, so each f32 op is
// the reference's op in the reference's order.  Lane l holds positions
// l, l+64, l+128, l+192.
constexpr int kWaveFinishMax = 256;

__device__ __forceinline__ float rdl(float v, int l)
{
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// Sequential f32 accumulation cum_{j+1} = cum_j + sh[j], j in [0, len), in
// the reference's order, stopping at the first j with pred(cum_{j+1}).
// One wave; sh is wave-private LDS, zero past the values (len <= 256).  The
// values are read with uniform addresses (LDS broadcast) eight at a time,
// so the adds form a plain VGPR chain; lane i of each group keeps the
// running sum after its element, and one ballot per group finds the stop.
// Returns j (or len) and the running sum there (or after len) in *sum.
template <class P>
__device__ __forceinline__ int wave_seq(const float *sh, int len, P pred, float *sum)
{
    const int lane = lane_id();
    float cum = 0.0f;
#pragma nounroll
    for (int g = 0; g < len; g += 8) {
        const float4 a = *reinterpret_cast<const float4 *>(sh + g);
        const float4 b = *reinterpret_cast<const float4 *>(sh + g + 4);
        const float vals[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        const int base = g & 63;
        float cv = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            cum = cum + vals[i];
            cv = lane == base + i ? cum : cv;
        }
        const int j = (g - base) + lane;
        const uint64_t hit = __ballot(lane >= base && lane < base + 8 && j < len && pred(cv));
        if (hit) {
            const int L = (int)__builtin_ctzll(hit);
            *sum = rdl(cv, L);
            return (g - base) + L;
        }
    }
    *sum = cum;   // the zero padding past len leaves the sum unchanged
    return len;
}

template <class YV, class IX>
__device__ int finish_wave(RowSmem &sm, int n, YV yv, IX idx, float top_p, float r)
{
    const int lane = lane_id();
    const float m = yv(0);
    if (isinf(m)) return (int)idx(n - 1);
    float *sh = sm.fin;
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const int j = c * 64 + lane;
        sh[j] = (j < n) ? glibc_expf(yv(j) - m) : 0.0f;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    float sum;
    (void)wave_seq(sh, n, [](float) { return false; }, &sum);          // src/sampler.rs:54
#pragma unroll
    for (int c = 0; c < 4; c++) sh[c * 64 + lane] = sh[c * 64 + lane] / sum;   // :55 (0 / sum = 0)
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    int cut = n;
    if (top_p < 1.0f) {
        float s2;
        const int stop = wave_seq(sh, n, [top_p](float c) { return c >= top_p; }, &s2);   // :59-64
        cut = stop < n ? stop + 1 : n;
        // the renormalising sum (:67) equals the running sum at the cut
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const int j = c * 64 + lane;
            sh[j] = j < cut ? sh[j] / s2 : 0.0f;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
    }
    float c;
    const int pick = wave_seq(sh, cut, [r](float cc) { return r < cc; }, &c);   // :72-77
    return (int)idx(pick < cut ? pick : cut - 1);
}

// --------------------------------------------------------------------------
// Softmax, nucleus and draw over n candidates sorted descending.  yv(j) gives
// the scaled logit of candidate j, idx(j) its token id.  Mirrors
// src/sampler.rs:53-78 exactly (block_seqsum reproduces every f32 sum).
template <class YV, class IX>
__device__ int finish_sorted(RowSmem &sm, int n, YV yv, IX idx, float top_p, float r)
{
    if (n <= kWaveFinishMax) {
        if (wave_id() == 0) {
            int tk = finish_wave(sm, n, yv, idx, top_p, r);
            if (lane_id() == 0) sm.tok = tk;
        }
        GS_SUB0(6);
        __syncthreads();
        const int tk = sm.tok;
        __syncthreads();
        return tk;
    }
    const float m = yv(0);
    if (isinf(m)) {
        // y - m is NaN for some element (src/sampler.rs:54), every probability
        // is NaN, no comparison succeeds and the reference returns the last
        // kept candidate (src/sampler.rs:78).
        return (int)idx(n - 1);
    }
    auto e_of = [&](int j) { return glibc_expf(yv(j) - m); };
    float sum;
    block_seqsum(e_of, n, 0.0f, [](float) { return false; }, &sum, sm.seq);
    auto p_of = [&](int j) { return e_of(j) / sum; };
    int cut = n;
    if (top_p < 1.0f) {
        float s2;
        int stop = block_seqsum(p_of, n, 0.0f, [top_p](float c) { return c >= top_p; }, &s2, sm.seq);
        cut = stop < n ? stop + 1 : n;
        auto q_of = [&](int j) { return p_of(j) / s2; };
        float c;
        int pick = block_seqsum(q_of, cut, 0.0f, [r](float cc) { return r < cc; }, &c, sm.seq);
        return (int)idx(pick < cut ? pick : cut - 1);
    }
    float c;
    int pick = block_seqsum(p_of, n, 0.0f, [r](float cc) { return r < cc; }, &c, sm.seq);
    return (int)idx(pick < n ? pick : n - 1);
}

// --------------------------------------------------------------------------
// Bitonic sort of sm.x.tk.cand[0..P) descending, P a power of two.
__device__ void bitonic_desc(RowSmem &sm, int P)
{
    for (int k = 2; k <= P; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = threadIdx.x; i < P; i += kThreads) {
                int l = i ^ j;
                if (l > i) {
                    uint64_t a = sm.x.tk.cand[i], b = sm.x.tk.cand[l];
                    bool desc = (i & k) == 0;
                    if (desc ? (a < b) : (a > b)) { sm.x.tk.cand[i] = b; sm.x.tk.cand[l] = a; }
                }
            }
            __syncthreads();
        }
    }
}

__device__ __forceinline__ uint64_t cand_of(uint32_t key, uint32_t idx)
{
    return ((uint64_t)key << 32) | (uint64_t)(~idx);
}

// Block exclusive sum scan of one u32 per thread; returns exclusive prefix and
// writes the total to *tot.
__device__ uint32_t block_excl_u32(uint32_t v, uint32_t *tot, RowSmem &sm)
{
    const int lane = lane_id(), w = wave_id();
    const uint32_t incl = wave_incl_u32(v);
    if (lane == 63) sm.red_u32[w] = incl;
    __syncthreads();
    uint32_t pre = 0, all = 0;
    for (int i = 0; i < kWaves; i++) { if (i < w) pre += sm.red_u32[i]; all += sm.red_u32[i]; }
    __syncthreads();
    *tot = all;
    return pre + incl - v;
}

// --------------------------------------------------------------------------
// Radix-select step over the histogram sm.x.tk.u.hist[0..nbins): the bin holding
// the need-th largest key (need >= 1) and the count of keys in higher bins.
// If fewer than `need` keys exist, returns bin 0.
__device__ void select_bin(RowSmem &sm, uint32_t nbins, uint32_t need, uint32_t *bin, uint32_t *above)
{
    const int t = threadIdx.x;
    const uint32_t per = (nbins + kThreads - 1) / kThreads;
    uint32_t mine = 0;
    for (uint32_t q = 0; q < per; q++) {
        uint32_t bt = t * per + q;            // index from the top
        if (bt < nbins) mine += sm.x.tk.u.hist[nbins - 1 - bt];
    }
    if (t == 0) { sm.sel_prefix = 0; sm.sel_above = 0; }
    uint32_t tot;
    uint32_t ex = block_excl_u32(mine, &tot, sm);   // contains barriers
    if (ex < need && ex + mine >= need) {
        uint32_t c = ex;
        for (uint32_t q = 0; q < per; q++) {
            uint32_t bt = t * per + q;
            uint32_t b = nbins - 1 - bt;
            uint32_t h = sm.x.tk.u.hist[b];
            if (c + h >= need) { sm.sel_prefix = b; sm.sel_above = c; break; }
            c += h;
        }
    }
    __syncthreads();
    *bin = sm.sel_prefix;
    *above = sm.sel_above;
    __syncthreads();
}

// Sort sm.x.tk.cand[0..n) descending (keys are unique).  Rank sort for n <= 1024:
// every element counts the larger keys (broadcast LDS reads), one scatter.
__device__ void sort_cand_desc(RowSmem &sm, int n)
{
    const int t = threadIdx.x;
    if (n > 1024) {
        int P = 1;
        while (P < n) P <<= 1;
        for (int i = n + t; i < P; i += kThreads) sm.x.tk.cand[i] = 0ull;
        __syncthreads();
        bitonic_desc(sm, P);
        return;
    }
    uint64_t *tmp = reinterpret_cast<uint64_t *>(sm.x.tk.u.hist);   // 2048 u64 of scratch
    for (int i = t; i < n; i += kThreads) tmp[i] = sm.x.tk.cand[i];
    __syncthreads();
    if (t < n) {
        const uint64_t me = tmp[t];
        int r = 0;
        int j = 0;
        for (; j + 4 <= n; j += 4)
            r += (tmp[j] > me) + (tmp[j + 1] > me) + (tmp[j + 2] > me) + (tmp[j + 3] > me);
        for (; j < n; j++) r += tmp[j] > me;
        sm.x.tk.cand[r] = me;
    }
    __syncthreads();
}

// --------------------------------------------------------------------------
// Top-k path.
//
// XSPACE = true selects on the keys of the raw (penalized) logits x instead
// of y = x / T.  Division by T > 0 is monotone, so the order by x refines the
// order by y; it differs only where distinct x round to the same y.  After the
// survivors are sorted by y, the selection is accepted only if every element
// left out maps to a y strictly below the k-th survivor's y; otherwise the
// caller reruns with XSPACE = false (select directly on y).  This keeps the
// division out of the per-element loop.
// Returns the token; *ok = false asks for the y-space rerun.
template <bool XSPACE>
__device__ int topk_row(RowSmem &sm, const float *row, int V, int k, float T, float top_p,
                        bool has_pen, float r, bool aligned, int *status, bool *ok)
{
    const int t = threadIdx.x;
    *ok = true;
    auto keyof = [&](float x) { return XSPACE ? f2key(x) : f2key(x / T); };
    // Radix select over the 32-bit keys in 3 levels: 12, 12, 8 bits.
    uint32_t prefix = 0;        // key bits above `shift` fixed so far
    int shift = 32;
    uint32_t above = 0;         // elements with key strictly above the in-play range
    int nan = 0;
    bool fits = false;
    for (int level = 0; level < 3; level++) {
        const int wbits = level < 2 ? 12 : 8;
        const int nsh = shift - wbits;
        const uint32_t nbins = 1u << wbits;
        for (uint32_t i = t; i < nbins; i += kThreads) sm.x.tk.u.hist[i] = 0;
        __syncthreads();
        if (level == 0) {
            row_for_each(row, V, aligned, [&](int, float x) {
                nan |= (int)isnan(x) | ((int)isinf(x) & (int)isinf(T));
                atomicAdd(&sm.x.tk.u.hist[keyof(x) >> nsh], 1u);
            });
        } else {
            row_for_each(row, V, aligned, [&](int, float x) {
                uint32_t key = keyof(x);
                if ((key >> shift) == prefix) atomicAdd(&sm.x.tk.u.hist[(key >> nsh) & (nbins - 1)], 1u);
            });
        }
        __syncthreads();
        if (has_pen) {
            // Move penalized ids from their raw bin to their penalized bin.
            for (int s = t; s < kHashSlots; s += kThreads) {
                uint32_t id = sm.hkey[s];
                if (id == kEmpty) continue;
                uint32_t kr = keyof(row[id]);
                uint32_t kp = keyof(__uint_as_float(sm.hval[s]));
                if (shift == 32 || (kr >> shift) == prefix) atomicSub(&sm.x.tk.u.hist[(kr >> nsh) & (nbins - 1)], 1u);
                if (shift == 32 || (kp >> shift) == prefix) atomicAdd(&sm.x.tk.u.hist[(kp >> nsh) & (nbins - 1)], 1u);
            }
            __syncthreads();
        }
        if (level == 0 && block_or(nan, sm)) { *status = GS_ERR_NAN; return 0; }
        GS_STAMP(2);
        uint32_t b, sel_above;
        select_bin(sm, nbins, (uint32_t)k - above, &b, &sel_above);
        const uint32_t in_bin = sm.x.tk.u.hist[b];
        above += sel_above;
        prefix = (shift == 32 ? 0u : (prefix << wbits)) | b;
        shift = nsh;
        __syncthreads();
        if (above + in_bin <= (uint32_t)kCandCap) { fits = true; break; }
    }
    GS_STAMP(3);
    if (XSPACE && !fits) { *ok = false; return 0; }
    // Collect candidates: key >> shift >= prefix (when the tie range fits),
    // else key > K* plus the first (k - above) ids equal to K* in index order.
    if (t == 0) sm.ncand = 0;
    __syncthreads();
    const uint32_t kstar = prefix;  // a full key only when !fits (shift == 0)
    row_for_each(row, V, aligned, [&](int i, float x) {
        uint32_t key = keyof(x);
        bool take = fits ? ((key >> shift) >= prefix) : (key > kstar);
        if (take && !(has_pen && hash_find(sm, (uint32_t)i) >= 0)) {
            int slot = atomicAdd(&sm.ncand, 1);
            if (slot < kCandCap) sm.x.tk.cand[slot] = cand_of(f2key(x / T), (uint32_t)i);
        }
    });
    if (has_pen) {
        for (int s = t; s < kHashSlots; s += kThreads) {
            uint32_t id = sm.hkey[s];
            if (id == kEmpty) continue;
            float x = __uint_as_float(sm.hval[s]);
            uint32_t key = keyof(x);
            bool take = fits ? ((key >> shift) >= prefix) : (key > kstar);
            if (take) {
                int slot = atomicAdd(&sm.ncand, 1);
                if (slot < kCandCap) sm.x.tk.cand[slot] = cand_of(f2key(x / T), id);
            }
        }
    }
    __syncthreads();
    if (!XSPACE && !fits) {
        // Ordered selection of the first `need` elements equal to K*.
        uint32_t need = (uint32_t)k - above;
        uint32_t taken = 0;
        for (int base = 0; base < V && taken < need; base += kThreads) {
            int i = base + t;
            bool eq = false;
            if (i < V) eq = f2key(eff_scaled(sm, has_pen, (uint32_t)i, row[i], T)) == kstar;
            uint32_t tot;
            uint32_t ex = block_excl_u32(eq ? 1u : 0u, &tot, sm);
            if (eq && taken + ex < need) {
                int slot = atomicAdd(&sm.ncand, 1);
                if (slot < kCandCap) sm.x.tk.cand[slot] = cand_of(kstar, (uint32_t)i);
            }
            taken += tot;
        }
        __syncthreads();
    }
    GS_STAMP(4);
    const int nc = min(sm.ncand, kCandCap);
    sort_cand_desc(sm, nc);
    GS_STAMP(5);
    const int n = k;   // nc >= k by construction
    if (XSPACE && shift < 32) {
        // Elements left out have x-key < thr; their y is at most y_out.
        const uint32_t thr = prefix << shift;
        if (thr > 0x007fffffu) {   // below that key every real x is a candidate
            float y_out = key2f(thr - 1u) / T;
            uint32_t yk = (uint32_t)(sm.x.tk.cand[n - 1] >> 32);
            if (!(f2key(y_out) < yk)) { *ok = false; __syncthreads(); return 0; }
        }
    }
    auto yv = [&](int j) { return key2f((uint32_t)(sm.x.tk.cand[j] >> 32)); };
    auto ix = [&](int j) { return ~(uint32_t)sm.x.tk.cand[j]; };
    *status = GS_OK;
    return finish_sorted(sm, n, yv, ix, top_p, r);
}

// --------------------------------------------------------------------------
// Top-k path, one streaming pass plus one cached re-read.
//
// Pass 1 keeps only each thread's maximum raw logit (no atomics).  Among the
// 1024 thread maxima, the (k + U)-th largest (U = distinct penalized ids)
// is a lower bound tau on the k-th largest effective logit: those k + U
// maxima are distinct elements and at most U of them are penalized, so at
// least k unpenalized elements are >= tau.  Pass 2 collects every element
// whose effective logit is >= tau, they are sorted by y = x / T and the
// selection is accepted as in topk_row<true> (no element left out may tie
// the k-th y).  Returns ok = false when the bound is unusable (k + U > 1024,
// too many elements above tau); the caller then runs the radix select.
__device__ int topk_row_tmax(RowSmem &sm, const float *row, int V, int k, float T, float top_p,
                             bool has_pen, int nuniq, float r, bool aligned, int *status, bool *ok)
{
    const int t = threadIdx.x;
    *ok = false;
    const uint32_t need = (uint32_t)k + (uint32_t)nuniq;
    if (need > (uint32_t)kThreads) return 0;
    float tmax = -INFINITY;
    bool any = false;
    int nan = 0;
    row_for_each(row, V, aligned, [&](int, float x) {
        nan |= (int)isnan(x) | ((int)isinf(x) & (int)isinf(T));
        tmax = fmaxf(tmax, x);
        any = true;
    });
    if (block_or(nan, sm)) { *ok = true; *status = GS_ERR_NAN; return 0; }
    GS_STAMP(2);
    const uint32_t tk = any ? f2key(tmax) : 0u;
    // Two 12-bit radix levels over the 1024 thread maxima.
    uint32_t prefix = 0, above = 0;
    for (int level = 0; level < 2; level++) {
        const int sh = level == 0 ? 20 : 8;
        for (int i = t; i < 4096; i += kThreads) sm.x.tk.u.hist[i] = 0;
        __syncthreads();
        if (level == 0 || (tk >> 20) == prefix) atomicAdd(&sm.x.tk.u.hist[(tk >> sh) & 4095u], 1u);
        __syncthreads();
        uint32_t b, ab;
        select_bin(sm, 4096, need - above, &b, &ab);
        above += ab;
        prefix = level == 0 ? b : ((prefix << 12) | b);
    }
    const uint32_t tau = prefix << 8;   // >= need thread maxima have key >= tau
    GS_STAMP(3);
    if (t == 0) sm.ncand = 0;
    __syncthreads();
    row_for_each(row, V, aligned, [&](int i, float x) {
        if (f2key(x) >= tau && !(has_pen && hash_find(sm, (uint32_t)i) >= 0)) {
            int slot = atomicAdd(&sm.ncand, 1);
            if (slot < kCandCap) sm.x.tk.cand[slot] = cand_of(f2key(x / T), (uint32_t)i);
        }
    });
    if (has_pen) {
        for (int s = t; s < kHashSlots; s += kThreads) {
            uint32_t id = sm.hkey[s];
            if (id == kEmpty) continue;
            float x = __uint_as_float(sm.hval[s]);
            if (f2key(x) >= tau) {
                int slot = atomicAdd(&sm.ncand, 1);
                if (slot < kCandCap) sm.x.tk.cand[slot] = cand_of(f2key(x / T), id);
            }
        }
    }
    __syncthreads();
    GS_STAMP(4);
    const int nc = sm.ncand;
    __syncthreads();
    if (nc > kCandCap || nc < k) return 0;
    sort_cand_desc(sm, nc);
    GS_STAMP(5);
    if (tau > 0x007fffffu) {
        float y_out = key2f(tau - 1u) / T;
        uint32_t yk = (uint32_t)(sm.x.tk.cand[k - 1] >> 32);
        if (!(f2key(y_out) < yk)) return 0;
    }
    *ok = true;
    auto yv = [&](int j) { return key2f((uint32_t)(sm.x.tk.cand[j] >> 32)); };
    auto ix = [&](int j) { return ~(uint32_t)sm.x.tk.cand[j]; };
    *status = GS_OK;
    return finish_sorted(sm, k, yv, ix, top_p, r);
}

// Top-k for rows held in registers (V <= kThreads * 4 * kRegF4, V a multiple
// of 4, 16-byte aligned).  The caller loads the row once, before the penalty
// table is built.  The bound is the one of topk_row_tmax (the (k + U)-th
// largest of the 1024 thread maxima), found with one histogram level over
// the spread of the thread maxima: bin = (max key - key) >> shift, with the
// shift that maps that spread onto kSelBins bins.  Wave 0 scans the
// histogram and publishes the bin (a barrier: the scan is VALU work that
// every wave of a SIMD would otherwise repeat there).  The candidates are
// compacted per wave (one LDS atomic per wave), the penalized ids are left
// out through the id bitmap and come back from the penalty table with their
// penalized value, and a rank sort places only the first k.
constexpr int kRegF4 = 8;
constexpr int kSelBins = 2048;
__device__ __forceinline__ float f4c(const float4 &v, int c)
{
    return c == 0 ? v.x : (c == 1 ? v.y : (c == 2 ? v.z : v.w));
}
// LDS state of topk_row_reg, cleared before the kernel's first barrier.
__device__ __forceinline__ void reg_clear(RowSmem &sm, bool has_pen, int V)
{
    const int t = threadIdx.x;
    if (has_pen) {
        for (int i = t; i < kHashSlots; i += kThreads) { sm.hkey[i] = kEmpty; sm.hval[i] = 0u; }
        const int nw = min((V + 31) >> 5, kPenBitsWords);
        for (int i = t; i < nw; i += kThreads) sm.x.tk.pbits[i] = 0u;
    }
    for (int i = t; i < kSelBins; i += kThreads) sm.x.tk.u.hist[i] = 0u;
    if (t == 0) { sm.ncand = 0; sm.flag_snan = 0; }
}

// Penalty table of a register row (src/sampler.rs:23-30), built alongside
// the row pass: this thread's window id goes in now; the thread that created
// a slot (the returned slot, else -1) stores the penalized value after the
// next barrier, when the count is complete.  Also sets the id's bit.
__device__ __forceinline__ int pen_insert(RowSmem &sm, const PenLoad &pl, bool has_pen)
{
    int myslot = -1;
    if (has_pen && pl.id != kEmpty) {
        uint32_t h = hash_slot(pl.id);
        for (;;) {
            const uint32_t prev = atomicCAS(&sm.hkey[h], kEmpty, pl.id);
            if (prev == kEmpty || prev == pl.id) {
                if (prev == kEmpty) { atomicAdd(&sm.nuniq, 1); myslot = (int)h; }
                atomicAdd(&sm.hval[h], 1u);
                break;
            }
            h = (h + 1) & (kHashSlots - 1);
        }
        atomicOr(&sm.x.tk.pbits[pl.id >> 5], 1u << (pl.id & 31u));   // V <= 32 * kPenBitsWords: every id has a bit
    }
    return myslot;
}

// Greedy (T <= 0) for rows held in registers: the argmax of the penalized
// logits, the last index among equal maxima (src/sampler.rs:15-19: max_by
// keeps the last of equal elements; -0 and +0 compare equal).  A NaN
// anywhere makes the reference panic (V > 1).
__device__ __forceinline__ int greedy_row_reg(RowSmem &sm, const float *row, float4 (&rv)[kRegF4], PenLoad pl, int V, bool has_pen,
                              float pen, int *status)
{
    const int t = threadIdx.x, lane = lane_id(), w = wave_id();
    const int n4 = V >> 2;
    if (pl.id >= (uint32_t)V) pl.id = kEmpty;   // also kEmpty itself
    if (pl.id != kEmpty) pl.raw = ldg(row + pl.id);
    const int myslot = pen_insert(sm, pl, has_pen);
    uint64_t nanm = 0;
#pragma unroll
    for (int u = 0; u < kRegF4; u++) {
        nanm |= __ballot(__builtin_isunordered(rv[u].x, rv[u].y));
        nanm |= __ballot(__builtin_isunordered(rv[u].z, rv[u].w));
    }
    __syncthreads();   // counts and bitmap complete
    float bv = -INFINITY;
    int bi = -1;
    bool pnan = false;
    // elements in index order (u, then c), so >= keeps the last maximum
#pragma unroll
    for (int u = 0; u < kRegF4; u++) {
        const int q = u * kThreads + t;
        const uint32_t nib = (has_pen && q < n4) ? (sm.x.tk.pbits[q >> 3] >> ((q & 7) * 4)) & 15u : 0u;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const float x = f4c(rv[u], c);
            if (q < n4 && !((nib >> c) & 1u) && x >= bv) { bv = x; bi = 4 * q + c; }
        }
    }
    if (myslot >= 0) {
        const float pv = penalize(pl.raw, sm.hval[myslot], pen);
        pnan = isnan(pv);
        if (pv > bv || (pv == bv && (int)pl.id > bi)) { bv = pv; bi = (int)pl.id; }
    }
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) {
        const float ov = __shfl_xor(bv, d, 64);
        const int oi = __shfl_xor(bi, d, 64);
        if (ov > bv || (ov == bv && oi > bi)) { bv = ov; bi = oi; }
    }
    const bool wnan = (nanm != 0) || __any(pnan);
    if (lane == 0) { sm.red_f32[w] = bv; sm.red_i32[w] = bi; sm.red_u32[w] = wnan ? 1u : 0u; }
    __syncthreads();
    float v = sm.red_f32[0];
    int ix = sm.red_i32[0];
    uint32_t anynan = sm.red_u32[0];
#pragma unroll
    for (int i = 1; i < kWaves; i++) {
        const float ov = sm.red_f32[i];
        const int oi = sm.red_i32[i];
        if (ov > v || (ov == v && oi > ix)) { v = ov; ix = oi; }
        anynan |= sm.red_u32[i];
    }
    *status = (anynan && V > 1) ? GS_ERR_NAN : GS_OK;
    return ix < 0 ? 0 : ix;
}

// SEL: select only -- return with the k best, sorted (key of y, ~id), in
// the first k u64 of sm.x.tk.u.hist and *ok set, without sampling.
template <bool SEL = false>
__device__ __forceinline__ int topk_row_reg(RowSmem &sm, const float *row, float4 (&rv)[kRegF4], PenLoad pl, int V, int k, float T,
                            float top_p, bool has_pen, float pen, float r, int *status, bool *ok)
{
    const int t = threadIdx.x, lane = lane_id(), w = wave_id();
    const int n4 = V >> 2;
    const int n4r = min(n4, kThreads * kRegF4);   // float4s held in registers (the whole row, or its head)
    *ok = false;
    if (pl.id >= (uint32_t)V) pl.id = kEmpty;   // also kEmpty itself
    if (pl.id != kEmpty) pl.raw = ldg(row + pl.id);
    const int myslot = pen_insert(sm, pl, has_pen);
    // Slots past the row (clamped loads) become -inf, below every bound
    // used.  Done here, after the table inserts: overwriting a register that
    // a load is still filling waits for that load.
    const int wfirst = __builtin_amdgcn_readfirstlane(t & ~63);   // the wave's first thread
#pragma unroll
    for (int u = 0; u < kRegF4; u++)
        if (u * kThreads + wfirst + 63 >= n4r) {                     // wave-uniform: most waves skip
            if (u * kThreads + t >= n4r) rv[u] = make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
        }
    // Thread maximum and NaN test.
    float fmx = -INFINITY;
    float mu[kRegF4];        // per float4 maxima: the candidate passes skip float4s with no hit in the wave
    uint64_t nanm = 0;
#pragma unroll
    for (int u = 0; u < kRegF4; u++) {
        mu[u] = fmaxf(fmaxf(rv[u].x, rv[u].y), fmaxf(rv[u].z, rv[u].w));
        fmx = fmaxf(fmx, mu[u]);
        nanm |= __ballot(__builtin_isunordered(rv[u].x, rv[u].y));
        nanm |= __ballot(__builtin_isunordered(rv[u].z, rv[u].w));
    }
    const bool holds = t < n4r;
    const uint32_t tk = f2key(fmx);
    {
        const uint32_t wmax = wave_max_u32(holds ? tk : 0u);
        const uint32_t wmin = wave_min_u32(holds ? tk : 0xffffffffu);
        if (lane == 0) { sm.red_u32[w] = wmax; sm.red_i32[w] = (int)wmin; sm.red_f32[w] = nanm ? 1.0f : 0.0f; }
    }
    __syncthreads();
    uint32_t kmax = 0u, kmin = 0xffffffffu;
    bool anynan = false;
#pragma unroll
    for (int i = 0; i < kWaves; i++) {
        kmax = max(kmax, sm.red_u32[i]);
        kmin = min(kmin, (uint32_t)sm.red_i32[i]);
        anynan |= sm.red_f32[i] != 0.0f;
    }
    if (myslot >= 0) {
        const float l = penalize(pl.raw, sm.hval[myslot], pen);
        sm.hval[myslot] = __float_as_uint(l);
        if (isnan(l / T)) sm.flag_nan = 1;
    }
    // The bitmap is complete: a thread holding a penalized element takes
    // its maximum over the others, so the 1024 thread maxima are distinct
    // unpenalized elements and k of them bound the k-th largest.
    uint32_t tku = tk;
    if (has_pen) {
        uint32_t nib[kRegF4], anyp = 0u;
#pragma unroll
        for (int u = 0; u < kRegF4; u++) {
            const int q = u * kThreads + t;
            nib[u] = q < n4r ? (sm.x.tk.pbits[q >> 3] >> ((q & 7) * 4)) & 15u : 0u;
            anyp |= nib[u];
        }
        if (__builtin_expect(anyp != 0u, 0)) {
            float f = -INFINITY;
#pragma unroll
            for (int u = 0; u < kRegF4; u++)
#pragma unroll
                for (int c = 0; c < 4; c++)
                    if (!((nib[u] >> c) & 1u)) f = fmaxf(f, f4c(rv[u], c));
            tku = f2key(f);
        }
    }
    const uint32_t need = (uint32_t)k;
    const uint32_t nmax = (uint32_t)min(n4r, kThreads);     // threads holding elements
    if (anynan) { *ok = true; *status = GS_ERR_NAN; return 0; }
    GS_STAMP(2);
    // Histogram of the thread maxima: bin = (kmax - key) >> shift.  Bin b
    // is stored at ((b >> 2) & 7) * 256 + (b >> 5) * 4 + (b & 3), so that
    // lane L's 32 consecutive bins are 8 uint4 at q * 256 + 4 * L: the
    // scan below reads them without bank conflicts.
    const uint32_t spread = kmax - kmin;
    const int shift = spread < (uint32_t)kSelBins ? 0 : (32 - __clz((int)spread)) - 11;
    if (holds) {
        const uint32_t bin = min((kmax - tku) >> shift, (uint32_t)kSelBins - 1u);
        atomicAdd(&sm.x.tk.u.hist[((bin >> 2) & 7u) * 256u + (bin >> 5) * 4u + (bin & 3u)], 1u);
    }
    __syncthreads();
    // The table holds penalized values from here on (also for the general
    // paths the caller falls back to).
    if (sm.flag_nan) { *ok = true; *status = GS_ERR_NAN; return 0; }
    if (need > nmax) return 0;
    // Bin of the need-th largest thread maximum, scanned by wave 0 (the
    // scan is VALU work that every other wave would repeat on its SIMD).
    if (w == 0) {
        const uint4 *h4 = reinterpret_cast<const uint4 *>(sm.x.tk.u.hist) + lane;
        uint32_t hv[kSelBins / 64];
#pragma unroll
        for (int q = 0; q < kSelBins / 256; q++) {
            const uint4 v = h4[q * 64];
            hv[4 * q] = v.x; hv[4 * q + 1] = v.y; hv[4 * q + 2] = v.z; hv[4 * q + 3] = v.w;
        }
        uint32_t mine = 0u;
#pragma unroll
        for (int q = 0; q < kSelBins / 64; q++) mine += hv[q];
        const uint32_t incl = wave_scan_add(mine);
        const uint32_t excl = incl - mine;
        const uint64_t hit = __ballot(excl < need && incl >= need);
        const int L = (int)__builtin_ctzll(hit);            // exists: need <= nmax = total
        // In lane L: the first bin whose running count reaches need (the
        // running count is monotone, so it is the number of prefixes below).
        uint32_t c = excl, b = 0u;
#pragma unroll
        for (int q = 0; q < kSelBins / 64 - 1; q++) {
            c += hv[q];
            b += c < need ? 1u : 0u;
        }
        // the readlane stays out of the lane-0 branch: b must be computed in lane L
        const uint32_t bin = (uint32_t)L * (kSelBins / 64) + (uint32_t)__builtin_amdgcn_readlane((int)b, L);
        if (lane == 0) sm.reg_sel = bin;
    }
    __syncthreads();
    const uint32_t sel = sm.reg_sel;
    // Keys >= tau are exactly those whose bin is <= sel; at least `need`
    // thread maxima are among them.  tf is the same bound as a float
    // (x >= tf <=> f2key(x) >= tau for every non-NaN x).  A bound at -inf
    // (too few finite logits) is left to the general path.
    const uint64_t span = ((uint64_t)(sel + 1u) << shift) - 1u;
    const uint32_t tau = span >= kmax ? 0u : kmax - (uint32_t)span;
    if (tau <= f2key(-INFINITY)) { __syncthreads(); return 0; }
    const float tf = key2f(tau);
    GS_STAMP(3);
    // Candidates: a counting pass (one compare per element, counts in
    // scalar registers), one LDS reservation per wave, then the writes in
    // the same order.  Entries hold the raw (value, id); the penalty bitmap
    // and the division by T are applied afterwards, one candidate per thread.
    uint32_t wcnt = 0u;
    uint32_t uany = 0u;      // bit u: some lane of the wave holds a hit in float4 u
#pragma unroll
    for (int u = 0; u < kRegF4; u++) {
        if (__ballot(mu[u] >= tf) == 0) continue;
        uany |= 1u << u;
        wcnt += (uint32_t)__popcll(__ballot(rv[u].x >= tf));
        wcnt += (uint32_t)__popcll(__ballot(rv[u].y >= tf));
        wcnt += (uint32_t)__popcll(__ballot(rv[u].z >= tf));
        wcnt += (uint32_t)__popcll(__ballot(rv[u].w >= tf));
    }
    GS_SUB0(0);
    uint32_t wpos = 0u;
    if (lane == 0 && wcnt) wpos = atomicAdd((uint32_t *)&sm.ncand, wcnt);
    wpos = (uint32_t)__builtin_amdgcn_readfirstlane((int)wpos);
#pragma unroll
    for (int u = 0; u < kRegF4; u++) {
        if (!((uany >> u) & 1u)) continue;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const float x = f4c(rv[u], c);
            const uint64_t m = __ballot(x >= tf);
            if (__builtin_expect(m != 0, 0)) {   // rare: the common path falls through
                const uint32_t pos = wpos + (uint32_t)__popcll(m & lanemask_lt());
                if (x >= tf && pos < (uint32_t)kCandCap)
                    sm.x.tk.cand[pos] = ((uint64_t)__float_as_uint(x) << 32) | (uint32_t)(4 * (u * kThreads + t) + c);
                wpos += (uint32_t)__popcll(m);
            }
        }
    }
    GS_SUB0(1);
    if (n4 > n4r) {
        // A row longer than the registers hold: the bound of its head (k
        // unpenalized elements of the head reach it) also bounds the k-th
        // largest of the whole row.  The rest streams through the same
        // registers in one pass: slot u is consumed and refilled with the
        // float4 kRegF4 slots ahead, so kRegF4 loads per thread stay in
        // flight.  Elements at or above the bound (rare) join the list as
        // above; a NaN anywhere makes the row an error.  (Non-temporal
        // loads: each logit is read once.)
        const float4 *r4 = reinterpret_cast<const float4 *>(row);
        bool snan = false;
        auto ld = [&](int u) { return ldg_nt(r4 + min(n4r + u * kThreads + t, n4 - 1)); };
        float4 s0 = ld(0), s1 = ld(1), s2 = ld(2), s3 = ld(3), s4 = ld(4), s5 = ld(5), s6 = ld(6), s7 = ld(7);
        auto slot = [&](float4 &r, int base, int u) __attribute__((always_inline)) {
            const float4 v = r;
            const int q = base + u * kThreads + t;
            r = ldg_nt(r4 + min(q + kRegF4 * kThreads, n4 - 1));
            const bool in = q < n4;
            snan |= in && (__builtin_isunordered(v.x, v.y) || __builtin_isunordered(v.z, v.w));
            const bool hit = in && (v.x >= tf || v.y >= tf || v.z >= tf || v.w >= tf);
            if (__builtin_expect(__ballot(hit) != 0, 0)) {
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    const float x = c == 0 ? v.x : (c == 1 ? v.y : (c == 2 ? v.z : v.w));
                    const bool h = in && x >= tf;
                    const uint64_t m = __ballot(h);
                    if (m != 0) {
                        uint32_t p0 = 0u;
                        if (lane == 0) p0 = atomicAdd((uint32_t *)&sm.ncand, (uint32_t)__popcll(m));
                        p0 = (uint32_t)__builtin_amdgcn_readfirstlane((int)p0);
                        const uint32_t pos = p0 + (uint32_t)__popcll(m & lanemask_lt());
                        if (h && pos < (uint32_t)kCandCap)
                            sm.x.tk.cand[pos] = ((uint64_t)__float_as_uint(x) << 32) | (uint32_t)(4 * q + c);
                    }
                }
            }
        };
        static_assert(kRegF4 == 8, "the stream loop names its eight slots");
        for (int base = n4r; base < n4; base += kRegF4 * kThreads) {
            slot(s0, base, 0); slot(s1, base, 1); slot(s2, base, 2); slot(s3, base, 3);
            slot(s4, base, 4); slot(s5, base, 5); slot(s6, base, 6); slot(s7, base, 7);
        }
        if (snan) sm.flag_snan = 1;
    }
    constexpr uint32_t kPenFlag = 0x80000000u;   // entry holds an already penalized value
    // The penalized ids at or above the bound.  Sampling rows: each table
    // slot is checked by the thread that created it (its window id, its own
    // penalized value).  Chunk selection (SEL): a scan of the table, since
    // keeping the slot and id live to here raised the chunk kernel's VGPR
    // spills from 4 to 11 (C2 +0.6 us; the owner check saves 0.2 us on C1).
    if (!SEL && has_pen && myslot >= 0) {
        const uint32_t xb = sm.hval[myslot];
        if (f2key(__uint_as_float(xb)) >= tau) {
            const int slot = atomicAdd(&sm.ncand, 1);
            if (slot < kCandCap) sm.x.tk.cand[slot] = ((uint64_t)xb << 32) | (pl.id | kPenFlag);
        }
    }
    if (SEL && has_pen) {
        for (int s = t; s < kHashSlots; s += kThreads) {
            const uint32_t id = sm.hkey[s];
            if (id == kEmpty) continue;
            const uint32_t xb = sm.hval[s];
            if (f2key(__uint_as_float(xb)) >= tau) {
                const int slot = atomicAdd(&sm.ncand, 1);
                if (slot < kCandCap) sm.x.tk.cand[slot] = ((uint64_t)xb << 32) | (id | kPenFlag);
            }
        }
    }
    GS_SUB0(2);
    __syncthreads();
    GS_STAMP(4);
    if (n4 > n4r && sm.flag_snan) { *ok = true; *status = GS_ERR_NAN; return 0; }
    const int nc = sm.ncand;
    if (nc > kCandCap || nc < k) { __syncthreads(); return 0; }   // the fallback reuses the LDS
    // Raw entries -> (key of y, ~id); a penalized id found in the row is
    // dropped (key 0 sorts last), its table entry stands for it.
    for (int i = t; i < nc; i += kThreads) {
        const uint64_t e = sm.x.tk.cand[i];
        const float x = __uint_as_float((uint32_t)(e >> 32));
        const uint32_t tag = (uint32_t)e;
        const uint32_t id = tag & ~kPenFlag;
        const bool drop = has_pen && !(tag & kPenFlag) && ((sm.x.tk.pbits[id >> 5] >> (id & 31u)) & 1u);
        sm.x.tk.cand[i] = drop ? (uint64_t)(~id) : cand_of(f2key(x / T), id);
    }
    for (int i = nc + t; i < ((nc + 7) & ~7); i += kThreads) sm.x.tk.cand[i] = 0ull;   // pad: never larger
    GS_SUB0(3);
    __syncthreads();
    GS_SUB0(4);
    // Rank sort (keys unique), G threads per candidate, 8 entries per step
    // (four 16-byte LDS reads in flight); only the first k are placed.
    uint64_t *top = reinterpret_cast<uint64_t *>(sm.x.tk.u.hist);   // 2048 u64
    {
        const int nc8 = (nc + 7) >> 3;                 // steps of 8 (padding entries are 0)
        const int lg = nc <= kThreads / 4 ? 2 : (nc <= kThreads / 2 ? 1 : 0);
        const int G = 1 << lg;
        const int len = (nc8 + G - 1) >> lg;           // steps per thread
        for (int base = 0; base < (nc << lg); base += kThreads) {
            const int gi = base + t;
            const int i = gi >> lg, part = gi & (G - 1);
            const bool act = i < nc;
            const uint64_t me = act ? sm.x.tk.cand[i] : ~0ull;
            const int s0 = part * len, s1 = min(nc8, s0 + len);
            const ulonglong2 *c2 = reinterpret_cast<const ulonglong2 *>(sm.x.tk.cand);
            int rk = 0;
            for (int st = s0; st < s1; st++) {
                const ulonglong2 a0 = c2[4 * st], a1 = c2[4 * st + 1], a2 = c2[4 * st + 2], a3 = c2[4 * st + 3];
                rk += (a0.x > me) + (a0.y > me) + (a1.x > me) + (a1.y > me) +
                      (a2.x > me) + (a2.y > me) + (a3.x > me) + (a3.y > me);
            }
            if (lg >= 1) rk += __shfl_xor(rk, 1, 64);
            if (lg >= 2) rk += __shfl_xor(rk, 2, 64);
            if (act && part == 0 && rk < k) top[rk] = me;
        }
    }
    GS_SUB0(5);
    __syncthreads();
    GS_STAMP(5);
    {
        const uint32_t yk = (uint32_t)(top[k - 1] >> 32);   // 0: fewer than k kept
        const bool bad = yk == 0u || (tau > 0x007fffffu && !(f2key(key2f(tau - 1u) / T) < yk));
        if (bad) { __syncthreads(); return 0; }
    }
    *ok = true;
    if (SEL) { *status = GS_OK; return 0; }
    auto yv = [&](int j) { return key2f((uint32_t)(top[j] >> 32)); };
    auto ix = [&](int j) { return ~(uint32_t)top[j]; };
    *status = GS_OK;
    return finish_sorted(sm, k, yv, ix, top_p, r);
}

#include "gs_full.hpp"
#include "gs_full3.hpp"

// --------------------------------------------------------------------------
// Full-vocabulary path: stable LSD radix sort of (~key, index) in scratch.
// ~key ascending == key descending; stability keeps equal keys in index order.
// finish_sorted's result over the sorted row, plus the detail outputs
// (gs_detail): the kept ids, a_j / S, n, the cut, S, s2 and the tie flag.
// kA holds the sorted keys (complemented), for the tie test.
template <typename YV, typename IX>
__device__ int finish_detail(RowSmem &sm, int n, int V, YV yv, IX idx, const uint32_t *kA, float top_p, float r,
                             const gs_detail &d, int b)
{
    const int t = threadIdx.x;
    const float m = yv(0);
    auto e_of = [&](int j) { return glibc_expf(yv(j) - m); };
    float sum = NAN;
    if (!isinf(m)) block_seqsum(e_of, n, 0.0f, [](float) { return false; }, &sum, sm.seq);
    auto p_of = [&](int j) { return e_of(j) / sum; };
    const size_t cap = d.cap;
    for (int j = t; j < n && (size_t)j < cap; j += kThreads) {
        if (d.ids) d.ids[(size_t)b * cap + j] = idx(j);
        if (d.p) d.p[(size_t)b * cap + j] = p_of(j);
    }
    int cut = n, pos;
    float s2 = 1.0f;
    if (isinf(m)) {
        // every probability is NaN: no cut, no draw succeeds (src/sampler.rs:64, 76)
        s2 = NAN;
        pos = n - 1;
    } else if (top_p < 1.0f) {
        int stop = block_seqsum(p_of, n, 0.0f, [top_p](float c) { return c >= top_p; }, &s2, sm.seq);
        cut = stop < n ? stop + 1 : n;   // s2: the sum through the cut, or of every p (src/sampler.rs:67)
        auto q_of = [&](int j) { return p_of(j) / s2; };
        float c;
        int pick = block_seqsum(q_of, cut, 0.0f, [r](float cc) { return r < cc; }, &c, sm.seq);
        pos = pick < cut ? pick : cut - 1;
    } else {
        float c;
        int pick = block_seqsum(p_of, n, 0.0f, [r](float cc) { return r < cc; }, &c, sm.seq);
        pos = pick < n ? pick : n - 1;
    }
    const int tok = (int)idx(pos);
    // bit 0: equal keys meet inside [0, cut] or at the truncation boundary;
    // bit 1: the drawn element's key is shared (the token depends on the
    // order of equal keys; the sums never do: equal summands commute)
    int tie = 0;
    for (int j = t; j < cut && j + 1 < V; j += kThreads) tie |= (int)(kA[j] == kA[j + 1]);
    if (t == 0 && n < V) tie |= (int)(kA[n - 1] == kA[n]);
    if (t == 0 && ((pos > 0 && kA[pos - 1] == kA[pos]) || (pos + 1 < V && kA[pos + 1] == kA[pos]))) tie |= 2;
    tie = block_or(tie & 1, sm) | (block_or(tie >> 1, sm) << 1);
    if (t == 0) {
        if (d.n_kept) d.n_kept[b] = (uint32_t)n;
        if (d.cut) d.cut[b] = (uint32_t)cut;
        if (d.sums) { d.sums[2 * b] = sum; d.sums[2 * b + 1] = s2; }
        if (d.ties) d.ties[b] = (uint32_t)tie;
    }
    return tok;
}

__device__ int full_row(RowSmem &sm, const float *row, int V, int keep, float T, float top_p,
                        bool has_pen, float r, uint32_t *kA, uint32_t *iA, uint32_t *kB,
                        uint32_t *iB, int *status, const gs_detail *det = nullptr)
{
    const int t = threadIdx.x;
    int nan = 0;
    for (int i = t; i < V; i += kThreads) {
        float y = row[i] / T;
        nan |= isnan(y);
        kA[i] = ~f2key(y);
        iA[i] = (uint32_t)i;
    }
    __syncthreads();
    if (has_pen) {
        for (int s = t; s < kHashSlots; s += kThreads) {
            uint32_t id = sm.hkey[s];
            if (id != kEmpty) kA[id] = ~f2key(__uint_as_float(sm.hval[s]) / T);
        }
    }
    __threadfence_block();
    __syncthreads();
    if (block_or(nan, sm) && V > 1) { *status = GS_ERR_NAN; return 0; }

    const int lane = lane_id(), w = wave_id();
    uint32_t *src_k = kA, *src_i = iA, *dst_k = kB, *dst_i = iB;
    for (int pass = 0; pass < 4; pass++) {
        const int sh = pass * 8;
        for (int i = t; i < 256; i += kThreads) sm.x.tk.base[i] = 0;
        __syncthreads();
        for (int i = t; i < V; i += kThreads) atomicAdd(&sm.x.tk.base[(src_k[i] >> sh) & 255u], 1u);
        __syncthreads();
        if (t == 0) {
            uint32_t run = 0;
            for (int d = 0; d < 256; d++) { uint32_t c = sm.x.tk.base[d]; sm.x.tk.base[d] = run; run += c; }
        }
        __syncthreads();
        constexpr int kSlots = 4;
        for (int tile = 0; tile < V; tile += kThreads * kSlots) {
            for (int i = t; i < kWaves * 256; i += kThreads) sm.x.tk.u.wcnt[i] = 0;
            __syncthreads();
            uint32_t dig[kSlots], rnk[kSlots], kk[kSlots], ii[kSlots];
            bool val[kSlots];
            for (int q = 0; q < kSlots; q++) {
                int i = tile + w * 256 + q * 64 + lane;
                val[q] = i < V;
                kk[q] = val[q] ? src_k[i] : 0u;
                ii[q] = val[q] ? src_i[i] : 0u;
                uint32_t d = (kk[q] >> sh) & 255u;
                dig[q] = d;
                uint64_t act = __ballot(val[q]);
                uint64_t peers = act;
                for (int bit = 0; bit < 8; bit++) {
                    uint64_t bb = __ballot((d >> bit) & 1u);
                    peers &= ((d >> bit) & 1u) ? bb : ~bb;
                }
                uint32_t before = sm.x.tk.u.wcnt[w * 256 + d];
                rnk[q] = before + (uint32_t)__popcll(peers & lanemask_lt());
                // All lanes have read the counter before the leader bumps it
                // (one wave executes in lockstep; the barrier makes it explicit).
                __builtin_amdgcn_wave_barrier();
                if (val[q] && (peers & lanemask_lt()) == 0)
                    sm.x.tk.u.wcnt[w * 256 + d] = before + (uint32_t)__popcll(peers);
                __builtin_amdgcn_wave_barrier();
            }
            __syncthreads();
            for (int d = t; d < 256; d += kThreads) {
                uint32_t run = sm.x.tk.base[d];
                for (int ww = 0; ww < kWaves; ww++) {
                    uint32_t c = sm.x.tk.u.wcnt[ww * 256 + d];
                    sm.x.tk.u.wcnt[ww * 256 + d] = run;
                    run += c;
                }
                sm.x.tk.base[d] = run;
            }
            __syncthreads();
            for (int q = 0; q < kSlots; q++) {
                if (!val[q]) continue;
                uint32_t dst = sm.x.tk.u.wcnt[w * 256 + dig[q]] + rnk[q];
                dst_k[dst] = kk[q];
                dst_i[dst] = ii[q];
            }
            __syncthreads();
        }
        __threadfence_block();
        __syncthreads();
        uint32_t *tk = src_k; src_k = dst_k; dst_k = tk;
        uint32_t *ti = src_i; src_i = dst_i; dst_i = ti;
    }
    // After 4 passes the sorted data is back in (kA, iA).
    auto yv = [&](int j) { return key2f(~kA[j]); };
    auto ix = [&](int j) { return iA[j]; };
    *status = GS_OK;
    if (det) return finish_detail(sm, keep, V, yv, ix, kA, top_p, r, *det, blockIdx.x);
    return finish_sorted(sm, keep, yv, ix, top_p, r);
}

// The token and status of row b, written by thread 0 of the kernel that
// finishes the row: into the mapped completion word (single-row calls), or
// into tokens / status, followed by the decode step's commit of the row.
__device__ __forceinline__ void store_row(const RowArgs &a, int b, int tok, int status)
{
    if (a.done) {
        // Token, status and the call's sequence number in one 64-bit store:
        // the host sees all three or none, so no fence is needed.
        const uint64_t word = ((uint64_t)a.done_val << 32) | ((uint64_t)((uint32_t)status & 0xffu) << 24) |
                              (uint64_t)((uint32_t)tok & 0xffffffu);
        __hip_atomic_store(a.done, word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    } else {
        a.tokens[b] = (uint32_t)tok;
        if (a.status) a.status[b] = status;
        if (a.hook.rows) decode_commit_row(a.hook, b, (uint32_t)tok, status);
    }
}

// --------------------------------------------------------------------------
// Row paths: the small kernel serves greedy, degenerate and top-k rows; the
// full-vocabulary rows go to the binned kernel and, when its checks fail, to
// the sort kernel.  Each kernel derives the path from the row's parameters.
__host__ __device__ __forceinline__ bool is_full_path(const gs_params &p, int V)
{
    if (!(p.temperature > 0.0f) || V < 2) return false;
    const int keep = (p.top_k > 0 && p.top_k < (uint32_t)V) ? (int)p.top_k : V;
    return !(keep < V && keep <= kMaxTopK);
}

// The row kernel's modes.  kModeSmall: greedy, degenerate and top-k rows
// (and the virtual rows of chunked top-k rows); kModeBins: full-vocabulary
// rows by the exact binned path, and in the same block, when its checks fail
// (fb[b] = 1), the first binned form and then the sort path; kModeDetail: every
// row sorted, with the diagnostic outputs.  (A kernel that runs both kinds
// of rows in one launch was measured: instantiating it raises the binned
// kernel's register spills from 5 to 72, and c3 by 7%.)
enum { kModeSmall = 0, kModeBins = 1, kModeDetail = 3 };

// A row of the chunked top-k path (gs_kernels.hpp: chunk_count etc.).
__device__ __forceinline__ bool chunk_row(const gs_params &p, int V)
{
    return p.temperature > 0.0f && p.temperature < INFINITY && p.top_k > 0 && (int)p.top_k < V &&
           p.top_k <= kChunkMaxK;
}

// Row b of a batch by the kernel of mode MODE.  `chunked` (a.chunked, or
// the chunk kernel's own value) says how rows with chunk_row() true are
// handled: kChunkedX / kChunkedY sample the row's virtual row (penalized
// logits x, or scaled logits y), kChunkedSelf leaves them to the chunk
// kernel, 0 samples them as any other row.
template <int MODE>
__device__ __forceinline__ void sample_row(RowSmem &sm, const RowArgs &a, int b, int chunked)
{
    const int t = threadIdx.x;
    gs_params p = a.params ? a.params[b] : a.uparams;
    // A chunked top-k row: its virtual row (the chunks' best kp in index
    // order) is sampled as a row of width nch * kp with no penalty, and the
    // token maps back through cvidx.  Scaled values are sampled with T = 1
    // (y / 1 == y).
    const bool crow = MODE == kModeSmall && chunked && chunk_row(p, a.V);
    if (crow && chunked == kChunkedSelf) return;
    if (crow && chunked == kChunkedY) p.temperature = 1.0f;
    const int V = crow ? a.cnch * (((int)p.top_k + 3) & ~3) : a.V;
    // the detail kernel sorts every row with T > 0 (the rest: the small path)
    const bool sorted_row = MODE == kModeDetail && p.temperature > 0.0f && V >= 2;
    const bool full = MODE == kModeDetail ? sorted_row : is_full_path(p, V);
    if (MODE == kModeDetail && !sorted_row && t == 0) {
        if (a.det.n_kept) a.det.n_kept[b] = 0u;
        if (a.det.cut) a.det.cut[b] = 0u;
        if (a.det.ties) a.det.ties[b] = 0u;
    }
    if (MODE == kModeSmall && full) return;
    if (MODE == kModeBins && !full) {
        if (t == 0) a.fb[b] = 0;
        return;
    }
    GS_STAMP(8 * MODE);
#ifdef GS_TIMING
    if (MODE == kModeSmall && blockIdx.x == g_row && (threadIdx.x & 63) == 0)
        g_fails[1100 + (threadIdx.x >> 6)] = (int)__builtin_amdgcn_s_memrealtime();
    const uint64_t t_begin = __builtin_amdgcn_s_memrealtime();
#endif
    const float *row = crow ? a.cvrow + (size_t)b * a.cvld : a.logits + (size_t)b * a.ld;
    if (t == 0) { sm.nuniq = 0; sm.flag_nan = 0; }

    int tok = 0, status = GS_OK;
    const bool has_pen = !crow && (p.rep_penalty != 1.0f) && a.recent != nullptr;
    int W = 0;
    if (has_pen) {
        W = a.recent_len ? (int)a.recent_len[b] : a.W;
        if (W > a.W) W = a.W;
    }
    // Small top-k rows that fit in registers: issue the row loads before the
    // penalty table is built, so the two overlap.
    const int keep0 = (p.top_k > 0 && p.top_k < (uint32_t)V) ? (int)p.top_k : V;
    const bool regfit = MODE == kModeSmall && V > 1 && (V & 3) == 0 && V <= kThreads * 4 * kRegF4 &&
                        ((reinterpret_cast<uintptr_t>(row) & 15u) == 0);
    // Longer top-k rows (up to the penalty bitmap's reach): the head in
    // registers, the rest streamed once (topk_row_reg).
    const bool streamfit = MODE == kModeSmall && V > kThreads * 4 * kRegF4 && (V & 3) == 0 &&
                           V <= 32 * kPenBitsWords && ((reinterpret_cast<uintptr_t>(row) & 15u) == 0);
    const bool reg_greedy = regfit && p.temperature <= 0.0f;
    const bool regpath = ((regfit || streamfit) && p.temperature > 0.0f && p.temperature < INFINITY && keep0 < V) ||
                         reg_greedy;
    // The register paths issue the window id load first and the row loads
    // after it, and test the id (ids >= V are skipped) only after the first
    // barrier: loads complete in issue order, so a test before the row loads
    // are issued, or a wait for a load issued after them, would hold every
    // wave at that barrier until the whole row has arrived.  They load the
    // raw logits of the window ids themselves, after that barrier.  A short
    // host window arrives in the kernel arguments (kwin).
    PenLoad pl{kEmpty, 0.0f};
    const uint32_t *wsrc = nullptr;        // wave-uniform: no divergent join waits for the id
    if (regpath && has_pen && W > 0) {
        if (a.kwin_n) {
            const char __attribute__((address_space(4))) *ka =
                (const char __attribute__((address_space(4))) *)__builtin_amdgcn_kernarg_segment_ptr();
            wsrc = reinterpret_cast<const uint32_t *>((uintptr_t)(ka + offsetof(RowArgs, kwin)));
        } else {
            wsrc = a.recent + (size_t)b * a.ld_recent;
        }
    }
    uint32_t rid = kEmpty;
    if (wsrc) rid = ldg(wsrc + min(t, W - 1));
    float4 rv[kRegF4];
    if (regpath) {
        const float4 *r4 = reinterpret_cast<const float4 *>(row);
        const int n4 = V >> 2;
#pragma unroll
        for (int u = 0; u < kRegF4; u++) rv[u] = ldg_nt(r4 + min(u * kThreads + t, n4 - 1));
    }
    if (has_pen && !regpath) pl = pen_load(row, V, a.recent + (size_t)b * a.ld_recent, W, true);
    if (regpath) reg_clear(sm, has_pen, V);   // the register path builds its penalty table itself
    __syncthreads();
    if (has_pen && !regpath) build_penalty(sm, pl, p.temperature > 0.0f ? p.temperature : 1.0f, p.rep_penalty);
    if (wsrc && t < W) pl.id = rid;        // tested against V by the register paths
    GS_STAMP(8 * MODE + 1);

    // The uniform draw for this row (only consumed if T > 0).
    const float r = a.u ? a.u[b] : lcg_value(lcg_jump(a.lcg_state, (uint64_t)b));
    const bool aligned = ((reinterpret_cast<uintptr_t>(row) & 15u) == 0);
    const int keep = (p.top_k > 0 && p.top_k < (uint32_t)V) ? (int)p.top_k : V;

    if (MODE == kModeSmall || (MODE == kModeDetail && !sorted_row)) {
        if (V == 0) {
            tok = 0;
            status = p.temperature > 0.0f ? GS_ERR_EMPTY : GS_OK;
        } else if (!(p.temperature > 0.0f)) {
            // src/sampler.rs:39: `if temperature <= 0.0` -- a NaN temperature is
            // not <= 0, so it falls through to the division below.
            if (reg_greedy) tok = greedy_row_reg(sm, row, rv, pl, V, has_pen, p.rep_penalty, &status);
            else if (p.temperature <= 0.0f) greedy_row(sm, row, V, has_pen, &tok, &status);
            else {
                // T is NaN: every scaled logit is NaN; the sort panics for V > 1.
                tok = 0;
                status = V > 1 ? GS_ERR_NAN : GS_OK;
            }
        } else if (V == 1) {
            tok = 0;   // a single pair: no comparison can panic; token 0.
        } else if (sm.flag_nan) {
            status = GS_ERR_NAN;
        } else {
            bool ok;
            if (regpath)
                tok = topk_row_reg(sm, row, rv, pl, V, keep, p.temperature, p.top_p, has_pen, p.rep_penalty, r,
                                   &status, &ok);
            else
                tok = topk_row_tmax(sm, row, V, keep, p.temperature, p.top_p, has_pen, sm.nuniq, r,
                                    aligned, &status, &ok);
            if (!ok)
                tok = topk_row<true>(sm, row, V, keep, p.temperature, p.top_p, has_pen, r, aligned,
                                     &status, &ok);
            if (!ok)
                tok = topk_row<false>(sm, row, V, keep, p.temperature, p.top_p, has_pen, r, aligned,
                                      &status, &ok);
        }
    } else if (MODE == kModeBins) {
        bool done = false;
        if (sm.flag_nan) { status = GS_ERR_NAN; done = true; }
        else if (keep == V && ((reinterpret_cast<uintptr_t>(row) & 3u) == 0)) {
            uint64_t *gl = reinterpret_cast<uint64_t *>(a.scratch + (size_t)b * a.scratch_stride);
            const uint32_t lcap = (uint32_t)(a.scratch_stride / 2);
            done = full_v3_row(sm, row, V, p.temperature, p.top_p, has_pen, r, gl, lcap, &tok, &status);
        }
        if (t == 0) a.fb[b] = done ? 0 : 1;
        if (!done && keep == V && ((reinterpret_cast<uintptr_t>(row) & 3u) == 0)) {
            // the first binned form (per-bin classes and thresholds)
            __syncthreads();
            uint64_t *gl = reinterpret_cast<uint64_t *>(a.scratch + (size_t)b * a.scratch_stride);
            const uint32_t lcap = (uint32_t)(a.scratch_stride / 2);
            done = full_v2_row(sm, row, V, p.temperature, p.top_p, has_pen, r, gl, lcap, &tok, &status);
        }
        if (!done) {
            __syncthreads();
            const size_t off = (size_t)b * a.scratch_stride;
            tok = full_row(sm, row, V, keep, p.temperature, p.top_p, has_pen, r, a.scratch + off,
                           a.scratch + off + V, a.scratch + off + 2 * (size_t)V,
                           a.scratch + off + 3 * (size_t)V, &status, nullptr);
        }
    } else {
        bool done = false;
        if (sm.flag_nan) { status = GS_ERR_NAN; done = true; }
        if (!done) {
            const size_t off = (size_t)b * a.scratch_stride;
            tok = full_row(sm, row, V, keep, p.temperature, p.top_p, has_pen, r, a.scratch + off,
                           a.scratch + off + V, a.scratch + off + 2 * (size_t)V,
                           a.scratch + off + 3 * (size_t)V, &status, MODE == kModeDetail ? &a.det : nullptr);
        }
        if (MODE == kModeDetail && status != GS_OK && t == 0) {
            if (a.det.n_kept) a.det.n_kept[b] = 0u;
            if (a.det.cut) a.det.cut[b] = 0u;
            if (a.det.ties) a.det.ties[b] = 0u;
        }
    }
    GS_STAMP(8 * MODE + 7);
#ifdef GS_TIMING
    if (t == 0 && b < 256 && MODE == kModeBins) g_fails[256 + b] = (int)(__builtin_amdgcn_s_memrealtime() - t_begin);
#endif
    if (crow) tok = status == GS_OK ? (int)ldg(a.cvidx + (size_t)b * a.cvld + tok) : 0;
    if (t == 0) store_row(a, b, tok, status);
}

template <int MODE>
__global__ void __launch_bounds__(kThreads)
sample_rows_kernel(RowArgs a)
{
    __shared__ RowSmem sm;
    sample_row<MODE>(sm, a, blockIdx.x, a.chunked);
}

// Single-row register path as a kernel of its own (B = 1): only the code of
// the register-resident rows (V <= 32768, V % 4 == 0, 16-byte aligned row,
// greedy or 0 < k < V with k <= kMaxTopK, finite T), so it needs far fewer
// registers and no scratch.  The rare rows whose bound check fails report
// kStatusRetry; the host then runs sample_rows_kernel<kModeSmall> on the row.
constexpr int kStatusRetry = 0x7f;
__global__ void __launch_bounds__(kThreads)
reg_row_kernel(RowArgs a)
{
    __shared__ RowSmem sm;
    const int t = threadIdx.x;
    const int b = blockIdx.x;
    const int V = a.V;
    const gs_params p = a.uparams;
    const float *row = a.logits + (size_t)b * a.ld;
    GS_STAMP(0);
    if (t == 0) { sm.nuniq = 0; sm.flag_nan = 0; }
    const bool has_pen = (p.rep_penalty != 1.0f) && (a.recent != nullptr || a.kwin_n);
    const int W = has_pen ? a.W : 0;
    // Window id first, then the row (see sample_rows_kernel).
    const uint32_t *wsrc = nullptr;
    if (W > 0) {
        if (a.kwin_n) {
            const char __attribute__((address_space(4))) *ka =
                (const char __attribute__((address_space(4))) *)__builtin_amdgcn_kernarg_segment_ptr();
            wsrc = reinterpret_cast<const uint32_t *>((uintptr_t)(ka + offsetof(RowArgs, kwin)));
        } else {
            wsrc = a.recent + (size_t)b * a.ld_recent;
        }
    }
    uint32_t rid = kEmpty;
    if (wsrc) rid = ldg(wsrc + min(t, W - 1));
    float4 rv[kRegF4];
    {
        const float4 *r4 = reinterpret_cast<const float4 *>(row);
        const int n4 = V >> 2;
#pragma unroll
        for (int u = 0; u < kRegF4; u++) rv[u] = ldg_nt(r4 + min(u * kThreads + t, n4 - 1));
    }
    reg_clear(sm, has_pen, V);
    __syncthreads();
    GS_STAMP(1);
    PenLoad pl{kEmpty, 0.0f};
    if (t < W) pl.id = rid;
    int tok, status = GS_OK;
    if (p.temperature <= 0.0f) {
        tok = greedy_row_reg(sm, row, rv, pl, V, has_pen, p.rep_penalty, &status);
    } else {
        const float r = a.u ? a.u[b] : lcg_value(lcg_jump(a.lcg_state, (uint64_t)b));
        const int keep = (int)p.top_k;
        bool ok;
        tok = topk_row_reg(sm, row, rv, pl, V, keep, p.temperature, p.top_p, has_pen, p.rep_penalty, r,
                           &status, &ok);
        if (!ok) { tok = 0; status = kStatusRetry; }
    }
    GS_STAMP(7);
    if (t == 0) store_row(a, b, tok, status);
}

__global__ void window_push_kernel(uint32_t *win, int B, size_t ld, int W, size_t pos,
                                   const uint32_t *tok)
{
    int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b < B) win[(size_t)b * ld + (pos % (size_t)W)] = tok[b];
}

// What src/sampler.rs:37 and :41 leave in the caller's logits: each id of the
// row's window penalized once per occurrence (apply_rep_penalty, :23-30),
// then every logit divided by T when T > 0 (a row with T <= 0 returns from
// greedy before the division, :39).  Grid: (chunks of kMutChunk logits, B).
constexpr int kMutChunk = 4096;
__global__ void __launch_bounds__(256)
writeback_kernel(float *logits, size_t ld, int V, const gs_params *params, gs_params up,
                 const uint32_t *recent, size_t ld_recent, const uint32_t *recent_len, int W)
{
    __shared__ uint32_t cnt[kMutChunk];
    const int b = blockIdx.y;
    const int base = blockIdx.x * kMutChunk;
    const int n = min(kMutChunk, V - base);
    const gs_params p = params ? params[b] : up;
    const bool pen = recent != nullptr && p.rep_penalty != 1.0f;
    for (int i = threadIdx.x; i < n; i += blockDim.x) cnt[i] = 0u;
    __syncthreads();
    if (pen) {
        int w = recent_len ? (int)recent_len[b] : W;
        if (w > W) w = W;
        const uint32_t *rec = recent + (size_t)b * ld_recent;
        for (int j = threadIdx.x; j < w; j += blockDim.x) {
            const uint32_t id = rec[j];
            if (id >= (uint32_t)base && id < (uint32_t)(base + n)) atomicAdd(&cnt[id - base], 1u);
        }
    }
    __syncthreads();
    const bool div = !(p.temperature <= 0.0f);
    float *row = logits + (size_t)b * ld + base;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        float l = row[i];
        const uint32_t c = cnt[i];
        if (c) l = penalize(l, c, p.rep_penalty);
        if (div) l = l / p.temperature;
        row[i] = l;
    }
}

__global__ void synth_kernel(float *out, int B, int V, size_t ld, uint64_t seed, uint64_t c0, float sigma)
{
    size_t n = (size_t)B * V;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
        size_t b = i / (size_t)V, c = i - b * (size_t)V;
        out[b * ld + c] = synth_logit(seed, c0 + i, sigma);
    }
}

} // namespace gs

#ifdef GS_TIMING
extern "C" int gs_debug_vt(uint32_t *out)
{
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(gs::g_vt), sizeof(uint32_t) * 256 * 64) == hipSuccess ? 0 : -5;
}
extern "C" int gs_debug_stages(uint32_t *out)
{
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(gs::g_stages), sizeof(uint32_t) * 256 * 32) == hipSuccess ? 0 : -5;
}
extern "C" int gs_debug_stamps(uint64_t *out)
{
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(gs::g_stamp), sizeof(uint64_t) * 32) == hipSuccess ? 0 : -5;
}
extern "C" int gs_debug_fails(int *out)
{
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(gs::g_fails), sizeof(int) * 1280) == hipSuccess ? 0 : -5;
}
#endif
#if defined(GS_TIMING) || defined(GS_DIAG)
extern "C" int gs_debug_v3dump(int *out)
{
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(gs::g_v3dump), sizeof(int) * 64 * 256) == hipSuccess ? 0 : -5;
}
extern "C" int gs_debug_v3diag(int *out, uint32_t *ts, int clear)
{
    if (clear) {
        static int zeros[1024 * 32];
        static uint32_t z2[256 * 32];
        if (hipMemcpyToSymbol(HIP_SYMBOL(gs::g_v3diag), zeros, sizeof(zeros)) != hipSuccess) return -5;
        return hipMemcpyToSymbol(HIP_SYMBOL(gs::g_v3t), z2, sizeof(z2)) == hipSuccess ? 0 : -5;
    }
    if (hipMemcpyFromSymbol(out, HIP_SYMBOL(gs::g_v3diag), sizeof(int) * 1024 * 32) != hipSuccess) return -5;
    return hipMemcpyFromSymbol(ts, HIP_SYMBOL(gs::g_v3t), sizeof(uint32_t) * 256 * 32) == hipSuccess ? 0 : -5;
}
extern "C" int gs_debug_vdiag(int *out, int clear)
{
    if (clear) {
        static int zeros[1024 * 16];
        return hipMemcpyToSymbol(HIP_SYMBOL(gs::g_vdiag), zeros, sizeof(zeros)) == hipSuccess ? 0 : -5;
    }
    return hipMemcpyFromSymbol(out, HIP_SYMBOL(gs::g_vdiag), sizeof(int) * 1024 * 16) == hipSuccess ? 0 : -5;
}
#endif
#ifdef GS_TIMING
extern "C" int gs_debug_row(unsigned row)
{
    return hipMemcpyToSymbol(HIP_SYMBOL(gs::g_row), &row, sizeof(row)) == hipSuccess ? 0 : -5;
}
extern "C" int gs_debug_clear(const uint64_t *zeros)
{
    return hipMemcpyToSymbol(HIP_SYMBOL(gs::g_stamp), zeros, sizeof(uint64_t) * 32) == hipSuccess ? 0 : -5;
}
#endif

// Launch wrappers (host side of this translation unit).
namespace gs {

// --------------------------------------------------------------------------
// Split top-k for a few rows of a large vocabulary.  Pass 1: workgroup
// (c, b) takes elements [c0, c0 + L) of row b, applies the penalty
// (src/sampler.rs:23-30: the window's occurrences of each id in the chunk,
// one op per occurrence), scales by T, and keeps the kp largest under the
// sampler's order (y descending, index ascending).  It writes their
// penalized logits and ids to slots [c kp, (c + 1) kp) of row b's virtual
// row, in index order.  The global top-k is among the kept elements, and the
// virtual row lists them in index order, so sampling it (same penalized
// values, same division by T, no penalty) gives the same token.  A NaN in
// the chunk goes to the chunk's first slot, so the sampling reports it.
// Pass 2 samples the virtual rows.
constexpr int kSplitThreads = 256;
constexpr int kSplitPer = 2 * kSplitL / kSplitThreads;   // elements per thread, last chunk included
static_assert(kSplitMaxKp == kSelMaxKp, "split kp bound");

__global__ void __launch_bounds__(kSplitThreads)
split_select_kernel(RowArgs a, int nch, int kp, float *vrow, uint32_t *vidx, size_t vld)
{
    __shared__ SelSmem<kSplitThreads, kSplitPer> sm;
    const int c = blockIdx.x, b = blockIdx.y;
    const int c0 = c * kSplitL;
    const int L = c == nch - 1 ? a.V - c0 : kSplitL;
    const float *row = a.logits + (size_t)b * a.ld + c0;
    SelArgs s;
    s.T = a.uparams.temperature;
    s.rep = a.uparams.rep_penalty;
    s.kp = kp;
    s.recent = a.recent;
    s.ld_recent = a.ld_recent;
    s.recent_len = a.recent_len;
    s.W = a.W;
    s.vrow = vrow;
    s.vidx = vidx;
    s.vld = vld;
    chunk_select<kSplitThreads, kSplitPer>(sm, s, b, c, c0, L, [row](int i) { return ldg(row + i); });
}

// Chunked top-k path, pass 1: chunk c of row b (a row with chunk_row true;
// the others return) is [c V / nch, (c+1) V / nch), at most kChunkL logits,
// 32 per thread; its best kp = round_up(k, 4) go to slots [c kp, (c+1) kp)
// of row b's virtual row (stride vld), in index order.
constexpr int kChunkPer = kChunkL / kThreads;
__global__ void __launch_bounds__(kThreads)
chunk_topk_kernel(RowArgs a, int nch, float *vrow, uint32_t *vidx, size_t vld)
{
    __shared__ SelSmem<kThreads, kChunkPer> sm;
    const int c = blockIdx.x, b = blockIdx.y;
    const gs_params p = a.params ? a.params[b] : a.uparams;
    if (!chunk_row(p, a.V)) return;
    const int c0 = (int)((int64_t)c * a.V / nch);
    const int L = (int)((int64_t)(c + 1) * a.V / nch) - c0;
    const float *row = a.logits + (size_t)b * a.ld + c0;
    SelArgs s;
    s.T = p.temperature;
    s.rep = p.rep_penalty;
    s.kp = ((int)p.top_k + 3) & ~3;
    s.recent = a.recent;
    s.ld_recent = a.ld_recent;
    s.recent_len = a.recent_len;
    s.W = a.W;
    s.vrow = vrow;
    s.vidx = vidx;
    s.vld = vld;
    chunk_select<kThreads, kChunkPer>(sm, s, b, c, c0, L, [row](int i) { return ldg(row + i); });
}

// Sample virtual row b of scaled logits (chunk_rows_kernel's output: n =
// nch * kp values y and their ids, each chunk's kp sorted by (y
// descending, id ascending) -- the order the row's sort gives): the k best
// by rank, then the softmax, nucleus and draw of finish_sorted (the chunks
// report a NaN through the row's flags instead).  n <= kCandCap
// (kChunkSelfMaxN).  All threads of the block call it.
static_assert(kChunkSelfMaxN <= kCandCap, "virtual row of the one-launch chunked path");
// The loads of the virtual row into sm.x.tk.cand (device-scope atomic
// loads: the device-coherent level, where the chunks' stores are); the
// caller's barrier completes them.
__device__ __forceinline__ void load_vrow_y(RowSmem &sm, const RowArgs &a, int b, const gs_params &p)
{
    const int t = threadIdx.x;
    const int kp = ((int)p.top_k + 3) & ~3;
    const int n = a.cnch * kp;
    const float *vr = a.cvrow + (size_t)b * a.cvld;
    const uint32_t *vi = a.cvidx + (size_t)b * a.cvld;
    uint64_t *cand = sm.x.tk.cand;
    for (int i = t; i < n; i += kThreads) {
        const float y = __uint_as_float(__hip_atomic_load(reinterpret_cast<const uint32_t *>(vr) + i, __ATOMIC_RELAXED,
                                                          __HIP_MEMORY_SCOPE_AGENT));
        cand[i] = cand_of(f2key(y), __hip_atomic_load(vi + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
    }
}
// After load_vrow_y and a barrier; r is the row's draw.
__device__ __forceinline__ void finish_vrow_y(RowSmem &sm, const RowArgs &a, int b, const gs_params &p, float r)
{
    const int t = threadIdx.x;
    const int kp = ((int)p.top_k + 3) & ~3;
    const int n = a.cnch * kp;
    uint64_t *cand = sm.x.tk.cand;
    // Each chunk's kp entries are sorted (descending): an entry's rank is
    // its place in its chunk plus, for every other chunk, the length of the
    // prefix of larger entries there (binary lifting over all chunks at once).
    const int k = (int)p.top_k;
    const int nch = a.cnch;
    uint64_t *top = reinterpret_cast<uint64_t *>(sm.x.tk.u.hist);
    auto rank_all = [&](auto mc) {
        constexpr int kMaxCh = decltype(mc)::value;            // chunks searched (>= nch)
        for (int i = t; i < n; i += kThreads) {
            const int c = i / kp, j = i - c * kp;
            if (j >= k) continue;                               // rank >= j >= k
            const uint64_t me = cand[i];
            int pos[kMaxCh];
#pragma unroll
            for (int c2 = 0; c2 < kMaxCh; c2++) pos[c2] = 0;
#pragma unroll
            for (int step = (int)kChunkMaxK; step >= 1; step >>= 1) {
#pragma unroll
                for (int c2 = 0; c2 < kMaxCh; c2++) {
                    const int q = pos[c2] + step;
                    if (c2 < nch && c2 != c && q <= kp && cand[c2 * kp + q - 1] > me) pos[c2] = q;
                }
            }
            int rk = j;
#pragma unroll
            for (int c2 = 0; c2 < kMaxCh; c2++) rk += pos[c2];
            if (rk < k) top[rk] = me;
        }
    };
    static_assert(kChunkSelfMaxN / kChunkMaxK == 16, "chunk counts of the rank");
    if (nch <= 4) rank_all(std::integral_constant<int, 4>());
    else if (nch <= 8) rank_all(std::integral_constant<int, 8>());
    else rank_all(std::integral_constant<int, 16>());
    __syncthreads();
#ifdef GS_TIMING
    if (t == 0 && b == (int)g_row) g_fails[1006] = (int)__builtin_amdgcn_s_memrealtime();
#endif
    auto yv = [&](int j) { return key2f((uint32_t)(top[j] >> 32)); };
    auto ix = [&](int j) { return ~(uint32_t)top[j]; };
    const int tok = finish_sorted(sm, k, yv, ix, p.top_p, r);
    if (t == 0) store_row(a, b, tok, GS_OK);
}

// The chunked top-k path in one launch, for rows of V % 4 == 0 in 16-byte
// aligned rows: block (c, b) takes chunk c of row b (elements [c0, c1),
// c0 a multiple of 4, at most 32768 of them) through the register path's
// selection -- the chunk's kp best under the sampler's order, penalized
// (window ids inside the chunk) and scaled -- and writes their scaled
// logits y and ids to the chunk's kp slots of virtual row
// b, sorted by (y descending, id ascending).  The last block of row b to
// finish (a device-scope counter) samples the virtual row (finish_vrow_y)
// and clears the counter.  A chunk whose selection
// cannot be decided sets the row's fallback flag: the finishing block then
// samples the whole row.  A NaN in a chunk (or in its penalized values)
// sets the row's NaN flag: the row is an error.
__global__ void __launch_bounds__(kThreads)
chunk_rows_kernel(RowArgs a)
{
    __shared__ RowSmem sm;
    const int c = blockIdx.x, b = blockIdx.y;
    const int t = threadIdx.x;
    const gs_params p = a.params ? a.params[b] : a.uparams;
    if (!chunk_row(p, a.V)) {
        // another small-path row of the batch (per-row params): its first
        // block samples it here, so no separate small-row launch is needed
        if (c == 0 && !is_full_path(p, a.V)) sample_row<kModeSmall>(sm, a, b, kChunkedSelf);
        return;
    }
#ifdef GS_TIMING
#define CR_TS(i) do { if (t == 0 && b == (int)g_row) g_fails[1000 + 8 * c + (i)] = (int)__builtin_amdgcn_s_memrealtime(); } while (0)
#else
#define CR_TS(i) do { } while (0)
#endif
    CR_TS(0);
    // the draw, for the block that finishes the row (loaded now: off the tail)
    const float r = a.u ? a.u[b] : lcg_value(lcg_jump(a.lcg_state, (uint64_t)b));
    const int nch = a.cnch;
    const int kp = ((int)p.top_k + 3) & ~3;
    const int q4 = a.V >> 2;
    const int c0 = 4 * (int)((int64_t)c * q4 / nch);
    const int L = 4 * (int)((int64_t)(c + 1) * q4 / nch) - c0;
    const float *row = a.logits + (size_t)b * a.ld + c0;
    const bool has_pen = p.rep_penalty != 1.0f && a.recent != nullptr;
    int W = 0;
    if (has_pen) {
        W = a.recent_len ? (int)a.recent_len[b] : a.W;
        if (W > a.W) W = a.W;
    }
    // the window id load first, then the chunk's loads (as in the row kernel)
    uint32_t rid = kEmpty;
    if (has_pen && W > 0) rid = ldg(a.recent + (size_t)b * a.ld_recent + min(t, W - 1));
    float4 rv[kRegF4];
    {
        const float4 *r4 = reinterpret_cast<const float4 *>(row);
        const int n4 = L >> 2;
#pragma unroll
        for (int u = 0; u < kRegF4; u++) rv[u] = ldg_nt(r4 + min(u * kThreads + t, n4 - 1));
    }
    reg_clear(sm, has_pen, L);
    if (t == 0) { sm.nuniq = 0; sm.flag_nan = 0; }
    __syncthreads();
    PenLoad pl{kEmpty, 0.0f};
    if (has_pen && t < W) pl.id = rid - (uint32_t)c0;     // ids outside the chunk wrap to >= L: skipped
    int status = GS_OK;
    bool ok;
    CR_TS(1);
    topk_row_reg<true>(sm, row, rv, pl, L, kp, p.temperature, 1.0f, has_pen, p.rep_penalty, 0.0f, &status, &ok);
    CR_TS(2);
    float *vrow = const_cast<float *>(a.cvrow) + (size_t)b * a.cvld + (size_t)c * kp;
    uint32_t *vidx = const_cast<uint32_t *>(a.cvidx) + (size_t)b * a.cvld + (size_t)c * kp;
    // The slots are written with device-scope relaxed atomic stores, which
    // the caches do not hold back (no L2 write-back fence needed); every
    // wave waits for its stores to complete before the barrier, then one
    // thread counts the chunk.  The last block reads the slots with
    // device-scope atomic loads.
    auto put = [&](int i, float y, uint32_t id) {
        __hip_atomic_store(reinterpret_cast<uint32_t *>(vrow) + i, __float_as_uint(y), __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(vidx + i, id, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    };
    if (ok && status == GS_OK) {
        const uint64_t *top = reinterpret_cast<const uint64_t *>(sm.x.tk.u.hist);
        if (t < kp) {
            const uint64_t e = top[t];
            put(t, key2f((uint32_t)(e >> 32)), (uint32_t)c0 + ~(uint32_t)e);
        }
    } else if (t == 0) {
        // bit 0: the whole row must be sampled; bit 1: a NaN (the row is an error)
        atomicOr(a.csync + 2 * (size_t)b + 1, ok ? 2u : 1u);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_s_waitcnt(0 | (0x7 << 4) | (0xf << 8));   // vmcnt(0): this wave's stores are complete
    __syncthreads();
    if (t == 0) sm.clast = atomicAdd(a.csync + 2 * (size_t)b, 1u) == (uint32_t)(nch - 1) ? 1 : 0;
    __syncthreads();
    CR_TS(3);
    if (!sm.clast) return;
    // The slot loads below are device-scope atomic loads: they read the
    // device-coherent level, where the other chunks' agent-scope stores
    // (complete before their counter adds: the vmcnt(0) wait above) already
    // are.  The fence keeps them after the counter's result.  (A device-scope
    // acquire fence here, which on gfx950 also invalidates the caches, was
    // measured: C2 21.6 -> 38.2 us per batch.)
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    CR_TS(4);
    // Every thread reads the flags (final: every chunk set its bits before
    // its counter add); the slots are loaded in the same round trip, and
    // used when no flag is set.
    const uint32_t flags = __hip_atomic_load(a.csync + 2 * (size_t)b + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    load_vrow_y(sm, a, b, p);
    __syncthreads();
    if (t == 0) {
        __hip_atomic_store(a.csync + 2 * (size_t)b, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(a.csync + 2 * (size_t)b + 1, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    if (flags & 2u) {
        if (t == 0) store_row(a, b, 0, GS_ERR_NAN);   // a NaN anywhere: the reference's sort panics
    } else if (flags & 1u) {
        sample_row<kModeSmall>(sm, a, b, 0);
    } else {
        finish_vrow_y(sm, a, b, p, r);
    }
    CR_TS(5);
}

// Pass 2: sample virtual row b (its width nch * kp is a multiple of 4 and
// the row is 16-byte aligned; no penalty: the values are already penalized):
// the register path, else the general top-k paths; the token is mapped
// back through vidx.  All threads of the block call it.
__device__ void finish_virtual_row(RowSmem &sm, const RowArgs &a, int b, const gs_params &p, const float *vrow,
                                   const uint32_t *vidx, size_t vld, int nch)
{
    const int t = threadIdx.x;
    const float *vr = vrow + (size_t)b * vld;
    const int V2 = nch * (((int)p.top_k + 3) & ~3);
    float4 rv[kRegF4];
    {
        const float4 *r4 = reinterpret_cast<const float4 *>(vr);
        const int n4 = V2 >> 2;
#pragma unroll
        for (int u = 0; u < kRegF4; u++) rv[u] = ldg_nt(r4 + min(u * kThreads + t, n4 - 1));
    }
    reg_clear(sm, false, V2);
    if (t == 0) { sm.nuniq = 0; sm.flag_nan = 0; }
    __syncthreads();
    const PenLoad pl{kEmpty, 0.0f};
    const float r = a.u ? a.u[b] : lcg_value(lcg_jump(a.lcg_state, (uint64_t)b));
    const int k = (int)p.top_k;
    int status = GS_OK;
    bool ok;
    int tok = topk_row_reg(sm, vr, rv, pl, V2, k, p.temperature, p.top_p, false, 1.0f, r, &status, &ok);
    if (!ok) tok = topk_row<true>(sm, vr, V2, k, p.temperature, p.top_p, false, r, true, &status, &ok);
    if (!ok) tok = topk_row<false>(sm, vr, V2, k, p.temperature, p.top_p, false, r, true, &status, &ok);
    if (t == 0) store_row(a, b, status == GS_OK ? (int)ldg(vidx + (size_t)b * vld + tok) : 0, status);
}

__global__ void __launch_bounds__(kThreads)
split_finish_kernel(RowArgs a, const float *vrow, const uint32_t *vidx, size_t vld, int nch)
{
    __shared__ RowSmem sm;
    finish_virtual_row(sm, a, blockIdx.x, a.uparams, vrow, vidx, vld, nch);
}

hipError_t launch_sample_rows(const RowArgs &a, int B, hipStream_t st)
{
    // with per-row params a batch may hold rows of both kinds
    const bool full = a.params || is_full_path(a.uparams, a.V);
    const bool small = a.params || !full;
    if (small) hipLaunchKernelGGL(sample_rows_kernel<kModeSmall>, dim3(B), dim3(kThreads), 0, st, a);
    if (full) hipLaunchKernelGGL(sample_rows_kernel<kModeBins>, dim3(B), dim3(kThreads), 0, st, a);
    return hipGetLastError();
}
hipError_t launch_sample_rows_forked(const RowArgs &a, int B, hipStream_t st, hipStream_t side, hipEvent_t fork,
                                    hipEvent_t join)
{
    // the full-vocabulary rows on st; the small-path rows on `side` at the
    // same time (the CUs the full rows leave idle); st waits for both
    if (hipEventRecord(fork, st) != hipSuccess || hipStreamWaitEvent(side, fork, 0) != hipSuccess)
        return hipGetLastError();
    hipLaunchKernelGGL(sample_rows_kernel<kModeBins>, dim3(B), dim3(kThreads), 0, st, a);
    hipLaunchKernelGGL(sample_rows_kernel<kModeSmall>, dim3(B), dim3(kThreads), 0, side, a);
    if (hipEventRecord(join, side) != hipSuccess || hipStreamWaitEvent(st, join, 0) != hipSuccess)
        return hipGetLastError();
    return hipGetLastError();
}
hipError_t launch_detail_rows(const RowArgs &a, int B, hipStream_t st)
{
    hipLaunchKernelGGL(sample_rows_kernel<kModeDetail>, dim3(B), dim3(kThreads), 0, st, a);
    return hipGetLastError();
}
hipError_t launch_reg_row(const RowArgs &a, hipStream_t st)
{
    hipLaunchKernelGGL(reg_row_kernel, dim3(1), dim3(kThreads), 0, st, a);
    return hipGetLastError();
}
bool reg_row_fits(const gs_params &p, size_t V, const void *row)
{
    if (V < 2 || (V & 3) != 0 || V > (size_t)(kThreads * 4 * kRegF4) || ((uintptr_t)row & 15u) != 0) return false;
    if (p.temperature <= 0.0f) return true;                  // greedy (a NaN T is not <= 0)
    return p.temperature > 0.0f && p.temperature < INFINITY && p.top_k > 0 && (size_t)p.top_k < V &&
           p.top_k <= (uint32_t)kMaxTopK;
}
bool split_fits(const gs_params &p, size_t V)
{
    if (!(p.temperature > 0.0f && p.temperature < INFINITY)) return false;
    if (V <= kRegMaxV || V > (size_t)0x7fffffff) return false;
    if (p.top_k == 0 || (size_t)p.top_k >= V) return false;
    const size_t kp = ((size_t)p.top_k + 3) & ~(size_t)3;
    return kp <= (size_t)kSplitMaxKp && (V / kSplitL) * kp <= kSplitMaxWidth;
}
size_t split_width(const gs_params &p, size_t V)
{
    return (V / kSplitL) * (((size_t)p.top_k + 3) & ~(size_t)3);
}
hipError_t launch_split(const RowArgs &a, int B, float *vrow, uint32_t *vidx, hipStream_t st)
{
    const int nch = a.V / kSplitL;
    const int kp = ((int)a.uparams.top_k + 3) & ~3;
    const size_t vld = (size_t)nch * kp;
    hipLaunchKernelGGL(split_select_kernel, dim3(nch, B), dim3(kSplitThreads), 0, st, a, nch, kp, vrow, vidx, vld);
    hipLaunchKernelGGL(split_finish_kernel, dim3(B), dim3(kThreads), 0, st, a, (const float *)vrow,
                       (const uint32_t *)vidx, vld, nch);
    return hipGetLastError();
}
hipError_t launch_chunked(RowArgs a, int B, float *vrow, uint32_t *vidx, uint32_t *csync, hipStream_t st)
{
    const int nch = chunk_count((size_t)a.V);
    const size_t vld = chunk_stride((size_t)a.V);
    a.cvrow = vrow;
    a.cvidx = vidx;
    a.cvld = vld;
    a.cnch = nch;
    if (csync) {
        // one launch samples the chunked rows and the batch's other
        // small-path rows; with per-row params the full-vocabulary kernels
        // follow for the rest
        a.chunked = kChunkedSelf;
        a.csync = csync;
        hipLaunchKernelGGL(chunk_rows_kernel, dim3(nch, B), dim3(kThreads), 0, st, a);
        if (a.params) hipLaunchKernelGGL(sample_rows_kernel<kModeBins>, dim3(B), dim3(kThreads), 0, st, a);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(chunk_topk_kernel, dim3(nch, B), dim3(kThreads), 0, st, a, nch, vrow, vidx, vld);
    // the virtual rows go through the small kernel (in order: a fork and
    // join of streams costs more than the short small-row kernel would gain)
    a.chunked = kChunkedX;
    return launch_sample_rows(a, B, st);
}
hipError_t launch_window_push(uint32_t *win, int B, size_t ld, int W, size_t pos,
                              const uint32_t *tok, hipStream_t st)
{
    hipLaunchKernelGGL(window_push_kernel, dim3((B + 255) / 256), dim3(256), 0, st, win, B, ld, W, pos, tok);
    return hipGetLastError();
}
hipError_t launch_writeback(float *logits, int B, int V, size_t ld, const gs_params *params, const gs_params &up,
                           const uint32_t *recent, size_t ld_recent, const uint32_t *recent_len, int W,
                           hipStream_t st)
{
    const int chunks = (V + kMutChunk - 1) / kMutChunk;
    hipLaunchKernelGGL(writeback_kernel, dim3(chunks, B), dim3(256), 0, st, logits, ld, V, params, up, recent,
                       ld_recent, recent_len, W);
    return hipGetLastError();
}
hipError_t launch_synth(float *out, int B, int V, size_t ld, uint64_t seed, uint64_t c0, float sigma,
                        hipStream_t st)
{
    size_t n = (size_t)B * V;
    int blocks = (int)((n + 255) / 256);
    if (blocks > 65536) blocks = 65536;
    hipLaunchKernelGGL(synth_kernel, dim3(blocks), dim3(256), 0, st, out, B, V, ld, seed, c0, sigma);
    return hipGetLastError();
}
} // namespace gs
