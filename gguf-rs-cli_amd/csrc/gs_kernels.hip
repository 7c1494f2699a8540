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
#include "gs_block.hpp"
#include "gs_kernels.hpp"

namespace gs {

constexpr int kHashSlots = 2 * kMaxWindow;     // open addressing, load <= 1/2
constexpr int kHistBins = 4096;                 // 12-bit radix digits
constexpr int kCandCap = 2048;                  // LDS candidate capacity
constexpr uint32_t kEmpty = 0xffffffffu;

struct RowSmem {
    uint32_t hkey[kHashSlots];                  // penalized ids
    uint32_t hval[kHashSlots];                  // occurrence count, then f32 bits of the penalized logit
    union {
        uint32_t hist[kHistBins];
        uint32_t wcnt[kWaves * 256];            // radix sort: per-wave digit counts
        float ev[kHistBins];                    // candidates: exp values
    } u;
    uint64_t cand[kCandCap];                    // (key << 32) | ~idx, sorted descending
    SeqSmem seq;
    uint32_t base[256];
    int ncand;
    int nuniq;
    int flag_nan;
    uint32_t sel_prefix;
    uint32_t sel_above;
    uint32_t red_u32[kWaves];
    float red_f32[kWaves];
    int red_i32[kWaves];
    int tok;
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

// Build the penalty table for this row.  Returns the number of unique ids.
__device__ void build_penalty(RowSmem &sm, const float *row, int V, const uint32_t *rec, int W,
                              float T, float pen)
{
    const int t = threadIdx.x;
    for (int i = t; i < kHashSlots; i += kThreads) { sm.hkey[i] = kEmpty; sm.hval[i] = 0; }
    if (t == 0) sm.nuniq = 0;
    __syncthreads();
    for (int j = t; j < W; j += kThreads) {
        uint32_t id = rec[j];
        if ((int)id >= V || id == kEmpty) continue;   // src/sampler.rs:26 logits.get_mut
        uint32_t h = hash_slot(id);
        for (;;) {
            uint32_t prev = atomicCAS(&sm.hkey[h], kEmpty, id);
            if (prev == kEmpty || prev == id) { atomicAdd(&sm.hval[h], 1u); break; }
            h = (h + 1) & (kHashSlots - 1);
        }
    }
    __syncthreads();
    for (int i = t; i < kHashSlots; i += kThreads) {
        uint32_t id = sm.hkey[i];
        if (id != kEmpty) {
            float l = penalize(row[id], sm.hval[i], pen);
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
// Softmax, nucleus and draw over n candidates sorted descending.  yv(j) gives
// the scaled logit of candidate j, idx(j) its token id.  Mirrors
// src/sampler.rs:53-78 exactly (block_seqsum reproduces every f32 sum).
template <class YV, class IX>
__device__ int finish_sorted(RowSmem &sm, int n, YV yv, IX idx, float top_p, float r)
{
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
// Bitonic sort of sm.cand[0..P) descending, P a power of two.
__device__ void bitonic_desc(RowSmem &sm, int P)
{
    for (int k = 2; k <= P; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = threadIdx.x; i < P; i += kThreads) {
                int l = i ^ j;
                if (l > i) {
                    uint64_t a = sm.cand[i], b = sm.cand[l];
                    bool desc = (i & k) == 0;
                    if (desc ? (a < b) : (a > b)) { sm.cand[i] = b; sm.cand[l] = a; }
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
    uint32_t incl = v;
    for (int d = 1; d < 64; d <<= 1) {
        uint32_t o = __shfl_up(incl, d, 64);
        if (lane >= d) incl += o;
    }
    if (lane == 63) sm.red_u32[w] = incl;
    __syncthreads();
    uint32_t pre = 0, all = 0;
    for (int i = 0; i < kWaves; i++) { if (i < w) pre += sm.red_u32[i]; all += sm.red_u32[i]; }
    __syncthreads();
    *tot = all;
    return pre + incl - v;
}

// --------------------------------------------------------------------------
// Top-k path.  Returns the token (or sets *status).
__device__ int topk_row(RowSmem &sm, const float *row, int V, int k, float T, float top_p,
                        bool has_pen, float r, int *status)
{
    const int t = threadIdx.x;
    // Radix select over the 32-bit keys in 3 levels: 12, 12, 8 bits.
    uint32_t prefix = 0;        // key bits above `shift` fixed so far
    int shift = 32;
    uint32_t above = 0;         // elements with key strictly above the in-play range
    int nan = 0;
    const int widths[3] = {12, 12, 8};
    int level = 0;
    bool fits = false;
    for (level = 0; level < 3; level++) {
        const int wbits = widths[level];
        const int nsh = shift - wbits;
        const uint32_t nbins = 1u << wbits;
        for (uint32_t i = t; i < nbins; i += kThreads) sm.u.hist[i] = 0;
        __syncthreads();
        for (int i = t; i < V; i += kThreads) {
            float y = row[i] / T;
            if (level == 0) nan |= isnan(y);
            uint32_t key = f2key(y);
            if (shift == 32 || (key >> shift) == prefix)
                atomicAdd(&sm.u.hist[(key >> nsh) & (nbins - 1)], 1u);
        }
        __syncthreads();
        if (has_pen) {
            // Move penalized ids from their raw bin to their penalized bin.
            for (int s = t; s < kHashSlots; s += kThreads) {
                uint32_t id = sm.hkey[s];
                if (id == kEmpty) continue;
                uint32_t kr = f2key(row[id] / T);
                uint32_t kp = f2key(__uint_as_float(sm.hval[s]) / T);
                if (shift == 32 || (kr >> shift) == prefix) atomicSub(&sm.u.hist[(kr >> nsh) & (nbins - 1)], 1u);
                if (shift == 32 || (kp >> shift) == prefix) atomicAdd(&sm.u.hist[(kp >> nsh) & (nbins - 1)], 1u);
            }
            __syncthreads();
        }
        if (level == 0 && block_or(nan, sm)) { *status = GS_ERR_NAN; return 0; }
        // Find the bin holding the k-th largest: scan bins from the top.
        // Thread t owns bins [c*t, c*t+c) counted from the top.
        const uint32_t per = (nbins + kThreads - 1) / kThreads;
        uint32_t mine = 0;
        for (uint32_t q = 0; q < per; q++) {
            uint32_t bt = t * per + q;            // index from the top
            if (bt < nbins) mine += sm.u.hist[nbins - 1 - bt];
        }
        uint32_t tot;
        uint32_t ex = block_excl_u32(mine, &tot, sm);
        const uint32_t need = (uint32_t)k - above;
        if (ex < need && ex + mine >= need) {
            uint32_t c = ex;
            for (uint32_t q = 0; q < per; q++) {
                uint32_t bt = t * per + q;
                uint32_t b = nbins - 1 - bt;
                uint32_t h = sm.u.hist[b];
                if (c + h >= need) { sm.sel_prefix = b; sm.sel_above = c; break; }
                c += h;
            }
        }
        __syncthreads();
        const uint32_t b = sm.sel_prefix;
        const uint32_t in_bin = sm.u.hist[b];
        above += sm.sel_above;
        prefix = (shift == 32 ? 0u : (prefix << wbits)) | b;
        shift = nsh;
        __syncthreads();
        if (above + in_bin <= (uint32_t)kCandCap) { fits = true; break; }
    }
    // Collect candidates: key >> shift >= prefix (when the tie range fits),
    // else key > K* plus the first (k - above) ids equal to K* in index order.
    if (t == 0) sm.ncand = 0;
    __syncthreads();
    const uint32_t kstar = prefix;  // valid as a full key only when !fits (shift == 0)
    for (int i = t; i < V; i += kThreads) {
        float y = row[i] / T;
        uint32_t key = f2key(y);
        bool take = fits ? ((key >> shift) >= prefix) : (key > kstar);
        if (take && !(has_pen && hash_find(sm, (uint32_t)i) >= 0)) {
            int slot = atomicAdd(&sm.ncand, 1);
            sm.cand[slot] = cand_of(key, (uint32_t)i);
        }
    }
    if (has_pen) {
        for (int s = t; s < kHashSlots; s += kThreads) {
            uint32_t id = sm.hkey[s];
            if (id == kEmpty) continue;
            uint32_t key = f2key(__uint_as_float(sm.hval[s]) / T);
            bool take = fits ? ((key >> shift) >= prefix) : (key > kstar);
            if (take) { int slot = atomicAdd(&sm.ncand, 1); sm.cand[slot] = cand_of(key, id); }
        }
    }
    __syncthreads();
    if (!fits) {
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
                sm.cand[slot] = cand_of(kstar, (uint32_t)i);
            }
            taken += tot;
        }
        __syncthreads();
    }
    const int nc = sm.ncand;
    int P = 1;
    while (P < nc) P <<= 1;
    for (int i = nc + t; i < P; i += kThreads) sm.cand[i] = 0ull;
    __syncthreads();
    bitonic_desc(sm, P);
    const int n = k;   // nc >= k by construction
    auto yv = [&](int j) { return key2f((uint32_t)(sm.cand[j] >> 32)); };
    auto ix = [&](int j) { return ~(uint32_t)sm.cand[j]; };
    *status = GS_OK;
    return finish_sorted(sm, n, yv, ix, top_p, r);
}

// --------------------------------------------------------------------------
// Full-vocabulary path: stable LSD radix sort of (~key, index) in scratch.
// ~key ascending == key descending; stability keeps equal keys in index order.
__device__ int full_row(RowSmem &sm, const float *row, int V, int keep, float T, float top_p,
                        bool has_pen, float r, uint32_t *kA, uint32_t *iA, uint32_t *kB,
                        uint32_t *iB, int *status)
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
        for (int i = t; i < 256; i += kThreads) sm.base[i] = 0;
        __syncthreads();
        for (int i = t; i < V; i += kThreads) atomicAdd(&sm.base[(src_k[i] >> sh) & 255u], 1u);
        __syncthreads();
        if (t == 0) {
            uint32_t run = 0;
            for (int d = 0; d < 256; d++) { uint32_t c = sm.base[d]; sm.base[d] = run; run += c; }
        }
        __syncthreads();
        constexpr int kSlots = 4;
        for (int tile = 0; tile < V; tile += kThreads * kSlots) {
            for (int i = t; i < kWaves * 256; i += kThreads) sm.u.wcnt[i] = 0;
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
                uint32_t before = sm.u.wcnt[w * 256 + d];
                rnk[q] = before + (uint32_t)__popcll(peers & lanemask_lt());
                // All lanes have read the counter before the leader bumps it
                // (one wave executes in lockstep; the barrier makes it explicit).
                __builtin_amdgcn_wave_barrier();
                if (val[q] && (peers & lanemask_lt()) == 0)
                    sm.u.wcnt[w * 256 + d] = before + (uint32_t)__popcll(peers);
                __builtin_amdgcn_wave_barrier();
            }
            __syncthreads();
            for (int d = t; d < 256; d += kThreads) {
                uint32_t run = sm.base[d];
                for (int ww = 0; ww < kWaves; ww++) {
                    uint32_t c = sm.u.wcnt[ww * 256 + d];
                    sm.u.wcnt[ww * 256 + d] = run;
                    run += c;
                }
                sm.base[d] = run;
            }
            __syncthreads();
            for (int q = 0; q < kSlots; q++) {
                if (!val[q]) continue;
                uint32_t dst = sm.u.wcnt[w * 256 + dig[q]] + rnk[q];
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
    return finish_sorted(sm, keep, yv, ix, top_p, r);
}

// --------------------------------------------------------------------------
__global__ void __launch_bounds__(kThreads)
sample_rows_kernel(RowArgs a)
{
    __shared__ RowSmem sm;
    const int b = blockIdx.x;
    const int t = threadIdx.x;
    const int V = a.V;
    const float *row = a.logits + (size_t)b * a.ld;
    gs_params p = a.params ? a.params[b] : a.uparams;
    if (t == 0) sm.flag_nan = 0;

    int tok = 0, status = GS_OK;
    const bool has_pen = (p.rep_penalty != 1.0f) && a.recent != nullptr;
    int W = 0;
    if (has_pen) {
        W = a.recent_len ? (int)a.recent_len[b] : a.W;
        if (W > a.W) W = a.W;
    }
    __syncthreads();
    if (has_pen) build_penalty(sm, row, V, a.recent + (size_t)b * a.ld_recent, W,
                               p.temperature > 0.0f ? p.temperature : 1.0f, p.rep_penalty);
    const bool pen_active = has_pen;

    // The uniform draw for this row (only consumed if T > 0).
    float r = 0.0f;
    if (a.u) r = a.u[b];
    else r = lcg_value(lcg_jump(a.lcg_state, (uint64_t)b));

    if (V == 0) {
        tok = 0;
        status = p.temperature > 0.0f ? GS_ERR_EMPTY : GS_OK;
    } else if (!(p.temperature > 0.0f)) {
        // src/sampler.rs:39: `if temperature <= 0.0` -- a NaN temperature is
        // not <= 0, so it falls through to the division below.
        if (p.temperature <= 0.0f) greedy_row(sm, row, V, pen_active, &tok, &status);
        else {
            // T is NaN: every scaled logit is NaN; sort panics for V > 1.
            tok = 0;
            status = V > 1 ? GS_ERR_NAN : GS_OK;
        }
    } else if (V == 1) {
        tok = 0;   // a single pair: no comparison can panic; token 0.
    } else {
        if (sm.flag_nan) status = GS_ERR_NAN;
        else {
            const int keep = (p.top_k > 0 && p.top_k < (uint32_t)V) ? (int)p.top_k : V;
            if (keep < V && keep <= kMaxTopK)
                tok = topk_row(sm, row, V, keep, p.temperature, p.top_p, pen_active, r, &status);
            else {
                const size_t off = (size_t)b * a.scratch_stride;
                tok = full_row(sm, row, V, keep, p.temperature, p.top_p, pen_active, r,
                               a.scratch + off, a.scratch + off + V,
                               a.scratch + off + 2 * (size_t)V, a.scratch + off + 3 * (size_t)V,
                               &status);
            }
        }
    }
    if (t == 0) {
        a.tokens[b] = (uint32_t)tok;
        if (a.status) a.status[b] = status;
    }
}

__global__ void window_push_kernel(uint32_t *win, int B, size_t ld, int W, size_t pos,
                                   const uint32_t *tok)
{
    int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b < B) win[(size_t)b * ld + (pos % (size_t)W)] = tok[b];
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

// Launch wrappers (host side of this translation unit).
namespace gs {
hipError_t launch_sample_rows(const RowArgs &a, int B, hipStream_t st)
{
    hipLaunchKernelGGL(sample_rows_kernel, dim3(B), dim3(kThreads), 0, st, a);
    return hipGetLastError();
}
hipError_t launch_window_push(uint32_t *win, int B, size_t ld, int W, size_t pos,
                              const uint32_t *tok, hipStream_t st)
{
    hipLaunchKernelGGL(window_push_kernel, dim3((B + 255) / 256), dim3(256), 0, st, win, B, ld, W, pos, tok);
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
