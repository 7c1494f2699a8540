// gs_block.hpp -- block-level building blocks (1024 threads = 16 wave64).
#pragma once
#include "gs_device.hpp"

namespace gs {

constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;

__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
__device__ __forceinline__ int wave_id() { return threadIdx.x >> 6; }
__device__ __forceinline__ uint64_t lanemask_lt() { return (1ull << lane_id()) - 1ull; }

// ---------------------------------------------------------------------------
// Exact emulation of a sequential f32 running sum.
//
// The reference accumulates in f32, one element at a time, in sorted order
// (src/sampler.rs:54 softmax sum, :61-63 nucleus cumsum, :67 renormalising sum,
// :74-75 multinomial CDF).  Sequential rounding is order dependent, so a tree
// reduction would not reproduce it.  It can still be evaluated in parallel:
//
// While the running sum s stays inside one binade [2^e, 2^(e+1)), every
// partial sum is an integer multiple of g = 2^(e-23), and
//     RN(s + a) = s + g * RNE_g(a)
// where RNE_g(a) is a rounded to an integer count of g.  Rounding ties (a an
// odd multiple of g/2) go to the even mantissa, so they depend only on the
// parity of s/g.  Hence, inside a binade, the sum is a prefix sum of integers
// whose elements are functions of one parity bit: f(p) = K + ((p + K) & 1) for
// a tie, f(p) = k otherwise.  Such functions compose associatively,
//     (f;h)(p) = f(p) + h((p + f(p)) & 1),
// so a block-wide scan gives every partial sum exactly.  The first element
// whose partial sum would leave the binade is evaluated with one real f32
// add, and the scan restarts from there.  The number of restarts is bounded
// by the number of binades the sum passes through (about 30 for p-sums).
//
// Subnormal sums need no special case: [0, 2^-125) has the single grid 2^-149,
// which is the e = -126 case.
// ---------------------------------------------------------------------------
struct ParFn { uint32_t f0, f1; };               // increment for parity 0 / 1
constexpr uint32_t kSat = 1u << 25;              // saturate: past any crossing

__device__ __forceinline__ uint32_t sat_add(uint32_t a, uint32_t b)
{
    uint32_t s = a + b;
    return s > kSat ? kSat : s;
}
// Branchless select (a ternary on the two fields gets lowered to an indexed
// load from a stack copy, which the backend places in LDS).
__device__ __forceinline__ uint32_t par_apply(const ParFn &f, uint32_t p)
{
    return f.f0 ^ ((f.f0 ^ f.f1) & (0u - (p & 1u)));
}
__device__ __forceinline__ ParFn par_compose(const ParFn &a, const ParFn &b)
{
    ParFn r;
    r.f0 = sat_add(a.f0, par_apply(b, (a.f0) & 1u));
    r.f1 = sat_add(a.f1, par_apply(b, (1u + a.f1) & 1u));
    return r;
}

// Binade exponent used for the grid of s (s >= 0, finite); subnormals -> -126.
__device__ __forceinline__ int grid_exp(float s)
{
    int e = (int)((__float_as_uint(s) >> 23) & 0xff) - 127;
    return e < -126 ? -126 : e;
}

// Increment function of summand a at grid exponent e.
__device__ __forceinline__ ParFn elem_fn(float a, int e)
{
    const float m = ldexpf(a, 23 - e);     // exact power-of-two scaling
    const bool big = !(m < (float)kSat);
    const float fl = floorf(m);
    const float fr = m - fl;               // exact
    const uint32_t K = big ? 0u : (uint32_t)fl;
    const uint32_t k = K + (fr > 0.5f ? 1u : 0u);
    const bool tie = fr == 0.5f;
    ParFn f;
    f.f0 = big ? kSat : (tie ? K + (K & 1u) : k);
    f.f1 = big ? kSat : (tie ? K + ((K + 1u) & 1u) : k);
    return f;
}

// Wave64 inclusive scan of ParFn with DPP moves (no LDS): Hillis-Steele
// inside each 16-lane row (row_shr 1, 2, 4, 8), then row_bcast:15 and
// row_bcast:31 across rows.  The operator is not commutative, so the value
// from the lower lane is always the left operand.
template <int CTRL>
__device__ __forceinline__ uint32_t dpp_mov(uint32_t v)
{
    return (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, CTRL, 0xf, 0xf, false);
}
// Wave64 inclusive sums with DPP moves (no LDS round trips): row_shr 1, 2,
// 4, 8 inside each 16-lane row (lanes without a source read 0), then
// row_bcast:15 and row_bcast:31 across rows.
__device__ __forceinline__ uint32_t wave_incl_u32(uint32_t v)
{
    const int lane = lane_id();
    v += dpp_mov<0x111>(v);
    v += dpp_mov<0x112>(v);
    v += dpp_mov<0x114>(v);
    v += dpp_mov<0x118>(v);
    uint32_t o = dpp_mov<0x142>(v);
    if ((lane & 31) >= 16) v += o;
    o = dpp_mov<0x143>(v);
    if (lane >= 32) v += o;
    return v;
}
template <int CTRL>
__device__ __forceinline__ double dpp_mov_f64(double v)
{
    const uint64_t u = (uint64_t)__double_as_longlong(v);
    const uint32_t lo = dpp_mov<CTRL>((uint32_t)u), hi = dpp_mov<CTRL>((uint32_t)(u >> 32));
    return __longlong_as_double((long long)(((uint64_t)hi << 32) | lo));
}
__device__ __forceinline__ double wave_incl_f64(double v)
{
    const int lane = lane_id();
    v += dpp_mov_f64<0x111>(v);      // (a lane without a source reads +0.0)
    v += dpp_mov_f64<0x112>(v);
    v += dpp_mov_f64<0x114>(v);
    v += dpp_mov_f64<0x118>(v);
    double o = dpp_mov_f64<0x142>(v);
    if ((lane & 31) >= 16) v += o;
    o = dpp_mov_f64<0x143>(v);
    if (lane >= 32) v += o;
    return v;
}
template <int CTRL>
__device__ __forceinline__ void dpp_step(ParFn &v, bool take)
{
    ParFn o;
    o.f0 = dpp_mov<CTRL>(v.f0);
    o.f1 = dpp_mov<CTRL>(v.f1);
    if (take) v = par_compose(o, v);
}
__device__ __forceinline__ ParFn wave_scan_incl(ParFn v)
{
    const int lane = lane_id(), rl = lane & 15;
    dpp_step<0x111>(v, rl >= 1);      // row_shr:1
    dpp_step<0x112>(v, rl >= 2);      // row_shr:2
    dpp_step<0x114>(v, rl >= 4);      // row_shr:4
    dpp_step<0x118>(v, rl >= 8);      // row_shr:8
    dpp_step<0x142>(v, (lane & 31) >= 16);   // row_bcast:15
    dpp_step<0x143>(v, lane >= 32);          // row_bcast:31
    return v;
}

// Wave64 inclusive add-scan of u32 with DPP moves (same pattern as above).
__device__ __forceinline__ uint32_t wave_scan_add(uint32_t v)
{
    const int lane = lane_id(), rl = lane & 15;
    uint32_t o;
    o = dpp_mov<0x111>(v); if (rl >= 1) v += o;
    o = dpp_mov<0x112>(v); if (rl >= 2) v += o;
    o = dpp_mov<0x114>(v); if (rl >= 4) v += o;
    o = dpp_mov<0x118>(v); if (rl >= 8) v += o;
    o = dpp_mov<0x142>(v); if ((lane & 31) >= 16) v += o;
    o = dpp_mov<0x143>(v); if (lane >= 32) v += o;
    return v;
}

// Wave64 sum of a u64, returned in every lane (the inclusive DPP scan's
// last lane).
template <int CTRL>
__device__ __forceinline__ uint64_t dpp_mov_u64(uint64_t v)
{
    return ((uint64_t)dpp_mov<CTRL>((uint32_t)(v >> 32)) << 32) | dpp_mov<CTRL>((uint32_t)v);
}
__device__ __forceinline__ uint64_t wave_sum_u64(uint64_t v)
{
    const int lane = lane_id();
    v += dpp_mov_u64<0x111>(v);
    v += dpp_mov_u64<0x112>(v);
    v += dpp_mov_u64<0x114>(v);
    v += dpp_mov_u64<0x118>(v);
    uint64_t o = dpp_mov_u64<0x142>(v);
    if ((lane & 31) >= 16) v += o;
    o = dpp_mov_u64<0x143>(v);
    if (lane >= 32) v += o;
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, 63);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(v >> 32), 63);
    return ((uint64_t)hi << 32) | lo;
}

// Wave64 maximum / minimum of a u32, returned in every lane.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v)
{
    const int lane = lane_id(), rl = lane & 15;
    uint32_t o;
    o = dpp_mov<0x111>(v); if (rl >= 1) v = max(v, o);
    o = dpp_mov<0x112>(v); if (rl >= 2) v = max(v, o);
    o = dpp_mov<0x114>(v); if (rl >= 4) v = max(v, o);
    o = dpp_mov<0x118>(v); if (rl >= 8) v = max(v, o);
    o = dpp_mov<0x142>(v); if ((lane & 31) >= 16) v = max(v, o);
    o = dpp_mov<0x143>(v); if (lane >= 32) v = max(v, o);
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v)
{
    return ~wave_max_u32(~v);
}

// Integer increment of summand a at grid exponent e (capped at kSat), and
// whether it is an exact rounding tie.
__device__ __forceinline__ uint32_t elem_inc(float a, int e, bool *tie)
{
    const float m = ldexpf(a, 23 - e);
    const bool big = !(m < (float)kSat);
    const float fl = floorf(m);
    const float fr = m - fl;
    *tie = !big && fr == 0.5f;
    return big ? kSat : (uint32_t)fl + (fr > 0.5f ? 1u : 0u);
}

struct SeqSmem {
    ParFn wave_tot[kWaves];
    int first;
    float s;
    int start;
};

// Block-wide exclusive scan of ParFn in thread order; returns the exclusive
// prefix for this thread.
__device__ __forceinline__ ParFn block_scan_excl(ParFn v, SeqSmem &sm)
{
    const int lane = lane_id(), w = wave_id();
    ParFn incl = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        ParFn o;
        o.f0 = __shfl_up(incl.f0, d, 64);
        o.f1 = __shfl_up(incl.f1, d, 64);
        if (lane >= d) incl = par_compose(o, incl);
    }
    if (lane == 63) sm.wave_tot[w] = incl;
    __syncthreads();
    ParFn pre = {0u, 0u};
    for (int i = 0; i < w; i++) pre = par_compose(pre, sm.wave_tot[i]);
    ParFn ex;
    ex.f0 = __shfl_up(incl.f0, 1, 64);
    ex.f1 = __shfl_up(incl.f1, 1, 64);
    if (lane == 0) { ex.f0 = 0u; ex.f1 = 0u; }
    return par_compose(pre, ex);
}

// Sequential accumulation s_{j+1} = RN(s_j + a(j)), j in [0, n), s_0 = s_init,
// stopping at the first j with pred(s_{j+1}).  Returns that j (or n) and the
// running sum at the stop (or at the end) in *s_out.  `a` must be a pure
// function of j; it is evaluated by several threads.  All threads must call.
constexpr int kSeqPer = 4;                        // elements per thread per tile
template <class LoadA, class Pred>
__device__ int block_seqsum(LoadA a, int n, float s_init, Pred pred, float *s_out, SeqSmem &sm)
{
    const int t = threadIdx.x;
    float s = s_init;
    int pos = 0;
    // Leading steps from s == 0 are done one at a time (0 + a == a exactly).
    while (pos < n && s == 0.0f) {
        s = s + a(pos);
        if (pred(s)) { *s_out = s; return pos; }
        pos++;
    }
    const int tile = kThreads * kSeqPer;
    while (pos < n) {
        const int tend = min(pos + tile, n);
        float av[kSeqPer];
#pragma unroll
        for (int q = 0; q < kSeqPer; q++) {
            int j = pos + t * kSeqPer + q;
            av[q] = (j < tend) ? a(j) : 0.0f;
        }
        int start = pos;
        for (;;) {
            const int e = grid_exp(s);
            const uint32_t M = (uint32_t)ldexpf(s, 23 - e);   // exact, < 2^24
            ParFn fn[kSeqPer];
            ParFn loc = {0u, 0u};
#pragma unroll
            for (int q = 0; q < kSeqPer; q++) {
                int j = pos + t * kSeqPer + q;
                if (j >= start && j < tend) fn[q] = elem_fn(av[q], e);
                else { fn[q].f0 = 0u; fn[q].f1 = 0u; }
                loc = par_compose(loc, fn[q]);
            }
            if (t == 0) sm.first = 0x7fffffff;
            ParFn ex = block_scan_excl(loc, sm);   // contains a barrier
            // Walk my elements.
            const uint32_t pM = M & 1u;
            uint32_t before = par_apply(ex, pM);
            int my_first = 0x7fffffff;
#pragma unroll
            for (int q = 0; q < kSeqPer; q++) {
                int j = pos + t * kSeqPer + q;
                uint32_t inc = par_apply(fn[q], (pM + before) & 1u);
                uint32_t after = sat_add(before, inc);
                if (j >= start && j < tend && my_first == 0x7fffffff) {
                    bool cross = (M + after) >= (1u << 24);
                    bool stop = !cross && pred(ldexpf((float)(M + after), e - 23));
                    if (cross || stop) my_first = j;
                }
                before = after;
            }
            if (my_first != 0x7fffffff) atomicMin(&sm.first, my_first);
            __syncthreads();
            const int first = sm.first;
            if (first == 0x7fffffff) {
                // Whole remainder of the tile stays in the binade: the thread
                // owning the last element publishes the new sum.
                int last = tend - 1;
                int owner = (last - pos) / kSeqPer;
                if (t == owner) {
                    uint32_t b2 = par_apply(ex, pM);
#pragma unroll
                    for (int q = 0; q < kSeqPer; q++) {
                        int j = pos + t * kSeqPer + q;
                        if (j <= last) b2 = sat_add(b2, par_apply(fn[q], (pM + b2) & 1u));
                    }
                    sm.s = ldexpf((float)(M + b2), e - 23);
                }
                __syncthreads();
                s = sm.s;
                __syncthreads();
                break;
            }
            // Event at `first`: the owner evaluates it exactly.
            int owner = (first - pos) / kSeqPer;
            if (t == owner) {
                uint32_t b2 = par_apply(ex, pM);
                float sb = s;
                float sa = s;
#pragma unroll
                for (int q = 0; q < kSeqPer; q++) {
                    int j = pos + t * kSeqPer + q;
                    if (j >= start && j < first) b2 = sat_add(b2, par_apply(fn[q], (pM + b2) & 1u));
                    if (j == first) {
                        sb = ldexpf((float)(M + b2), e - 23);  // exact sum before `first`
                        sa = sb + av[q];                        // the reference's f32 add
                    }
                }
                sm.s = sa;
                sm.start = pred(sa) ? -1 - first : first + 1;
            }
            __syncthreads();
            s = sm.s;
            const int nxt = sm.start;
            __syncthreads();
            if (nxt < 0) { *s_out = s; return -1 - nxt; }
            start = nxt;
            if (start >= tend) break;
        }
        pos = tend;
    }
    *s_out = s;
    return n;
}

} // namespace gs
