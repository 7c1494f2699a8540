// gs_select.hpp -- one chunk of a row's top-k, for the split top-k path: the
// chunk's kp best elements under the sampler's order, written in index order
// to the chunk's slots of the row's virtual row (split_select_kernel).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "gs_device.hpp"

namespace gs {

constexpr int kSelMaxKp = 128;        // kp = round_up(k, 4) <= kSelMaxKp

// What the selection needs of the row: its temperature (> 0, finite) and
// penalty (src/sampler.rs:23-30, 41), its window, and where the virtual row
// of row b lives (vrow / vidx + b * vld; chunk c owns slots [c kp, (c+1) kp)).
struct SelArgs {
    float T, rep;
    int kp;
    const uint32_t *recent;           // row b's window at recent + b * ld_recent, or null
    size_t ld_recent;
    const uint32_t *recent_len;       // per-row window lengths, or null (W)
    int W;
    float *vrow;
    uint32_t *vidx;
    size_t vld;
};

constexpr int kSelHist = 2048;        // bins of the thread maxima's keys

template <int NT, int PER>
struct SelSmem {
    uint32_t cnt[NT * PER / 2];       // window occurrences per chunk element, two u16 per word
    uint64_t tmax[NT];                // thread maxima at or above the histogram's edge
    uint32_t hist[kSelHist];
    uint32_t red[2 * (NT / 64)];      // per-wave key min / max
    uint32_t edge;
    int nlist;
    uint64_t cand[PER * kSelMaxKp];
    float candx[PER * kSelMaxKp];
    uint64_t top[kSelMaxKp];
    float topx[kSelMaxKp];
    uint64_t tau;
    int ncand;
    int nan;
};

// Chunk c of row b: elements c0 + i for i < L, kp <= L <= NT * PER, element i
// held by thread i % NT; val(i) is its raw logit.  Candidates are ordered by
// (key of y << 32) | ~id: larger is earlier in the sampler's order (y
// descending, then index ascending).  Applies the penalty (the
// window's occurrences of each id in the chunk, one op per occurrence),
// divides by T, keeps the kp largest keys and writes their penalized logits
// and ids in index order.  A NaN in the chunk goes to its first slot.  All
// NT threads call it (it has barriers).
//
// At least kp threads hold elements (kp <= min(L, NT)), so the kp-th largest
// thread maximum (keys carry the id: all distinct) bounds the kp-th largest
// element: at least kp elements reach it and at most kp * PER.
template <int NT, int PER, class Val>
__device__ void chunk_select(SelSmem<NT, PER> &sm, const SelArgs &s, int b, int c, int c0, int L, Val val)
{
    const int t = threadIdx.x;
    const bool has_pen = s.rep != 1.0f && s.recent != nullptr;
    int W = 0;
    if (has_pen) {
        W = s.recent_len ? (int)s.recent_len[b] : s.W;
        if (W > s.W) W = s.W;
    }
    float x[PER];
#pragma unroll
    for (int u = 0; u < PER; u++) {
        const int i = u * NT + t;
        x[u] = i < L ? val(i) : -INFINITY;
    }
    if (has_pen)
        for (int i = t; i < (L + 1) / 2; i += NT) sm.cnt[i] = 0u;
    if (t == 0) { sm.ncand = 0; sm.nan = 0; }
    __syncthreads();
    if (has_pen) {
        const uint32_t *rec = s.recent + (size_t)b * s.ld_recent;
        for (int j = t; j < W; j += NT) {
            const uint32_t d = ldg(rec + j) - (uint32_t)c0;   // ids >= V never fall in a chunk
            if (d < (uint32_t)L) atomicAdd(&sm.cnt[d >> 1], 1u << ((d & 1u) * 16u));   // W < 65536
        }
        __syncthreads();
    }
    // keys of y (the element's id completes the order): 32 bits per element
    uint32_t key[PER];
    uint64_t best = 0ull;
    bool nan = false;
    const uint16_t *cnt16 = reinterpret_cast<const uint16_t *>(sm.cnt);
#pragma unroll
    for (int u = 0; u < PER; u++) {
        const int i = u * NT + t;
        key[u] = 0u;
        if (i < L) {
            float xv = x[u];
            if (has_pen) {
                const uint32_t n = cnt16[i];
                if (n) xv = penalize(xv, n, s.rep);
            }
            x[u] = xv;
            const float y = xv / s.T;
            nan |= isnan(y);
            key[u] = f2key(y);
            const uint64_t k = ((uint64_t)key[u] << 32) | (uint64_t)(~(uint32_t)(c0 + i));
            best = k > best ? k : best;
        }
    }
    // tau = the kp-th largest thread maximum (keys carry the id: all
    // distinct).  A histogram of the maxima's y keys over their range finds
    // an edge with at least kp maxima at or above it; those maxima are
    // ranked among themselves.
    const bool has = t < L;                            // threads without elements have best 0
    const uint32_t bk = (uint32_t)(best >> 32);
    const int lane = t & 63, w = t >> 6;
    {
        uint32_t lo = has ? bk : 0xffffffffu, hi = has ? bk : 0u;
        for (int d = 32; d > 0; d >>= 1) {
            lo = min(lo, (uint32_t)__shfl_xor((int)lo, d, 64));
            hi = max(hi, (uint32_t)__shfl_xor((int)hi, d, 64));
        }
        if (lane == 0) { sm.red[2 * w] = lo; sm.red[2 * w + 1] = hi; }
    }
    for (int i = t; i < kSelHist; i += NT) sm.hist[i] = 0u;
    if (__any(nan) && lane == 0) sm.nan = 1;
    if (t == 0) sm.nlist = 0;
    __syncthreads();
    uint32_t kmin = 0xffffffffu, kmax = 0u;
#pragma unroll
    for (int i = 0; i < NT / 64; i++) { kmin = min(kmin, sm.red[2 * i]); kmax = max(kmax, sm.red[2 * i + 1]); }
    const uint64_t range = (uint64_t)(kmax - kmin) + 1u;
    if (has) atomicAdd(&sm.hist[(uint32_t)(((uint64_t)(bk - kmin) * kSelHist) / range)], 1u);
    __syncthreads();
    if (w == 0) {
        // lane l sums bins [32 l, 32 l + 32); suffix sums over lanes find the
        // bin j holding the kp-th largest maximum
        constexpr int kPerLane = kSelHist / 64;
        uint32_t own = 0u;
#pragma unroll 8
        for (int i = 0; i < kPerLane; i++) own += sm.hist[lane * kPerLane + i];
        uint32_t suf = own;                            // bins of lanes >= lane
        for (int d = 1; d < 64; d <<= 1) {
            const uint32_t o = (uint32_t)__shfl_down((int)suf, d, 64);
            if (lane + d < 64) suf += o;
        }
        const uint32_t above = suf - own;              // bins of lanes > lane
        if (suf >= (uint32_t)s.kp && above < (uint32_t)s.kp) {
            uint32_t acc = above;
            int j = lane * kPerLane;
            for (int i = kPerLane - 1; i >= 0; i--) {
                acc += sm.hist[lane * kPerLane + i];
                if (acc >= (uint32_t)s.kp) { j = lane * kPerLane + i; break; }
            }
            // the smallest key whose bin is >= j
            sm.edge = kmin + (uint32_t)(((uint64_t)j * range + kSelHist - 1) / kSelHist);
        }
    }
    __syncthreads();
    if (has && bk >= sm.edge) sm.tmax[atomicAdd(&sm.nlist, 1)] = best;
    __syncthreads();
    {
        const int nl = sm.nlist;
        for (int i = t; i < nl; i += NT) {
            const uint64_t me = sm.tmax[i];
            int rk = 0;
            for (int j = 0; j < nl; j++) rk += sm.tmax[j] > me;
            if (rk == s.kp - 1) sm.tau = me;
        }
    }
    __syncthreads();
    const uint64_t tau = sm.tau;
#pragma unroll
    for (int u = 0; u < PER; u++) {
        const int i = u * NT + t;
        const uint64_t k = ((uint64_t)key[u] << 32) | (uint64_t)(~(uint32_t)(c0 + i));
        if (i < L && k >= tau) {
            const int pos = atomicAdd(&sm.ncand, 1);
            sm.cand[pos] = k;
            sm.candx[pos] = x[u];
        }
    }
    __syncthreads();
    const int nc = sm.ncand;
    for (int i = t; i < nc; i += NT) {
        const uint64_t me = sm.cand[i];
        int rk = 0;
        for (int j = 0; j < nc; j++) rk += sm.cand[j] > me;
        if (rk < s.kp) { sm.top[rk] = me; sm.topx[rk] = sm.candx[i]; }
    }
    __syncthreads();
    if (t < s.kp) {
        const uint32_t id = ~(uint32_t)sm.top[t];
        int pos = 0;
        for (int j = 0; j < s.kp; j++) pos += (~(uint32_t)sm.top[j]) < id;
        const size_t o = (size_t)b * s.vld + (size_t)c * s.kp + pos;
        s.vrow[o] = (sm.nan && pos == 0) ? __builtin_nanf("") : sm.topx[t];
        s.vidx[o] = id;
    }
}

} // namespace gs
