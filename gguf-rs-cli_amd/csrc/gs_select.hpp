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

template <int NT, int PER>
struct SelSmem {
    uint32_t cnt[NT * PER];           // window occurrences per chunk element
    uint64_t tmax[NT];
    uint64_t cand[PER * kSelMaxKp];
    float candx[PER * kSelMaxKp];
    uint64_t top[kSelMaxKp];
    float topx[kSelMaxKp];
    uint64_t tau;
    int ncand;
    int nan;
};

// (key of y << 32) | ~id: larger is earlier in the sampler's order (y
// descending, then index ascending).
__device__ __forceinline__ uint64_t sel_key(float y, uint32_t id) { return ((uint64_t)f2key(y) << 32) | (uint64_t)(~id); }

// Chunk c of row b: elements c0 + i for i < L, kp <= L <= NT * PER, element i
// held by thread i % NT; val(i) is its raw logit.  Applies the penalty (the
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
        for (int i = t; i < L; i += NT) sm.cnt[i] = 0u;
    if (t == 0) { sm.ncand = 0; sm.nan = 0; }
    __syncthreads();
    if (has_pen) {
        const uint32_t *rec = s.recent + (size_t)b * s.ld_recent;
        for (int j = t; j < W; j += NT) {
            const uint32_t d = ldg(rec + j) - (uint32_t)c0;   // ids >= V never fall in a chunk
            if (d < (uint32_t)L) atomicAdd(&sm.cnt[d], 1u);
        }
        __syncthreads();
    }
    uint64_t key[PER];
    uint64_t best = 0ull;
    bool nan = false;
#pragma unroll
    for (int u = 0; u < PER; u++) {
        const int i = u * NT + t;
        key[u] = 0ull;
        if (i < L) {
            float xv = x[u];
            if (has_pen) {
                const uint32_t n = sm.cnt[i];
                if (n) xv = penalize(xv, n, s.rep);
            }
            x[u] = xv;
            const float y = xv / s.T;
            nan |= isnan(y);
            key[u] = sel_key(y, (uint32_t)(c0 + i));
            best = key[u] > best ? key[u] : best;
        }
    }
    sm.tmax[t] = best;
    if (__any(nan) && (t & 63) == 0) sm.nan = 1;
    __syncthreads();
    {
        int rk = 0;
        const ulonglong2 *t2 = reinterpret_cast<const ulonglong2 *>(sm.tmax);
#pragma unroll 8
        for (int j = 0; j < NT / 2; j++) {
            const ulonglong2 v = t2[j];
            rk += (v.x > best) + (v.y > best);
        }
        if (rk == s.kp - 1) sm.tau = best;             // threads without elements have best 0
    }
    __syncthreads();
    const uint64_t tau = sm.tau;
#pragma unroll
    for (int u = 0; u < PER; u++) {
        if (key[u] >= tau && key[u] != 0ull) {
            const int pos = atomicAdd(&sm.ncand, 1);
            sm.cand[pos] = key[u];
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
