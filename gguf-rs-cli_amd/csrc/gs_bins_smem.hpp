// gs_bins_smem.hpp -- LDS layout of the binned full-vocabulary path.
#pragma once
#include <stdint.h>

namespace gs {

constexpr int kBins = 4096;        // bins of d' = y - m0 over [-kDLo, kDUp]
constexpr int kOverCap = 256;      // elements above the bin range (d' > kDUp)
constexpr int kMaxGroups = 256;    // runs of consecutive collected bins

struct BinsSmem {
    uint32_t cnt[kBins];           // pass 1: count; then collected bin -> cursor, bulk bin -> run index
    uint32_t off[kBins + 1];       // list segment of bin b: [off[b], off[b+1])
    // esum and k2 together double as a u64 mass array during pass 1 and plan A
    alignas(8) uint32_t esum[kBins];  // bulk bin: sum of seq-1 increments (later seq 3)
    uint32_t k2[kBins];            // bulk bin: sum of seq-2 increments (collected bin: f32 mass, transiently)
    uint32_t meta[kBins];          // flags, tie count and grid exponents
    float pre_e[kBins + 1];        // summand mass before bin b (plan B), for plan C
    uint32_t nzc[kBins];           // segment sort: nonzero entries of bin b, then their prefix
    uint32_t icur[kBins];          // pass 3: cursor of bin b's element indices
    uint64_t over[kOverCap];       // (key << 32) | ~idx of d' > kDUp
    uint32_t gbeg[kMaxGroups];     // group g: list range [gbeg, gend)
    uint32_t gend[kMaxGroups];
    uint64_t run[kMaxGroups + 1];  // bulk increment sum of run g (between groups g-1 and g)
    uint32_t runt[kMaxGroups + 1]; // seq-1 rounding ties inside run g
    int runb[kMaxGroups + 1];      // packed grid exponents and flags of run g
    uint32_t wbase[kMaxGroups + 1];// walk array: position of run g's marker
    float m0, m, s2lo, s2hi, Slo, Shi;
    float hw2, inv_s, inv_s2;
    float inv_s2c, hw3;            // merged pass 3: 1 / centre of the s2 range, seq-3 tolerance
    int ngroups, ndefer, nover, fail, ncollect, nties;
    int cut_g, ixlim, ixlast;
};

} // namespace gs
