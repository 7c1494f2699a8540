// gs_full_smem.hpp -- LDS layout of the exact full-vocabulary path (gs_full.hpp).
#pragma once
#include <stddef.h>
#include <stdint.h>
#include "gs_block.hpp"

namespace gs {

constexpr int kFBins = 4096;        // bins of d' = y - m0 over [-18.5, 3]
constexpr int kFOverCap = 256;      // elements above the bin range (d' > 3)
constexpr int kFMassBins = 1143;    // top bins whose mass pass 1 accumulates exactly
constexpr int kRecCap = 1023;       // threshold records per pass (10-bit index, 1023 = none)
constexpr uint32_t kNoRec = 0x3ffu;
constexpr int kTieCap = 64;         // rounding ties inside bag bins, per accumulation
constexpr int kWSeg = 64;           // walk: binade segments resolved per round

// Bin classes of one accumulation (see gs_full.hpp).
enum : uint32_t { kCNone = 0, kCUni = 1, kCRec = 2, kCBag = 3, kCLst = 4 };

// A bin whose summands take two integer increments (lvl and lvl + 1):
// elements with y >= up add lvl + 1, elements with thr <= y < up are rounding
// ties, the rest add lvl.  Pass counters: hi (y >= up), tie.  For the seq-3
// records of a nucleus row (s2 known only to a range) thr / up bound the
// elements whose increment the range leaves open (deferred).
struct FullRec {
    float thr, up;
    uint32_t hi, tie;
};
// A rounding tie inside a bag bin, and the increment function of a bag bin
// that holds ties.
struct FullTie {
    uint64_t en;
    uint32_t key;     // bin | accumulation << 16
    uint32_t k;       // the lower of the two increments
};
struct FullTieFn {
    uint32_t key;
    uint32_t f0, f1;
};

struct FullSmem {
    uint32_t cnt[kFBins];   // exact element count per bin (penalized values moved)
    uint32_t seg[kFBins];   // list segment start of a listed bin
    uint32_t sege[kFBins];  // list cursor of a listed bin: its segment's end after the pass
    // seq 1: bits 0-2 class, 3-12 record, 13 listed in pass 2, 14 increment
    // function in the tie table, 16-23 grid exponent + 128
    uint32_t w1[kFBins];
    // seq 1, then seq 2: the level of a uniform / record bin, the increment
    // sum of a bag bin; transiently the raw values of penalized ids per bin
    // (pass 1), walk item offsets of listed bins, a walk's cached increment
    // functions
    uint32_t v1[kFBins];
    // seqs 2/3: bits 0-2 class of seq 2, 3-5 class of seq 3, 6-15 seq-2
    // record, 16-25 seq-3 record, 26 listed in pass 3, 27 visited by pass 3,
    // 28 / 29 seq-2 / seq-3 function in the tie table
    uint32_t w23[kFBins];
    // seq 3: level or increment sum.  Before plan B, w23 and v3 (adjacent)
    // hold walk 1's cached increment functions, then plan B's u64 masses.
    uint32_t v3[kFBins];
    uint8_t ex[kFBins][2];  // grid exponents of seqs 2 and 3 + 128
    union {
        FullRec rec[kRecCap + 1];
        uint64_t mass64[kFMassBins];
    } u;
    uint64_t over[kFOverCap];
    FullTie ties[kTieCap];
    FullTieFn tiefn[kTieCap];
    int nties, ntiefn;
    uint64_t exptab[32];
    // walk: per binade segment of the current round
    uint32_t sj[kWSeg + 1];     // first item
    int se[kWSeg + 1];          // grid exponent
    uint32_t sF0[kWSeg + 1], sF1[kWSeg + 1];   // increments before the crossing item (last of the segment)
    float sv[kWSeg + 1];        // the crossing item's summand
    uint32_t sM[kWSeg + 1];     // the sum at the segment's start, in grid units
    float ss[kWSeg + 1];        // the sum at the segment's start
    ParFn wtot[kWaves];         // segmented scan: per-wave totals
    uint32_t wst[kWaves];
    uint32_t nbF0[kWaves], nbF1[kWaves], nbb[kWaves];   // each wave's last item, for the next wave
    float nbv[kWaves];
    int wfail, wfkind, wev, nseg, round_end;
    float wfs, wevs, wends;
    float m0, m, S;
    int nover, nrec, fail, ndefer, cutb, last2, last3;
    uint32_t list_end;
};

// ---------------------------------------------------------------------------
// LDS of the increment-histogram path (gs_full3.hpp).
constexpr int kF3Lvl = 12288;       // words of 16-bit level counters (two per word)
constexpr int kF3H = 2 * kF3Lvl;    // level counters
constexpr int kF3L1 = 8192;         // levels of seq 1 (pass 2)
constexpr int kF3L23 = 12288;       // levels of each of seqs 2 and 3 (pass 3)
constexpr int kF3Runs = 64;         // runs per accumulation
constexpr int kF3Regs = 192;        // regions of one walk
constexpr int kF3Ties = 64;         // rounding ties per accumulation
constexpr int kF3Tab = kFBins + 2;  // per-bin words: [0] above the bins, [1 + b] bin b, [kFBins + 1] below

// A run: consecutive bins whose elements the accumulation adds at one grid
// (2^(e-23)), none of them listed.  Its elements' increments k in [klo, khi]
// are counted in lvl[off + k].
struct F3Run {
    int off;               // level slot of increment k: off + k
    uint32_t klo, khi;
    int e;                 // grid exponent
    uint32_t base;         // first level slot (off + klo)
    uint32_t span;         // level slots
};
struct F3Reg { uint32_t b0, key, beg; };    // first bin, run id or kF3KeyListed / kF3KeyNone, list start
struct F3Tie { uint32_t run, k; uint64_t A; };   // an element at k + 1/2 grid units; A: the run's levels above it

struct Full3Smem {
    uint32_t cnt[kFBins];      // exact element count per bin (penalized values moved)
    uint32_t w[kF3Tab];        // pass 1: raw values of penalized ids per bin; pass 2: role words
    union {
        uint64_t mass64[kFMassBins];   // pass 1, plan A
        uint2 w23[kF3Tab];             // pass 3: role words of seqs 2, 3
    } u;
    alignas(16) uint32_t lvl[kF3Lvl + 1];  // level counters (plans: per-bin temporaries; walks: staged summands)
    alignas(16) float pre[kFBins + 1];   // predicted seq-1 sum before each bin ([kFBins]: the total); pass 3: element rings
    uint64_t over[kFOverCap];
    uint64_t exptab[32];
    F3Run run[2][kF3Runs];     // seq 1, then seq 2 | seq 3
    uint64_t rtot[2][kF3Runs]; // run totals of the walk
    F3Tie tie[2][kF3Ties];
    F3Reg reg[kF3Regs];
    uint32_t wlast[kWaves];    // region building: each wave's last key
    int nrun[2], ntie[2], nreg;
    uint32_t ltot[2];
    uint32_t lcount[2];        // increments counted into each level table (checks the 16-bit counters)
    float m0, m, S, s2, s2lo, s2hi, cb;
    int nover, fail, namb, ndef, bH, walk_res;
    uint32_t headend, list_end, cut_arr, cut_pos, tok_pos, tok_arr, list2;
    uint32_t qctr[2];          // passes 2 and 3: the next free chunk of the row
};
// walk 2 stages its summands over cnt and w as one array
static_assert(offsetof(Full3Smem, w) == offsetof(Full3Smem, cnt) + sizeof(uint32_t) * kFBins, "cnt, w adjacent");

} // namespace gs
