// gs_full.hpp -- exact full-vocabulary sampling without sorting the row.
// (Included inside namespace gs by gs_kernels.hip, after RowSmem, the block
// helpers and the penalty table.)
//
// The reference (src/sampler.rs:44-78) sorts all V scaled logits y
// (descending, ties by index here), then runs three sequential f32
// accumulations in sorted order:
//   seq 1  S  = sum of a_j = expf(y_j - max)                    (:53-54)
//   seq 2  cum of p_j = a_j / S until cum >= top_p: cut, s2      (:56, :59-67)
//   seq 3  cum of q_j = p_j / s2 (or p_j) until r < cum          (:68, :71-78)
// While a running f32 sum stays inside one binade [2^e, 2^(e+1)) every add
// is integer arithmetic on multiples of g = 2^(e-23): RN(s + v) = s + g k,
// k = v / g rounded to nearest, ties to even (the only case where k depends
// on s: the parity of s / g).  Each summand is a monotone function of y, so
// inside one bin of y its increment k is a monotone step function of y.
//
// The elements are counted into 4096 bins of d' = y - m0.  For each bin and
// accumulation the plan predicts the binade of the running sum and
// evaluates the exact increment at the bin's edges:
//   * one value          : every element of the bin adds lvl (no work);
//   * two values         : the bin gets a record (thr, up): elements with
//                          y >= up add lvl + 1, elements with thr <= y < up
//                          are rounding ties, the rest add lvl; a pass
//                          counts the first two groups;
//   * more, or a bin where the sum may change binade, reach top_p or pass
//     the draw r        : the bin is listed (its elements' keys and ids
//                          are written to a per-row list and sorted).
// A bin's contribution is then a function of one parity bit (ties go to
// even, and the elements above a tie are exactly those with y >= up), so the
// three accumulations are replayed exactly by a walk over the sorted list
// entries and the counted bins (f_walk), which checks every prediction.
//
// Passes over the row: pass 1 (HBM) counts, pass 2 (cache) serves seq 1,
// pass 3 (cache) seqs 2 and 3.  For a nucleus row s2 is known before pass 3
// only to a range [top_p, top_p + the largest summand of the cut's bins]; an
// element whose seq-3 increment that range leaves open is deferred (its id is
// written) and counted once s2 is exact.  Any failed check returns false:
// the row then takes the sort-based path (the same result, slower).

// Failure exits (development builds record the line per row).
#if defined(GS_TIMING) || defined(GS_DIAG)
// per row (< 1024): [0] failing line of the row, [1] failing line of a walk,
// [2..7] statistics (see F_STAT uses)
__device__ int g_vdiag[1024 * 16];
#define F_NOTE(k) do { if (threadIdx.x == 0 && blockIdx.x < 1024) g_vdiag[blockIdx.x * 16 + (k)] = __LINE__; } while (0)
#define F_STAT(k, v) do { if (threadIdx.x == 0 && blockIdx.x < 1024) g_vdiag[blockIdx.x * 16 + (k)] = (int)(v); } while (0)
#else
#define F_NOTE(k) do { } while (0)
#define F_STAT(k, v) do { } while (0)
#endif
#ifdef GS_TIMING
// sub-phase timestamps per row (< 256): 64 slots
__device__ uint32_t g_vt[256 * 64];
#define F_TS(k) do { if (threadIdx.x == 0 && blockIdx.x < 256) g_vt[blockIdx.x * 64 + (k)] = (uint32_t)__builtin_amdgcn_s_memrealtime(); } while (0)
#else
#define F_TS(k) do { } while (0)
#endif
#define F_FAIL() do { F_NOTE(0); return false; } while (0)
#define F_WFAIL() do { F_NOTE(1); return -1; } while (0)

constexpr float kExpErr = 1.0f / 4194304.0f;      // bound on |fast_exp / expf - 1| (2^-22)
// exp(d) via v_exp_f32 with the rounding error of d*log2(e) compensated:
// t = RN(d*L), err = d*L - t (exact by fma) + d*(log2(e) - L), then
// exp2(t) * (1 + err*ln2).  Measured on gfx950 against glibc expf over every
// f32 d in [-30, 0]: max relative error 1.19e-7 (2^-23); kExpErr allows 2x.
// (Summands with d < -30 are below 1e-13: their increments are 0, far from
// any rounding boundary.)
__device__ __forceinline__ float fast_exp(float d)
{
    const float L = 1.44269504f;             // RN(log2 e)
    const float Llo = 1.925963033500e-8f;    // log2 e - L
    const float t = d * L;
    float err = fmaf(d, L, -t);
    err = fmaf(d, Llo, err);
    const float e0 = __builtin_amdgcn_exp2f(t);
    return fmaf(e0, err * 0.693147182f, e0);
}

// Integer increment of a summand already scaled by 2^(23-b), known to
// relative accuracy hw.  False if the rounding cannot be decided.
__device__ __forceinline__ bool inc_of(float m, float hw, uint32_t *k)
{
    float fl = floorf(m);
    float fr = m - fl;
    float tol = fmaf(m, hw, 1.0e-6f);
    *k = (uint32_t)fl + (fr > 0.5f ? 1u : 0u);
    return fabsf(fr - 0.5f) > tol && m < 8388608.0f;
}

constexpr float kFDUp = 3.0f;                 // bins cover d' in [-kFDLo, kFDUp]
constexpr float kFDLo = 18.5f;                // below: a < 2^-26, adds +0 to every sum
constexpr float kFInvW = (float)kFBins / (kFDUp + kFDLo);
constexpr double kFDelta = 1.0 / 4096.0;      // relative margin of every prediction
constexpr float kFMassScale = 4294967296.0f;  // pass-1 masses in 2^-32 units
constexpr int kFMaxSeg = 512;                 // largest listed bin (wave sort)
constexpr uint32_t kFDeferCap = 16384;        // deferred seq-3 elements per row
constexpr uint32_t kFPen = 0x80000000u;       // deferred entry: the id's penalized value

__device__ __forceinline__ int f_bin(float dp)
{
    const int b = (int)((kFDUp - dp) * kFInvW);
    return min(max(b, 0), kFBins - 1);
}
__device__ __forceinline__ uint64_t f_entry(float y, uint32_t i) { return ((uint64_t)f2key(y) << 32) | (uint64_t)(~i); }
__device__ __forceinline__ float f_entry_y(uint64_t en) { return key2f((uint32_t)(en >> 32)); }
__device__ __forceinline__ uint32_t f_entry_id(uint64_t en) { return ~(uint32_t)en; }
// walk items: list entries, or a bin (high word 0, bin index in the low bits)
__device__ __forceinline__ uint64_t f_bin_item(int b) { return (uint64_t)(uint32_t)b; }
__device__ __forceinline__ bool f_is_bin(uint64_t it) { return (uint32_t)(it >> 32) == 0u; }

// Binade exponent of a positive normal double.
__device__ __forceinline__ int f_dexp(double x) { return (int)((__double_as_longlong(x) >> 52) & 0x7ff) - 1023; }

// Constants of the three summands.
struct FSeq {
    float m, S;
    bool nuc;
    const uint64_t *tab;   // expf's table (a copy in LDS)
};
// Exact summand of accumulation sq for scaled logit y (src/sampler.rs:54, :56, :68).
__device__ __forceinline__ float f_val(const FSeq &c, int sq, float y, float s2)
{
    const float a = glibc_expf_tab(y - c.m, c.tab);
    if (sq == 1) return a;
    const float p = a / c.S;
    if (sq == 2 || !c.nuc) return p;
    return p / s2;
}
// Increments of summand v at grid exponent e with a tie rounded down / up.
__device__ __forceinline__ void f_incs(float v, int e, uint32_t *dn, uint32_t *up)
{
    const float w = ldexpf(v, 23 - e);
    if (!(w < 33554432.0f)) { *dn = *up = kSat; return; }
    const float fl = floorf(w);
    const float fr = w - fl;
    *dn = (uint32_t)fl + (fr > 0.5f ? 1u : 0u);
    *up = (uint32_t)fl + (fr >= 0.5f ? 1u : 0u);
}
// Smallest y in [ylo, yhi] whose increment reaches lvl + 1 (ties counted as
// reaching it if `tie_up`); the increment must reach it at yhi.  The search
// starts at the y where the real summand crosses lvl + 1/2 grid steps (`est`)
// and gallops over f32 keys to the exact boundary.
__device__ float f_first(const FSeq &c, int sq, int e, uint32_t lvl, float ylo, float yhi, float s2, bool tie_up,
                         double est)
{
    auto reach = [&](uint32_t k) {
        uint32_t dn, up;
        f_incs(f_val(c, sq, key2f(k), s2), e, &dn, &up);
        return (tie_up ? up : dn) >= lvl + 1u;
    };
    const uint32_t klo = f2key(ylo), khi = f2key(yhi);
    if (reach(klo)) return ylo;
    // [lo, hi]: reach(lo) false, reach(hi) true
    uint32_t lo = klo, hi = khi;
    const float ye = (float)est;
    if (ye > ylo && ye < yhi) {
        const uint32_t k0 = f2key(ye);
        if (reach(k0)) {
            hi = k0;
            for (uint32_t d = 1; hi - d > lo; d <<= 1) {
                if (!reach(hi - d)) { lo = hi - d; break; }
                hi = hi - d;
            }
        } else {
            lo = k0;
            for (uint32_t d = 1; lo + d < hi; d <<= 1) {
                if (reach(lo + d)) { hi = lo + d; break; }
                lo = lo + d;
            }
        }
    }
    while (hi - lo > 1u) {
        const uint32_t mid = lo + ((hi - lo) >> 1);
        if (reach(mid)) hi = mid;
        else lo = mid;
    }
    return key2f(hi);
}
// A y-interval holding every element bin b can receive (the bin index is
// computed in f32; the margin covers its rounding).
__device__ __forceinline__ void f_range(float m0, int b, float *ylo, float *yhi)
{
    const double w = (double)(kFDUp + kFDLo) / kFBins;
    const double hi = (double)m0 + kFDUp - b * w, lo = (double)m0 + kFDUp - (b + 1) * w;
    const double tol = 2e-5 + 4e-6 * fmax(fabs(hi), fabs(lo));
    *yhi = (float)(hi + tol);
    *ylo = (float)(lo - tol);
}
// Increment function of a counted bin: nup elements add lvl + 1, then ntie
// rounding ties at lvl + 1/2 (the first goes to even from the parity before
// it, which leaves the sum even, so the others add lvl + (lvl & 1)), then
// nlo elements add lvl.
__device__ __forceinline__ ParFn f_binfn(uint32_t lvl, uint32_t nup, uint32_t ntie, uint32_t nlo)
{
    ParFn f;
#pragma unroll
    for (uint32_t p = 0; p < 2; p++) {
        uint64_t n = p + (uint64_t)(lvl + 1u) * nup;
        if (ntie) {
            n += lvl + ((n + lvl) & 1u);
            n += (uint64_t)(ntie - 1u) * (lvl + (lvl & 1u));
        }
        n += (uint64_t)lvl * nlo;
        const uint64_t d = n - p;
        const uint32_t v = d > kSat ? kSat : (uint32_t)d;
        if (p == 0) f.f0 = v;
        else f.f1 = v;
    }
    return f;
}
__device__ __forceinline__ ParFn f_fn_id() { return ParFn{0u, 0u}; }

// Classify one bin for accumulation sq at grid exponent e from its
// increments at the edges of its y-range: returns 0 (one increment: *lvl),
// 1 (two: *lvl and lvl + 1; f_threshold then finds the boundaries), 2 (more:
// list it).  For seq 3 of a nucleus row s2 lies in [s2lo, s2hi]: lvl is the
// lowest increment over the range.
__device__ int f_classify(const FSeq &c, int sq, int e, float ylo, float yhi, float s2lo, float s2hi,
                          uint32_t *lvl)
{
    uint32_t d0, u0, d1, u1;
    f_incs(f_val(c, sq, ylo, s2hi), e, &d0, &u0);
    f_incs(f_val(c, sq, yhi, s2lo), e, &d1, &u1);
    if (u1 - d0 > 1u || u1 < d0) return 2;
    *lvl = d0;
    return u1 == d0 ? 0 : 1;
}
// The summand of accumulation sq >= 2 from a = expf(y - m) (f_val's steps).
__device__ __forceinline__ float f_val_a(const FSeq &c, int sq, float a, float s2)
{
    const float p = a / c.S;
    return (sq == 2 || !c.nuc) ? p : p / s2;
}
// f_classify for sq >= 2 with a(ylo), a(yhi) already evaluated (plan B
// classifies both accumulations at the same edges).
__device__ __forceinline__ int f_classify_a(const FSeq &c, int sq, int e, float alo, float ahi, float s2lo,
                                            float s2hi, uint32_t *lvl)
{
    uint32_t d0, u0, d1, u1;
    f_incs(f_val_a(c, sq, alo, s2hi), e, &d0, &u0);
    f_incs(f_val_a(c, sq, ahi, s2lo), e, &d1, &u1);
    if (u1 - d0 > 1u || u1 < d0) return 2;
    *lvl = d0;
    return u1 == d0 ? 0 : 1;
}
// One boundary of a two-increment bin (f_classify returned 1): which == 0
// gives thr, the smallest y whose increment reaches lvl + 1 with a rounding
// tie counted as reaching it (for every s2 in the range: at s2lo); which ==
// 1 gives up, the smallest y that reaches lvl + 1 without a tie for every s2
// (at s2hi), or +inf if no y in the bin does.  Elements with y >= up add
// lvl + 1, those with thr <= y < up are ties (or, for seq 3 of a nucleus
// row, undecided until s2 is exact), the rest add lvl.
__device__ float f_threshold(const FSeq &c, int sq, int e, uint32_t lvl, float ylo, float yhi, float s2lo,
                             float s2hi, int which)
{
    // the real summand reaches (lvl + 1/2) g at y = m + ln((lvl + 1/2) g S s2)
    const double a = ldexp((double)lvl + 0.5, e - 23) * (sq >= 2 ? (double)c.S : 1.0);
    const bool s3 = sq == 3 && c.nuc;
    if (which == 0) {
        const double elo = (double)c.m + log(a * (s3 ? (double)s2lo : 1.0));
        return f_first(c, sq, e, lvl, ylo, yhi, s2lo, true, elo);
    }
    uint32_t d2, u2;
    f_incs(f_val(c, sq, yhi, s2hi), e, &d2, &u2);
    if (d2 < lvl + 1u) return INFINITY;
    const double ehi = (double)c.m + log(a * (s3 ? (double)s2hi : 1.0));
    return f_first(c, sq, e, lvl, ylo, yhi, s2hi, false, ehi);
}
// Pending record (set by a classification loop, resolved by f_thresholds):
// thr holds bin | sq << 12 | (grid exponent + 128) << 16, up holds lvl.
__device__ __forceinline__ FullRec f_rec_pending(int b, int sq, int e, uint32_t lvl)
{
    return FullRec{__uint_as_float((uint32_t)b | ((uint32_t)sq << 12) | ((uint32_t)(e + 128) << 16)),
                   __uint_as_float(lvl), 0u, 0u};
}

// Resolve the pending records [0, nrec) of a classification loop: two
// threads per record, all threads of the block.  The first half of the
// block finds the thr boundaries and the second half the up boundaries, so
// that no wave runs both searches one after the other.
__device__ void f_thresholds(RowSmem &sm, const FSeq &c, float m0, float s2lo, float s2hi)
{
    FullSmem &f = sm.x.fs;
    const int t = threadIdx.x;
    const int nr = min(f.nrec, kRecCap);
    for (int base = 0; base < nr; base += kThreads / 2) {
        const int r = base + (t % (kThreads / 2)), which = t / (kThreads / 2);
        uint32_t info = 0u, lvl = 0u;
        if (r < nr) {
            info = __float_as_uint(f.u.rec[r].thr);
            lvl = __float_as_uint(f.u.rec[r].up);
        }
        __syncthreads();
        if (r < nr) {
            const int b = (int)(info & 0xfffu), sq = (int)((info >> 12) & 3u), e = (int)((info >> 16) & 255u) - 128;
            float ylo, yhi;
            f_range(m0, b, &ylo, &yhi);
            const float v = f_threshold(c, sq, e, lvl, ylo, yhi, s2lo, s2hi, which);
            if (which == 0) f.u.rec[r].thr = v;
            else f.u.rec[r].up = v;
        }
        __syncthreads();
    }
}

// Fields of the per-bin words.
__device__ __forceinline__ uint32_t f_cls(uint32_t w1, uint32_t w23, int sq)
{
    return sq == 1 ? (w1 & 7u) : (sq == 2 ? (w23 & 7u) : ((w23 >> 3) & 7u));
}
__device__ __forceinline__ uint32_t f_recix(uint32_t w1, uint32_t w23, int sq)
{
    return sq == 1 ? ((w1 >> 3) & kNoRec) : (sq == 2 ? ((w23 >> 6) & kNoRec) : ((w23 >> 16) & kNoRec));
}
constexpr uint32_t kW1Listed = 1u << 13, kW1TieFn = 1u << 14;
constexpr uint32_t kW3Listed = 1u << 26, kW3Visit = 1u << 27, kW3TieFn2 = 1u << 28, kW3TieFn3 = 1u << 29;

// Increment function of bin item b in accumulation sq (a uniform, record or
// bag bin); *ok = false if the bin is none of these for that accumulation.
__device__ __forceinline__ ParFn f_item_fn(const FullSmem &f, int sq, int b, int *eb, bool *ok)
{
    const uint32_t w1 = f.w1[b], w23 = f.w23[b];
    const uint32_t cls = f_cls(w1, w23, sq);
    *ok = cls == kCUni || cls == kCRec || cls == kCBag;
    *eb = sq == 1 ? (int)((w1 >> 16) & 255u) - 128 : (int)f.ex[b][sq - 2] - 128;
    const uint32_t val = sq == 3 ? f.v3[b] : f.v1[b];
    if (cls == kCBag) {
        const bool tf = sq == 1 ? (w1 & kW1TieFn) != 0u : (w23 & (sq == 2 ? kW3TieFn2 : kW3TieFn3)) != 0u;
        if (tf) {
            const uint32_t key = (uint32_t)b | ((uint32_t)sq << 16);
            for (int i = 0; i < f.ntiefn; i++)
                if (f.tiefn[i].key == key) return ParFn{f.tiefn[i].f0, f.tiefn[i].f1};
            *ok = false;
        }
        const uint32_t v = val > kSat ? kSat : val;
        return ParFn{v, v};
    }
    const uint32_t n = f.cnt[b];
    uint32_t nup = 0u, ntie = 0u;
    if (cls == kCRec) {
        const uint32_t rr = f_recix(w1, w23, sq);
        nup = f.u.rec[rr].hi;
        ntie = f.u.rec[rr].tie;
    }
    return f_binfn(val, nup, ntie, n - nup - ntie);
}

// ---------------------------------------------------------------------------
// Block helpers.

// f(p, entry) for list positions p in [lo, hi), strided over the block; each
// thread issues U loads before it uses any (the loop bodies are short and
// end in LDS atomics, so one load per iteration would expose its latency).
template <int U, class F>
__device__ __forceinline__ void f_list_for_each(const uint64_t *gl, uint32_t lo, uint32_t hi, F f)
{
    for (uint32_t base = lo + threadIdx.x; base < hi; base += kThreads * U) {
        uint64_t e[U];
#pragma unroll
        for (int u = 0; u < U; u++) {
            const uint32_t q = base + (uint32_t)(u * kThreads);
            e[u] = q < hi ? ldg(gl + q) : 0ull;
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const uint32_t q = base + (uint32_t)(u * kThreads);
            if (q < hi) f(q, e[u]);
        }
    }
}
// The same scan through the per-wave buffer `buf` (kWaves doubles of LDS),
// with one barrier: the caller must pass a barrier before `buf` is written
// again.
__device__ double f_block_excl_f64_buf(double v, double *tot, double *buf)
{
    const int lane = lane_id(), w = wave_id();
    const double incl = wave_incl_f64(v);
    if (lane == 63) buf[w] = incl;
    __syncthreads();
    double pre = 0.0, all = 0.0;
    for (int i = 0; i < kWaves; i++) { if (i < w) pre += buf[i]; all += buf[i]; }
    *tot = all;
    return pre + incl - v;
}
__device__ double f_block_excl_f64(double v, double *tot, RowSmem &sm)
{
    const int lane = lane_id(), w = wave_id();
    const double incl = wave_incl_f64(v);
    if (lane == 63) sm.red_f64[w] = incl;
    __syncthreads();
    double pre = 0.0, all = 0.0;
    for (int i = 0; i < kWaves; i++) { if (i < w) pre += sm.red_f64[i]; all += sm.red_f64[i]; }
    __syncthreads();
    *tot = all;
    return pre + incl - v;
}
__device__ float f_block_max(float v, RowSmem &sm)
{
    for (int d = 32; d > 0; d >>= 1) v = fmaxf(v, __shfl_xor(v, d, 64));
    if (lane_id() == 0) sm.red_f32[wave_id()] = v;
    __syncthreads();
    float r = sm.red_f32[0];
    for (int i = 1; i < kWaves; i++) r = fmaxf(r, sm.red_f32[i]);
    __syncthreads();
    return r;
}
// Segmented scan element: `st` = a segment starts inside.
struct SegFn { uint32_t st; ParFn f; };
__device__ __forceinline__ SegFn seg_op(const SegFn &a, const SegFn &b)
{
    SegFn r;
    r.st = a.st | b.st;
    r.f = b.st ? b.f : par_compose(a.f, b.f);
    return r;
}
// Exclusive segmented scan of the block's SegFn values (thread order),
// together with an exclusive sum of one count per thread (*cex; *ctot the
// block's total): one pair of barriers for both.
__device__ SegFn f_block_seg_excl_cnt(SegFn v, uint32_t cnt, RowSmem &sm, ParFn *wtot, uint32_t *wst,
                                      uint32_t *cex, uint32_t *ctot)
{
    const int lane = lane_id(), w = wave_id();
    SegFn incl = v;
    uint32_t cin = cnt;
    for (int d = 1; d < 64; d <<= 1) {
        SegFn o;
        o.st = __shfl_up(incl.st, d, 64);
        o.f.f0 = __shfl_up(incl.f.f0, d, 64);
        o.f.f1 = __shfl_up(incl.f.f1, d, 64);
        const uint32_t oc = __shfl_up(cin, d, 64);
        if (lane >= d) { incl = seg_op(o, incl); cin += oc; }
    }
    if (lane == 63) { wtot[w] = incl.f; wst[w] = incl.st; sm.red_u32[w] = cin; }
    __syncthreads();
    SegFn pre{0u, f_fn_id()};
    uint32_t cpre = 0u, call = 0u;
    for (int i = 0; i < kWaves; i++) {
        if (i < w) { pre = seg_op(pre, SegFn{wst[i], wtot[i]}); cpre += sm.red_u32[i]; }
        call += sm.red_u32[i];
    }
    __syncthreads();
    SegFn ex;
    ex.st = __shfl_up(incl.st, 1, 64);
    ex.f.f0 = __shfl_up(incl.f.f0, 1, 64);
    ex.f.f1 = __shfl_up(incl.f.f1, 1, 64);
    if (lane == 0) ex = SegFn{0u, f_fn_id()};
    *cex = cpre + cin - cnt;
    *ctot = call;
    return seg_op(pre, ex);
}

// ---------------------------------------------------------------------------
// The walk: exact replay of one accumulation over a sorted item array
// (list entries and counted bins), stopping at the first item after which
// the predicate holds.  Items are processed in chunks of kThreads * kWC, each
// thread owning kWC consecutive items.  Per round: the binade of the sum
// before every item is predicted (a prefix scan of the items' increments at
// the predicted grids, refined twice); items of one predicted binade form a
// segment whose integer increments are composed by a segmented scan; one
// thread chains the segments (each ends with the item that leaves the
// binade, added with the reference's own f32 add); then every item checks
// its prediction.  The first failed check restarts the round from that
// item with the exact sum before it.  Returns the event item (and the sum
// after it), N if none (the final sum), -1 on failure.
constexpr int kWC = 4;
constexpr int kWMaxRounds = 96;
enum { kWFailCross = 1, kWFailBin = 2, kWFailRepred = 3 };
struct WArgs {
    FSeq c;
    int sq;
    float s2;
    int pk;          // 0 none, 1 s >= thr, 2 thr < s
    float thr;
    const uint32_t *c0, *c1;   // the bins' cached increment functions (f_cache_fns)
};
// Cache the increment functions of accumulation sq's bin items in two LDS
// arrays: c0[b] = f0, c1[b] = f1 | (grid exponent + 64) << 25, both capped
// at 2^24 (a bin adding that much leaves its binade anyway); a zero exponent
// field marks a bin that is not a bin item of sq.
__device__ void f_cache_fns(RowSmem &sm, int sq, uint32_t *c0, uint32_t *c1)
{
    FullSmem &f = sm.x.fs;
    for (int b = threadIdx.x; b < kFBins; b += kThreads) {
        int eb;
        bool ok;
        const ParFn fn = f_item_fn(f, sq, b, &eb, &ok);
        ok &= eb > -64 && eb < 64;
        c0[b] = min(fn.f0, 1u << 24);
        c1[b] = min(fn.f1, 1u << 24) | (ok ? (uint32_t)(eb + 64) << 25 : 0u);
    }
    __syncthreads();
}
__device__ __forceinline__ ParFn w_binfn(const WArgs &wa, int b, int *eb, bool *ok)
{
    const uint32_t a = wa.c0[b], c = wa.c1[b];
    *eb = (int)(c >> 25) - 64;
    *ok = (c >> 25) != 0u;
    return ParFn{a, c & 0x1ffffffu};
}
__device__ __forceinline__ bool w_pred(const WArgs &wa, float s)
{
    return wa.pk == 1 ? s >= wa.thr : (wa.pk == 2 ? wa.thr < s : false);
}

// Increment function of walk item q (an element's summand or a bin) at grid e.
__device__ __forceinline__ ParFn w_fn(const FullSmem &f, const WArgs &wa, bool bin, float v, int e, bool *bad)
{
    if (bin) {
        int eb;
        bool ok;
        const ParFn fn = w_binfn(wa, __float_as_int(v), &eb, &ok);
        *bad = !ok || (eb != e && (fn.f0 | fn.f1));
        return fn;
    }
    *bad = false;
    return elem_fn(v, e);
}

__device__ int f_walk(RowSmem &sm, const uint64_t *items, int N, const WArgs &wa, float *s_out, int slot)
{
    int nrounds = 0;
    const int tsb = 16 + 8 * (slot - 8);
    F_TS(tsb + 0);
    FullSmem &f = sm.x.fs;
    const int t = threadIdx.x, lane = lane_id(), w = wave_id();
    constexpr int kNone = 0x7fffffff;
    float s = 0.0f;
    int pos = 0;
    // The leading run below almost always ends after item 0: the first
    // chunk's items (from item 1) are loaded alongside it.
    const int pend = min(1 + kThreads * kWC, N);
    uint64_t pf[kWC];
#pragma unroll
    for (int q = 0; q < kWC; q++) {
        const int j = 1 + t * kWC + q;
        pf[q] = j < pend ? ldg(items + j) : 0ull;
    }
    // leading items from s == 0 (0 + v == v); every thread does the same
    while (pos < N && s == 0.0f) {
        const uint64_t it = ldg(items + pos);
        if (f_is_bin(it)) {
            int eb;
            bool ok;
            const ParFn fn = w_binfn(wa, (int)(uint32_t)it, &eb, &ok);
            if (!ok || fn.f0 || fn.f1) { *s_out = s; F_WFAIL(); }
        } else {
            s = f_val(wa.c, wa.sq, f_entry_y(it), wa.s2);
            if (w_pred(wa, s)) { *s_out = s; return pos; }
        }
        pos++;
    }
    F_TS(tsb + 7);
    float v[kWC];
    uint32_t isbin = 0u;
    auto take = [&](int q, uint64_t it) {
        if (f_is_bin(it)) { isbin |= 1u << q; v[q] = __int_as_float((int)(uint32_t)it); }
        else v[q] = f_val(wa.c, wa.sq, f_entry_y(it), wa.s2);
    };
    const bool pf_ok = pos == 1;
    if (pf_ok) {
#pragma unroll
        for (int q = 0; q < kWC; q++) {
            v[q] = 0.0f;
            if (1 + t * kWC + q < pend) take(q, pf[q]);
        }
    }
    for (bool first = true; pos < N; first = false) {
        const int cend = min(pos + kThreads * kWC, N);
        const int j0 = pos + t * kWC;
        if (!(first && pf_ok)) {
            isbin = 0u;
#pragma unroll
            for (int q = 0; q < kWC; q++) {
                v[q] = 0.0f;
                const int j = j0 + q;
                if (j < cend) take(q, ldg(items + j));
            }
        }
        int start = pos;
        for (int round = 0;; round++) {
            if (round >= kWMaxRounds) { *s_out = s; F_WFAIL(); }
            nrounds++;
            F_STAT(slot, nrounds);
            F_TS(tsb + 1);
            // ---- predicted grid of the sum before every item: three scans ----
            int e[kWC];
            double tpre = 0.0, tot;
            for (int it = 0; it < 3; it++) {
                double loc = 0.0;
                const double base = (double)s + tpre;
#pragma unroll
                for (int q = 0; q < kWC; q++) {
                    const int j = j0 + q;
                    if (it == 2) e[q] = 0;
                    if (j < start || j >= cend) continue;
                    const int eq = j == start ? grid_exp(s) : f_dexp(base + loc);
                    if (it == 2) e[q] = eq;
                    double cq;
                    if (isbin & (1u << q)) {
                        int eb;
                        bool ok;
                        const ParFn fn = w_binfn(wa, __float_as_int(v[q]), &eb, &ok);
                        cq = it == 0 ? ldexp(0.5 * ((double)fn.f0 + (double)fn.f1), eb - 23)
                                     : ldexp((double)fn.f0, eb - 23);
                    } else if (it == 0) {
                        cq = (double)v[q];
                    } else {
                        uint32_t dn, up;
                        f_incs(v[q], eq, &dn, &up);
                        cq = ldexp((double)dn, eq - 23);
                    }
                    loc += cq;
                }
                // (two buffers: the segment barrier below comes before either is reused)
                if (it < 2) tpre = f_block_excl_f64_buf(loc, &tot, it == 0 ? sm.red_f64 : sm.red_f64b);
            }
            F_TS(tsb + 2);
            // ---- segments: an item starts one if its grid differs from the item before ----
            int prev_e = __shfl_up(e[kWC - 1], 1, 64);
            if (lane == 63) sm.red_i32[w] = e[kWC - 1];
            __syncthreads();
            if (lane == 0) prev_e = w > 0 ? sm.red_i32[w - 1] : 0;
            uint32_t starts = 0u, nst = 0u;
            {
                int ep = prev_e;
#pragma unroll
                for (int q = 0; q < kWC; q++) {
                    const int j = j0 + q;
                    if (j >= start && j < cend && (j == start || e[q] != ep)) { starts |= 1u << q; nst++; }
                    ep = e[q];
                }
            }
            SegFn agg{0u, f_fn_id()};
#pragma unroll
            for (int q = 0; q < kWC; q++) {
                const int j = j0 + q;
                if (j < start || j >= cend) continue;
                bool bad;
                const ParFn fn = w_fn(f, wa, (isbin >> q) & 1u, v[q], e[q], &bad);
                agg = seg_op(agg, SegFn{(starts >> q) & 1u, fn});
            }
            // the segments' composed increments and each thread's first segment ordinal
            uint32_t nseg, ord0;
            const SegFn carry = f_block_seg_excl_cnt(agg, nst, sm, f.wtot, f.wst, &ord0, &nseg);   // contains barriers
            const int nused = (int)min(nseg, (uint32_t)kWSeg);
            F_TS(tsb + 3);
            // segment table: first item and grid of each segment; for each
            // segment followed by another, the prefix before its last item
            // (the one that leaves the binade) and that item's summand
            ParFn last_ex = f_fn_id();
            float last_v = 0.0f;
            bool last_bin = false;
            {
                uint32_t ord = ord0;
                SegFn run = carry;
                ParFn pex = f_fn_id();
                float pv = 0.0f;
                bool pbin = false;
#pragma unroll
                for (int q = 0; q < kWC; q++) {
                    const int j = j0 + q;
                    if (j < start || j >= cend) continue;
                    const bool st = (starts >> q) & 1u;
                    if (st) {
                        if (ord <= (uint32_t)kWSeg) { f.sj[ord] = (uint32_t)j; f.se[ord] = e[q]; }
                        if (q > 0 && ord >= 1u && ord - 1u < (uint32_t)nused) {
                            f.sF0[ord - 1u] = pex.f0;
                            f.sF1[ord - 1u] = pex.f1;
                            f.sv[ord - 1u] = pbin ? __int_as_float(0x7fc00000) : pv;
                        }
                        ord++;
                    }
                    bool bad;
                    const ParFn fn = w_fn(f, wa, (isbin >> q) & 1u, v[q], e[q], &bad);
                    pex = st ? f_fn_id() : run.f;
                    pv = v[q];
                    pbin = (isbin >> q) & 1u;
                    run = st ? SegFn{1u, fn} : SegFn{run.st, par_compose(run.f, fn)};
                }
                last_ex = pex;
                last_v = pv;
                last_bin = pbin;
            }
            // the previous thread's last item, for a segment starting at my first item
            {
                ParFn nex;
                nex.f0 = __shfl_up(last_ex.f0, 1, 64);
                nex.f1 = __shfl_up(last_ex.f1, 1, 64);
                float nv = __shfl_up(last_v, 1, 64);
                int nbin = __shfl_up((int)last_bin, 1, 64);
                if (lane == 63) { f.nbF0[w] = last_ex.f0; f.nbF1[w] = last_ex.f1; f.nbv[w] = last_v; f.nbb[w] = last_bin; }
                __syncthreads();
                if (lane == 0 && w > 0) { nex.f0 = f.nbF0[w - 1]; nex.f1 = f.nbF1[w - 1]; nv = f.nbv[w - 1]; nbin = f.nbb[w - 1]; }
                if ((starts & 1u) && j0 > start && ord0 >= 1u && ord0 - 1u < (uint32_t)nused) {
                    f.sF0[ord0 - 1u] = nex.f0;
                    f.sF1[ord0 - 1u] = nex.f1;
                    f.sv[ord0 - 1u] = nbin ? __int_as_float(0x7fc00000) : nv;
                }
            }
            if (t == 0) { f.wfail = kNone; f.wev = kNone; }
            __syncthreads();
            F_TS(tsb + 4);
            // ---- chain the segments (one thread) ----
            if (t == 0) {
                float cs = s;
                int nok = nused, rend = nseg > (uint32_t)nused ? (int)f.sj[nused] : cend;
                for (int k = 0; k < nused; k++) {
                    f.ss[k] = cs;
                    const int ek = f.se[k];
                    if (grid_exp(cs) != ek) {          // never for k = 0 (its grid is the sum's)
                        nok = k;
                        rend = (int)f.sj[k];
                        f.wfail = rend;
                        f.wfkind = kWFailRepred;
                        f.wfs = cs;
                        break;
                    }
                    const uint32_t M = (uint32_t)ldexpf(cs, 23 - ek);
                    f.sM[k] = M;
                    if (k + 1 < (int)nseg) {
                        const float vc = f.sv[k];
                        if (isnan(vc)) {               // a bin cannot leave the binade
                            nok = k + 1;
                            rend = (int)f.sj[k + 1] - 1;
                            f.wfail = rend;
                            f.wfkind = kWFailBin;
                            break;
                        }
                        const ParFn F{f.sF0[k], f.sF1[k]};
                        const uint32_t nb = M + par_apply(F, M & 1u);
                        cs = ldexpf((float)nb, ek - 23) + vc;   // the reference's f32 add
                        f.ss[k + 1] = cs;
                    }
                }
                f.nseg = nok;
                f.round_end = rend;
            }
            __syncthreads();
            const int nok = f.nseg, rend = f.round_end;
            F_TS(tsb + 5);
            // ---- check every item up to rend, find the event ----
            int myfail = kNone, mykind = 0, myev = kNone;
            float myfs = 0.0f, myevs = 0.0f, mylast = 0.0f;
            {
                uint32_t ord = ord0;
                SegFn run = carry;
                int k = (int)ord0 - 1;
#pragma unroll
                for (int q = 0; q < kWC; q++) {
                    const int j = j0 + q;
                    if (j < start || j >= rend) continue;
                    const bool st = (starts >> q) & 1u;
                    if (st) { k = (int)ord; ord++; }
                    bool bad;
                    const bool bin = (isbin >> q) & 1u;
                    const ParFn fn = w_fn(f, wa, bin, v[q], e[q], &bad);
                    const ParFn ex = st ? f_fn_id() : run.f;
                    run = st ? SegFn{1u, fn} : SegFn{run.st, par_compose(run.f, fn)};
                    if (myfail != kNone || myev != kNone) continue;
                    const int ek = e[q];
                    const uint32_t M = f.sM[k];
                    const uint32_t nb = M + par_apply(ex, M & 1u);
                    const bool crossing = k + 1 < (int)nseg && k + 1 <= kWSeg && j + 1 == (int)f.sj[k + 1];
                    float sa;
                    if (crossing) {
                        sa = f.ss[k + 1];
                    } else {
                        const uint32_t na = nb + par_apply(fn, nb & 1u);
                        if (bad || (bin && na >= (1u << 24))) { myfail = j; mykind = kWFailBin; continue; }
                        if (na >= (1u << 24)) {
                            myfail = j;
                            mykind = kWFailCross;
                            myfs = ldexpf((float)nb, ek - 23) + v[q];   // the reference's f32 add
                            continue;
                        }
                        sa = ldexpf((float)na, ek - 23);
                    }
                    if (w_pred(wa, sa)) {
                        if (bin) { myfail = j; mykind = kWFailBin; continue; }
                        myev = j;
                        myevs = sa;
                    }
                    mylast = sa;
                }
            }
            (void)nok;
            if (myfail != kNone) atomicMin(&f.wfail, myfail);
            if (myev != kNone) atomicMin(&f.wev, myev);
            __syncthreads();
            const int gfail = f.wfail, gev = f.wev;
            if (myfail == gfail && myfail != kNone) { f.wfkind = mykind; f.wfs = myfs; }
            if (myev == gev && myev != kNone) f.wevs = myevs;
            if (rend - 1 >= j0 && rend - 1 < j0 + kWC && rend - 1 >= start) f.wends = mylast;
            __syncthreads();
            const int kind = f.wfkind;
            const float fs = f.wfs, evs = f.wevs, ends = f.wends;
            const float snext = (rend < cend && gfail == kNone) ? f.ss[nseg > (uint32_t)nused ? nused : nok] : 0.0f;
            __syncthreads();
            F_TS(tsb + 6);
            if (gev < gfail) { *s_out = evs; return gev; }
            if (gfail != kNone) {
                if (kind == kWFailBin) {
                    F_STAT(14, gfail);
                    F_STAT(15, (int)(uint32_t)ldg(items + gfail) | ((int)f_is_bin(ldg(items + gfail)) << 31));
                    F_STAT(13, N);
                    *s_out = s;
                    F_WFAIL();
                }
                s = fs;
                if (kind == kWFailCross) {
                    if (w_pred(wa, s)) { *s_out = s; return gfail; }
                    start = gfail + 1;
                } else {
                    start = gfail;
                }
            } else if (rend >= cend) {
                s = rend > start ? ends : s;
                start = cend;
            } else {
                s = snext;
                start = rend;
            }
            if (start >= cend) break;
        }
        pos = cend;
    }
    *s_out = s;
    return N;
}

// ---------------------------------------------------------------------------
// Rank of list entry `en` in the list segment [st, end): the number of
// entries greater than it (the order is key descending, then index
// ascending; removed entries are 0 and rank below every real one).
__device__ __forceinline__ uint32_t f_rank(const uint64_t *gl, uint32_t st, uint32_t end, uint64_t en)
{
    uint32_t rank = 0u, i = st;
    for (; i + 4u <= end; i += 4u) {
        const uint64_t a0 = ldg(gl + i), a1 = ldg(gl + i + 1), a2 = ldg(gl + i + 2), a3 = ldg(gl + i + 3);
        rank += (a0 > en) + (a1 > en) + (a2 > en) + (a3 > en);
    }
    for (; i < end; i++) rank += ldg(gl + i) > en;
    return rank;
}

// The walk items of bins [0, nb), in order: the overflow entries, then per
// bin either its list entries sorted (`lst(b)`: ranked within its list
// segment [seg, sege)) or one bin item (`item(b)`).  A listed bin's first
// item offset goes to v1[b].  Returns the item count, -1 if it does not fit.
//
// The listed segments are ranked in LDS: `stage` (stage_cap u64 words of
// LDS that the caller does not use at this point) holds a table of the
// segments (bin, staging offset, size, list offset), then their entries,
// so every entry counts the larger entries of its segment with LDS
// broadcast reads.  Segments past the staging room (in bin order) are
// ranked from the list in global memory.
constexpr int kFTab = 256;            // listed segments in the staging table
constexpr uint32_t kFStaged = 0x80000000u;   // v1 flag: the bin's segment is staged
struct FTabEnt { uint32_t x, y, z, w; };      // bin, staging offset, size, list offset
template <class Lst, class Item>
__device__ int f_items(RowSmem &sm, const uint64_t *gl, uint64_t *items, size_t icap, int nb, int nov,
                       Lst lst, Item item, uint64_t *stage, int stage_cap, int tsb)
{
    (void)tsb;
    F_TS(tsb + 0);
    FullSmem &f = sm.x.fs;
    const int t = threadIdx.x;
    constexpr int kPer = kFBins / kThreads;
    FTabEnt *tab = reinterpret_cast<FTabEnt *>(stage);
    int *hdr = reinterpret_cast<int *>(stage + 2 * kFTab);     // [0] staged end, [1] staged segments
    uint64_t *se = stage + 2 * kFTab + 2;
    const uint32_t se_cap = (uint32_t)(stage_cap - 2 * kFTab - 2);
    uint32_t n[kPer], sz[kPer], loc = 0, nl = 0, szl = 0;
    bool isl[kPer];
#pragma unroll
    for (int c = 0; c < kPer; c++) {
        const int b = kPer * t + c;
        n[c] = 0u;
        isl[c] = false;
        sz[c] = 0u;
        if (b < nb && f.cnt[b]) {
            isl[c] = lst(b);
            n[c] = isl[c] ? f.cnt[b] : (item(b) ? 1u : 0u);
            if (isl[c]) sz[c] = f.sege[b] - f.seg[b];
        }
        loc += n[c];
        nl += isl[c];
        szl += sz[c];
    }
    if (t == 0) { hdr[0] = 0x7fffffff; hdr[1] = 0; }
    uint32_t tot, nl_tot, sz_tot;
    uint32_t o = block_excl_u32(loc, &tot, sm) + (uint32_t)nov;
    if ((size_t)tot + nov > icap) return -1;
    uint32_t ti = block_excl_u32(nl, &nl_tot, sm);
    uint32_t so = block_excl_u32(szl, &sz_tot, sm);
#pragma unroll
    for (int c = 0; c < kPer; c++) {
        const int b = kPer * t + c;
        if (n[c]) {
            if (isl[c]) {
                const bool staged = ti < (uint32_t)kFTab && so + sz[c] <= se_cap;
                if (staged) {
                    tab[ti] = FTabEnt{(uint32_t)b, so, sz[c], f.seg[b]};
                    atomicMax(&hdr[1], (int)ti + 1);
                } else {
                    atomicMin(&hdr[0], (int)so);      // staged segments end before this one
                }
                f.v1[b] = o | (staged ? kFStaged : 0u);
                ti++;
                so += sz[c];
            } else {
                stg(items + o, f_bin_item(b));
            }
        }
        o += n[c];
    }
    __syncthreads();
    F_TS(tsb + 1);
    const int nst = hdr[1];
    const uint32_t send = min((uint32_t)hdr[0], sz_tot);
    // the staged segment holding staging position j (table in offset order)
    auto seg_of = [&](uint32_t j) {
        int lo = 0, hi = nst - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (tab[mid].y <= j) lo = mid;
            else hi = mid - 1;
        }
        return lo;
    };
    for (uint32_t j = t; j < send; j += kThreads) {
        const FTabEnt e = tab[seg_of(j)];
        se[j] = ldg(gl + e.w + (j - e.y));
    }
    // the overflow entries (above the bins), ranked among themselves: their
    // LDS copy equals the list's first nover entries
    const int nover = f.nover;
    for (int p = t; p < nover; p += kThreads) {
        const uint64_t en = f.over[p];
        if (!en) continue;
        uint32_t rk = 0u;
        for (int q = 0; q < nover; q++) rk += f.over[q] > en;
        stg(items + rk, en);
    }
    __syncthreads();
    F_TS(tsb + 2);
    for (uint32_t j = t; j < send; j += kThreads) {
        const FTabEnt e = tab[seg_of(j)];
        const uint64_t me = se[j];
        if (!me) continue;                          // a removed entry
        uint32_t rk = 0u;
        const uint64_t *sg = se + e.y;
        for (uint32_t q = 0; q < e.z; q++) rk += sg[q] > me;
        if (rk < f.cnt[e.x]) stg(items + (f.v1[e.x] & ~kFStaged) + rk, me);
        else f.fail = 1;
    }
    F_TS(tsb + 3);
    // segments that were not staged: ranked from the list
    if (nst < (int)nl_tot) f_list_for_each<4>(gl, (uint32_t)nover, f.list_end, [&](uint32_t, uint64_t en) {
        if (!en) return;
        const int b = f_bin(f_entry_y(en) - f.m0);
        if (b >= nb || !lst(b) || (f.v1[b] & kFStaged)) return;
        const uint32_t rk = f_rank(gl, f.seg[b], f.sege[b], en);
        if (rk < f.cnt[b]) stg(items + f.v1[b] + rk, en);
        else f.fail = 1;
    });
    __threadfence_block();
    __syncthreads();
    F_TS(tsb + 4);
#pragma unroll
    for (int c = 0; c < kPer; c++)
        if (isl[c]) f.v1[kPer * t + c] &= ~kFStaged;
    __syncthreads();
    return f.fail ? -1 : (int)tot + nov;
}

// Bag bins of accumulation sq: the exact increments of their list entries
// are summed into v1 / v3 (zeroed by the caller); rounding ties are set
// aside, and each bag bin that holds some gets its increment function in the
// tie table: the ties are visited in order, each after the bin's non-tie
// elements above it.
__device__ void f_bags(RowSmem &sm, const uint64_t *gl, const FSeq &c, int sq, float s2)
{
    FullSmem &f = sm.x.fs;
    const int t = threadIdx.x, lane = lane_id();
    uint32_t *val = sq == 3 ? f.v3 : f.v1;
    const int tsb = 54 + 3 * sq;   // timing builds: 57.. (seq 1), 60.. (seq 2), 63 (seq 3)
    (void)tsb;
    if (t == 0) f.nties = 0;
    F_TS(tsb);
    __syncthreads();
    auto grid = [&](int b) {
        return sq == 1 ? (int)((f.w1[b] >> 16) & 255u) - 128 : (int)f.ex[b][sq - 2] - 128;
    };
    f_list_for_each<8>(gl, (uint32_t)f.nover, f.list_end, [&](uint32_t, uint64_t en) {
        if (!en) return;
        const float y = f_entry_y(en);
        const int b = f_bin(y - f.m0);
        if (f_cls(f.w1[b], f.w23[b], sq) != kCBag) return;
        // the increment from the compensated fast exp (relative error below
        // kExpErr, plus half an ulp per division) when that decides its
        // rounding; else (near a half step, where a rounding tie may be, or
        // from 2^23 up) from the exact summand
        uint32_t dn, up, k;
        const float af = fast_exp(y - c.m);
        const float vf = sq == 1 ? af : ((sq == 2 || !c.nuc) ? af / c.S : (af / c.S) / s2);
        if (inc_of(ldexpf(vf, 23 - grid(b)), 2.0f * kExpErr, &k)) dn = up = k;
        else f_incs(f_val(c, sq, y, s2), grid(b), &dn, &up);
        if (dn >= (1u << 24)) { f.fail = 1; return; }
        if (dn == up) {
            atomicAdd(&val[b], dn);
        } else {
            const int slot = atomicAdd(&f.nties, 1);
            if (slot < kTieCap) f.ties[slot] = FullTie{en, (uint32_t)b | ((uint32_t)sq << 16), dn};
            else f.fail = 1;
        }
    });
    __syncthreads();
    F_TS(tsb + 1);
    const int nt = min(f.nties, kTieCap);
    for (int i = wave_id(); i < nt; i += kWaves) {
        const uint32_t key = f.ties[i].key;
        bool first = true;
        for (int j = 0; j < i; j++) first &= f.ties[j].key != key;
        if (!first) continue;
        const int b = (int)(key & 0xffffu);
        const int e = grid(b);
        const uint32_t st = f.seg[b], end = f.sege[b];
        // the bin's ties, in the walk's order (entry descending)
        uint64_t done = ~0ull;           // entries below this one remain
        uint64_t n0 = 0, n1 = 1;         // the sum in grid units from parity 0 / 1
        uint32_t acc = 0u;               // non-tie increments added so far
        for (int k = 0; k < nt; k++) {
            // next tie of this bin: the largest entry below `done`
            uint64_t best = 0ull;
            uint32_t bk = 0u;
            for (int j = 0; j < nt; j++) {
                if (f.ties[j].key != key) continue;
                const uint64_t ej = f.ties[j].en;
                if (ej < done && ej > best) { best = ej; bk = f.ties[j].k; }
            }
            if (!best) break;
            // non-tie increments of entries above it
            uint32_t above = 0u;
            for (uint32_t q = st + lane; q < end; q += 64) {
                const uint64_t eq = ldg(gl + q);
                if (!eq || eq <= best) continue;
                uint32_t dn, up;
                f_incs(f_val(c, sq, f_entry_y(eq), s2), e, &dn, &up);
                if (dn == up) above += dn;
            }
            for (int d = 32; d > 0; d >>= 1) above += __shfl_xor(above, d, 64);
            n0 += above - acc;
            n1 += above - acc;
            acc = above;
            n0 += bk + ((n0 + bk) & 1u);
            n1 += bk + ((n1 + bk) & 1u);
            done = best;
        }
        const uint32_t tot = val[b];
        n0 += tot - acc;
        n1 += tot - acc;
        if (lane == 0) {
            const int slot = atomicAdd(&f.ntiefn, 1);
            if (slot < kTieCap) {
                const uint64_t d0 = n0, d1 = n1 - 1u;
                f.tiefn[slot] = FullTieFn{key, d0 > kSat ? kSat : (uint32_t)d0, d1 > kSat ? kSat : (uint32_t)d1};
                if (sq == 1) atomicOr(&f.w1[b], kW1TieFn);
                else atomicOr(&f.w23[b], sq == 2 ? kW3TieFn2 : kW3TieFn3);
            } else {
                f.fail = 1;
            }
        }
    }
    __syncthreads();
}

// The exact full-vocabulary path.  Returns true with *tok / *status set, or
// false to hand the row to the sort-based path.  `gl` is the row's scratch
// (lcap u64 words).
__device__ bool full_v2_row(RowSmem &sm, const float *row, int V, float T, float top_p, bool has_pen, float r,
                            uint64_t *gl, size_t lcap, int *tok, int *status)
{
    FullSmem &f = sm.x.fs;
    const int t = threadIdx.x;
    constexpr int kPer = kFBins / kThreads;
    static_assert(kPer * kThreads == kFBins, "bins per thread");
    const bool t_one = (T == 1.0f);
    const bool nuc = top_p < 1.0f;
    // scratch: list | seq-1 walk items | seq-2/3 walk items | deferred ids
    const size_t lsz = (size_t)V + kFOverCap + 2 * kHashSlots;
    const size_t isz = (size_t)V + kFBins + kFOverCap + 2 * kHashSlots;
    if (lcap < lsz + 2 * isz + kFDeferCap / 2) F_FAIL();
    uint64_t *items1 = gl + lsz;
    uint64_t *items = items1 + isz;
    uint32_t *defer = reinterpret_cast<uint32_t *>(items + isz);
    // the row need only be 4-byte aligned: the float4 passes start at the
    // first 16-byte boundary (element h0 < 4); the elements before it are
    // visited one per thread
    const int h0 = (int)(((16u - ((uint32_t)reinterpret_cast<uintptr_t>(row) & 15u)) & 15u) >> 2);
    const float4 *r4 = reinterpret_cast<const float4 *>(row + h0);
    const int n4 = (V - h0) >> 2;
    if (V < h0 || n4 == 0) F_FAIL();
    auto ydiv = [&](float x) { return t_one ? x : x / T; };
    auto pen_y = [&](int s) { return ydiv(__uint_as_float(sm.hval[s])); };

    for (int b = t; b < kFBins; b += kThreads) { f.cnt[b] = 0u; f.v1[b] = 0u; }
    for (int b = t; b < kFMassBins; b += kThreads) f.u.mass64[b] = 0ull;
    if (t < 32) f.exptab[t] = kExp2Tab[t];
    if (t == 0) { f.nover = 0; f.nrec = 0; f.fail = 0; f.ndefer = 0; f.ntiefn = 0; }

    // ---- pass 1 (HBM): counts, masses of the top bins, max, NaN -------------
    float tmax = -INFINITY;
    int nan = 0;
    float m0 = 0.0f;
    auto visit1 = [&](int i, float y) {
        nan |= (int)isnan(y);
        if (y > tmax && !(has_pen && hash_find(sm, (uint32_t)i) >= 0)) tmax = y;
        const float dp = y - m0;
        if (dp > kFDUp) {
            const int slot = atomicAdd(&f.nover, 1);
            if (slot < kFOverCap) f.over[slot] = f_entry(y, (uint32_t)i);
        } else if (dp >= -kFDLo) {
            const int b = f_bin(dp);
            atomicAdd(&f.cnt[b], 1u);
            if (b < kFMassBins)
                atomicAdd((unsigned long long *)&f.u.mass64[b], (unsigned long long)(fast_exp(dp) * kFMassScale));
        }
    };
    // The loop is instantiated for T == 1 and for a division, so that rows
    // with T == 1 carry no division (a select would compute it anyway).
    auto pass1 = [&](auto yf) -> bool {
        for (int base = 0; base < n4; base += kThreads * kUnroll) {
            float4 v[kUnroll];
#pragma unroll
            for (int u = 0; u < kUnroll; u++) v[u] = ldg(r4 + min(base + u * kThreads + t, n4 - 1));
            if (base == 0) {
                float lm = -INFINITY;
#pragma unroll
                for (int u = 0; u < kUnroll; u++)
                    if (u * kThreads + t < n4) lm = fmaxf(lm, fmaxf(fmaxf(v[u].x, v[u].y), fmaxf(v[u].z, v[u].w)));
                m0 = ydiv(f_block_max(lm, sm));
                if (!isfinite(m0)) return false;
            }
#pragma unroll
            for (int u = 0; u < kUnroll; u++) {
                const int q = base + u * kThreads + t;
                if (q < n4) {
                    visit1(h0 + 4 * q + 0, yf(v[u].x));
                    visit1(h0 + 4 * q + 1, yf(v[u].y));
                    visit1(h0 + 4 * q + 2, yf(v[u].z));
                    visit1(h0 + 4 * q + 3, yf(v[u].w));
                }
            }
        }
        return true;
    };
    if (!(t_one ? pass1([](float x) { return x; }) : pass1([&](float x) { return x / T; }))) F_FAIL();
    for (int i = h0 + (n4 << 2) + t; i < V; i += kThreads) visit1(i, ydiv(ldg(row + i)));
    if (t < h0) visit1(t, ydiv(ldg(row + t)));
    if (has_pen) {
        for (int s = t; s < kHashSlots; s += kThreads) {
            if (sm.hkey[s] == kEmpty) continue;
            const float y = pen_y(s);
            nan |= (int)isnan(y);
            tmax = fmaxf(tmax, y);
        }
    }
    if (block_or(nan, sm) || sm.flag_nan) { *status = GS_ERR_NAN; *tok = 0; return true; }
    const float m = f_block_max(tmax, sm);
    *status = GS_OK;
    if (!isfinite(m) || m0 > m || f.nover > kFOverCap) F_FAIL();
    GS_STAMP(10);
    if (t == 0) { f.m = m; f.m0 = m0; }

    // ---- penalty: the raw values of penalized ids leave, their penalized
    // values join (exact counts; v1 counts the raw values per bin, which the
    // list segments must still hold room for) ----------------------------------
    if (has_pen) {
        for (int j = t; j < f.nover; j += kThreads)
            if (hash_find(sm, f_entry_id(f.over[j])) >= 0) f.over[j] = 0ull;
        __syncthreads();
        for (int s = t; s < kHashSlots; s += kThreads) {
            const uint32_t id = sm.hkey[s];
            if (id == kEmpty) continue;
            const float dr = ydiv(ldg(row + id)) - m0;
            if (dr <= kFDUp && dr >= -kFDLo) {
                const int b = f_bin(dr);
                atomicSub(&f.cnt[b], 1u);
                atomicAdd(&f.v1[b], 1u);
                if (b < kFMassBins)
                    atomicAdd((unsigned long long *)&f.u.mass64[b], 0ull - (unsigned long long)(fast_exp(dr) * kFMassScale));
            }
            const float yp = pen_y(s);
            const float dq = yp - m0;
            if (dq > kFDUp) {
                const int slot = atomicAdd(&f.nover, 1);
                if (slot < kFOverCap) f.over[slot] = f_entry(yp, id);
            } else if (dq >= -kFDLo) {
                const int b = f_bin(dq);
                atomicAdd(&f.cnt[b], 1u);
                if (b < kFMassBins)
                    atomicAdd((unsigned long long *)&f.u.mass64[b], (unsigned long long)(fast_exp(dq) * kFMassScale));
            }
        }
        __syncthreads();
        if (f.nover > kFOverCap) F_FAIL();
    }
    const int nover = f.nover;
    const FSeq c{m, 1.0f, nuc, f.exptab};
    const double wbin = (double)(kFDUp + kFDLo) / kFBins;
    const double shift = (double)m0 - (double)m;
    auto e_at = [&](double bpos) { return exp((double)kFDUp - bpos * wbin + shift); };
    const double dl = 1.0 - kFDelta, dh = 1.0 + kFDelta;

    F_TS(0);
    // ---- plan A (seq 1): the running sum before each bin, predicted from
    // the masses (top bins) and the counts times the rounded increment of the
    // bin's centre (the rest), refined twice; then each bin's class:
    //   listed-and-sorted (the sum may change binade in it, or the top bin),
    //   uniform, record (two increments), or bag (more) ---------------------
    {
        double osum = 0.0;
        for (int j = t; j < nover; j += kThreads) {
            const uint64_t en = f.over[j];
            if (en) osum += (double)glibc_expf_tab(f_entry_y(en) - m, f.exptab);
        }
        double otot;
        f_block_excl_f64_buf(osum, &otot, sm.red_f64);
        osum = otot;
        uint32_t cn[kPer];
        double mb[kPer], ctr[kPer];
        const double mscale = exp(shift) / (double)kFMassScale;
        double loc = 0.0;
#pragma unroll
        for (int q = 0; q < kPer; q++) {
            const int b = kPer * t + q;
            cn[q] = f.cnt[b];
            ctr[q] = e_at((double)b + 0.5);
            mb[q] = b < kFMassBins ? (double)(int64_t)f.u.mass64[b] * mscale : (double)cn[q] * ctr[q];
            if (mb[q] < 0.0) mb[q] = 0.0;
            loc += mb[q];
        }
        F_TS(1);
        double tot;
        double pre = f_block_excl_f64_buf(loc, &tot, sm.red_f64b) + osum;
        double ct[kPer];
        for (int round = 0; round < 2; round++) {
            double lo = pre;
            loc = 0.0;
#pragma unroll
            for (int q = 0; q < kPer; q++) {
                const int b = kPer * t + q;
                ct[q] = mb[q];
                if (b >= kFMassBins && cn[q] && lo > 0.0) {
                    const double g = ldexp(1.0, f_dexp(lo) - 23);
                    ct[q] = (double)cn[q] * rint(ctr[q] / g) * g;
                }
                lo += ct[q];
                loc += ct[q];
            }
            pre = f_block_excl_f64_buf(loc, &tot, round == 0 ? sm.red_f64 : sm.red_f64b) + osum;   // (buffers alternate)
        }
        __syncthreads();
#if defined(GS_TIMING) || defined(GS_DIAG)
        if (t == 0 && blockIdx.x < 1024) g_vdiag[blockIdx.x * 16 + 14] = __float_as_int((float)(tot + osum));
#endif
        F_TS(2);
        // classes (records overwrite the masses: every thread has read
        // them); the predicted sums before / after each bin go through LDS
        {
            double lo = pre;
#pragma unroll
            for (int q = 0; q < kPer; q++) {
                const int b = kPer * t + q;
                f.seg[b] = __float_as_uint((float)lo);
                lo += ct[q];
                f.sege[b] = __float_as_uint((float)lo);
            }
        }
        // (interleaved bins: the costly record bins spread over the threads)
        __syncthreads();
#pragma unroll 1
        for (int q = 0; q < kPer; q++) {
            const int b = t + q * kThreads;
            const double lo = (double)__uint_as_float(f.seg[b]), hi = (double)__uint_as_float(f.sege[b]);
            const uint32_t n = f.cnt[b];
            uint32_t cls = kCNone, rec = kNoRec, lvl = 0u;
            int e = 0;
            if (n) {
                if (b == 0 || !(lo > 0.0) || f_dexp(lo * dl) != f_dexp(hi * dh)) {
                    cls = kCLst;
                } else {
                    e = f_dexp(lo);
                    float ylo, yhi;
                    f_range(m0, b, &ylo, &yhi);
                    const int k = f_classify(c, 1, e, ylo, yhi, 1.0f, 1.0f, &lvl);
                    cls = k == 0 ? kCUni : kCBag;
                    if (k == 1 && n < 65536u) {
                        const int rr = atomicAdd(&f.nrec, 1);
                        if (rr < kRecCap) { f.u.rec[rr] = f_rec_pending(b, 1, e, lvl); rec = (uint32_t)rr; cls = kCRec; }
                    }
                }
            }
            const bool listed = cls == kCBag || cls == kCLst;
            f.w1[b] = cls | (rec << 3) | (listed ? kW1Listed : 0u) | ((uint32_t)(e + 128) << 16);
            const uint32_t cap = listed ? n + f.v1[b] : 0u;
            if (cls == kCLst && cap > (uint32_t)(16 * kThreads)) f.fail = 1;
            f.v1[b] = cls == kCBag ? 0u : lvl;
            f.sege[b] = cap;
        }
        F_TS(3);
        __syncthreads();
        f_thresholds(sm, c, m0, 1.0f, 1.0f);
        uint32_t capl = 0;
#pragma unroll
        for (int q = 0; q < kPer; q++) capl += f.sege[kPer * t + q];
        uint32_t ltot;
        uint32_t o = block_excl_u32(capl, &ltot, sm) + (uint32_t)nover;
#pragma unroll
        for (int q = 0; q < kPer; q++) {
            const int b = kPer * t + q;
            const uint32_t cap = f.sege[b];
            f.seg[b] = o;
            f.sege[b] = o;
            o += cap;
        }
        if (t == 0) f.list_end = (uint32_t)nover + ltot;
    }
    for (int j = t; j < nover; j += kThreads) stg(gl + j, f.over[j]);
    __syncthreads();
    GS_STAMP(11);
    if (f.fail || f.list_end > lsz) F_FAIL();

    // ---- pass 2 (cache): seq-1 record counts; listed bins written ----------
    auto visit2 = [&](int i, float y) {
        const float dp = y - m0;
        if (!(dp <= kFDUp) || dp < -kFDLo) return;
        const int b = f_bin(dp);
        const uint32_t w = f.w1[b];
        if ((w & 7u) == kCRec) {
            FullRec &rc = f.u.rec[(w >> 3) & kNoRec];
            if (y >= rc.up) atomicAdd(&rc.hi, 1u);
            else if (y >= rc.thr) atomicAdd(&rc.tie, 1u);
        } else if (w & kW1Listed) {
            const uint32_t slot = atomicAdd(&f.sege[b], 1u);
            if (slot < lsz) stg(gl + slot, f_entry(y, (uint32_t)i));
        }
    };
    // (non-temporal loads: the row streams past the L2 lines of the list
    // entries written here instead of evicting them half-written; measured,
    // the fetches of pass 3 do not grow)
    if (t_one) row_for_each_any<true>(row, V, visit2);
    else row_for_each_any<true>(row, V, [&](int i, float x) { visit2(i, x / T); });
    __syncthreads();
    if (has_pen) {
        // the raw values of penalized ids leave: listed entries are zeroed,
        // counted ones uncounted; then the penalized values are visited
        for (int s = t; s < kHashSlots; s += kThreads) {
            const uint32_t id = sm.hkey[s];
            if (id == kEmpty) continue;
            const float y = ydiv(ldg(row + id));
            const float dp = y - m0;
            if (!(dp <= kFDUp) || dp < -kFDLo) continue;
            const int b = f_bin(dp);
            const uint32_t w = f.w1[b];
            if (w & kW1Listed) {
                for (uint32_t p = f.seg[b]; p < f.sege[b]; p++)
                    if (ldg(gl + p) != 0ull && f_entry_id(ldg(gl + p)) == id) stg(gl + p, (uint64_t)0);
            } else if ((w & 7u) == kCRec) {
                FullRec &rc = f.u.rec[(w >> 3) & kNoRec];
                if (y >= rc.up) atomicSub(&rc.hi, 1u);
                else if (y >= rc.thr) atomicSub(&rc.tie, 1u);
            }
        }
        __threadfence_block();
        __syncthreads();
        for (int s = t; s < kHashSlots; s += kThreads)
            if (sm.hkey[s] != kEmpty) visit2((int)sm.hkey[s], pen_y(s));
        __threadfence_block();
        __syncthreads();
    }
    GS_STAMP(12);
    int nov = 0;
    for (int j = 0; j < nover; j++) nov += f.over[j] != 0ull;   // (the LDS copy of the list's first nover entries)
    f_bags(sm, gl, c, 1, 1.0f);
    if (f.fail) F_FAIL();
    GS_STAMP(13);

    // ---- walk seq 1: S (src/sampler.rs:54) -----------------------------------
    int N = f_items(sm, gl, items1, isz, kFBins, nov, [&](int b) { return (f.w1[b] & 7u) == kCLst; },
                    [&](int b) {
                        int eb;
                        bool ok;
                        const ParFn fn = f_item_fn(f, 1, b, &eb, &ok);
                        return ok && (fn.f0 | fn.f1) != 0u;
                    },
                    reinterpret_cast<uint64_t *>(f.w23), kFBins, 40);   // w23 and v3: unused until walk 1
    if (N < 0) F_FAIL();
    F_STAT(0, 0);
    F_STAT(1, 0);
    F_STAT(2, N);
    F_STAT(3, f.list_end);
    GS_STAMP(14);
    float S;
    {
        f_cache_fns(sm, 1, f.w23, f.v3);
        WArgs wa{c, 1, 1.0f, 0, 0.0f, f.w23, f.v3};
        if (f_walk(sm, items1, N, wa, &S, 8) != N) F_FAIL();
    }
    if (!(S > 0.0f) || !isfinite(S)) F_FAIL();
    F_STAT(11, __float_as_int(S));
    GS_STAMP(16);
    const FSeq c2{m, S, nuc, f.exptab};

    // ---- plan B (seqs 2, 3): masses per bin, the cut and the draw; classes --
    {
        // masses of the listed-and-sorted bins (fast exp: a prediction), in 2^-40 units (u64
        // sums in w23 and v3: the same result in any order)
        uint64_t *mf = reinterpret_cast<uint64_t *>(f.w23);
        static_assert(offsetof(FullSmem, v3) == offsetof(FullSmem, w23) + 4 * kFBins, "w23, v3 adjacent");
        for (int b = t; b < kFBins; b += kThreads) mf[b] = 0ull;
        __syncthreads();
        F_TS(5);
        f_list_for_each<8>(gl, (uint32_t)nover, f.list_end, [&](uint32_t, uint64_t en) {
            if (!en) return;
            const float y = f_entry_y(en);
            const int b = f_bin(y - m0);
            if ((f.w1[b] & 7u) == kCLst)   // (a prediction: the fast exp is close enough)
                atomicAdd((unsigned long long *)&mf[b], (unsigned long long)ldexpf(fast_exp(y - m), 40));
        });
        F_TS(6);
        double osum = 0.0;
        for (int p = t; p < nover; p += kThreads) {
            const uint64_t en = ldg(gl + p);
            if (en) osum += (double)glibc_expf_tab(f_entry_y(en) - m, f.exptab);
        }
        double otot;
        f_block_excl_f64_buf(osum, &otot, sm.red_f64b);
        osum = otot;
        double mass[kPer], loc = 0.0;
        uint32_t cn[kPer], w1[kPer];
#pragma unroll
        for (int q = 0; q < kPer; q++) {
            const int b = kPer * t + q;
            cn[q] = f.cnt[b];
            w1[q] = f.w1[b];
            mass[q] = 0.0;
            const uint32_t cls = w1[q] & 7u;
            if (cls == kCLst) {
                mass[q] = ldexp((double)mf[b], -40);
            } else if (cls != kCNone) {
                int eb;
                bool ok;
                const ParFn fn = f_item_fn(f, 1, b, &eb, &ok);
                mass[q] = ldexp(0.5 * ((double)fn.f0 + (double)fn.f1), eb - 23);
            }
            loc += mass[q];
        }
        double tot;
        const double pre = f_block_excl_f64(loc, &tot, sm) + osum;   // (barriers: masses and records read)
        tot += osum;
        F_TS(7);
        const double iS = 1.0 / (double)S;
        if (t == 0) { f.cutb = kFBins; f.nrec = 0; f.last2 = -1; f.last3 = -1; }
        __syncthreads();
        if (nuc) {
            if (tot * iS < (double)top_p * (1.0 + 2.0 * kFDelta)) F_FAIL();   // the cut may not happen
            double lo = pre;
#pragma unroll
            for (int q = 0; q < kPer; q++) {
                const double hi = lo + mass[q];
                if (cn[q] && hi * iS * dh >= (double)top_p) { atomicMin(&f.cutb, kPer * t + q); break; }
                lo = hi;
            }
        }
        __syncthreads();
        float s2lo = 1.0f, s2hi = 1.0f;
        if (nuc) {
            // s2 = the nucleus sum at the cut: >= top_p, and above it by at
            // most the cut element's summand (<= the largest of the cut bin,
            // or of the overflow when that may already reach top_p) plus a
            // rounding step
            const double vmax = osum * iS * dh >= (double)top_p ? iS : e_at((double)f.cutb) * 1.001 * iS;
            s2lo = top_p;
            s2hi = __double2float_ru((double)top_p + vmax + ldexp((double)top_p, -22));
        }
        F_TS(8);
        // the predicted sums before / after each bin go through LDS (w23, v3:
        // every thread has read the masses)
        {
            double lo = pre;
#pragma unroll
            for (int q = 0; q < kPer; q++) {
                const int b = kPer * t + q;
                f.w23[b] = __float_as_uint((float)lo);
                lo += mass[q];
                f.v3[b] = __float_as_uint((float)lo);
            }
        }
        int l23 = -1;
        __syncthreads();
#pragma unroll 1
        for (int q = 0; q < kPer; q++) {
            const int b = t + q * kThreads;      // interleaved (see plan A)
            const double lo = (double)__uint_as_float(f.w23[b]), hi = (double)__uint_as_float(f.v3[b]);
            const uint32_t n = f.cnt[b];
            const double c2lo = lo * iS, c2hi = hi * iS;
            const bool rel2 = nuc && n && c2lo * dl < (double)top_p;
            // seq 3 over the whole range of s2: the lowest sum before the bin
            // and the highest after it
            const double c3lo = c2lo / (double)s2hi, c3hi = c2hi / (double)s2lo;
            const bool rel3 = n && (nuc ? rel2 : true) && c3lo * dl <= (double)r;
            const bool listed2 = (f.w1[b] & kW1Listed) != 0u;
            uint32_t cl2 = kCNone, cl3 = kCNone, r2 = kNoRec, r3 = kNoRec, lvl2 = 0u, lvl3 = 0u;
            int e2 = 0, e3 = 0;
            float ylo = 0.0f, yhi = 0.0f, alo = 0.0f, ahi = 0.0f;
            if (rel2 || rel3) {
                f_range(m0, b, &ylo, &yhi);
                alo = glibc_expf_tab(ylo - c2.m, c2.tab);
                ahi = glibc_expf_tab(yhi - c2.m, c2.tab);
            }
            if (rel2) {
                if (!(c2lo > 0.0) || f_dexp(c2lo * dl) != f_dexp(c2hi * dh) || c2hi * dh >= (double)top_p) {
                    cl2 = kCLst;
                } else {
                    e2 = f_dexp(c2lo);
                    const int k = f_classify_a(c2, 2, e2, alo, ahi, 1.0f, 1.0f, &lvl2);
                    cl2 = k == 0 ? kCUni : kCBag;
                    if (k == 1 && !listed2 && n < 65536u) {
                        const int rr = atomicAdd(&f.nrec, 1);
                        if (rr < kRecCap) { f.u.rec[rr] = f_rec_pending(b, 2, e2, lvl2); r2 = (uint32_t)rr; cl2 = kCRec; }
                    }
                }
            }
            if (rel3) {
                if (!(c3lo > 0.0) || f_dexp(c3lo * dl) != f_dexp(c3hi * dh) || c3hi * dh > (double)r) {
                    cl3 = kCLst;
                } else {
                    e3 = f_dexp(c3lo);
                    const int k = f_classify_a(c2, 3, e3, alo, ahi, s2lo, s2hi, &lvl3);
                    cl3 = k == 0 ? kCUni : kCBag;
                    if (k == 1 && !listed2 && n < 65536u) {
                        const int rr = atomicAdd(&f.nrec, 1);
                        if (rr < kRecCap) { f.u.rec[rr] = f_rec_pending(b, 3, e3, lvl3); r3 = (uint32_t)rr; cl3 = kCRec; }
                    }
                }
            }
            const bool need = cl2 == kCBag || cl2 == kCLst || cl3 == kCBag || cl3 == kCLst;
            const bool listed3 = !listed2 && need;
            // a listed bin's elements are all in the list: bags instead of records
            if (listed3 && cl2 == kCRec) { cl2 = kCBag; r2 = kNoRec; }
            if (listed3 && cl3 == kCRec) { cl3 = kCBag; r3 = kNoRec; }
            const bool visit = !listed2 && (listed3 || cl2 == kCRec || cl3 == kCRec);
            if ((cl2 == kCLst || cl3 == kCLst) && n > (uint32_t)(16 * kThreads)) f.fail = 1;
            f.w23[b] = cl2 | (cl3 << 3) | (r2 << 6) | (r3 << 16) | (listed3 ? kW3Listed : 0u) | (visit ? kW3Visit : 0u);
            f.ex[b][0] = (uint8_t)(e2 + 128);
            f.ex[b][1] = (uint8_t)(e3 + 128);
            f.v1[b] = cl2 == kCBag ? 0u : lvl2;
            f.v3[b] = cl3 == kCBag ? 0u : lvl3;
            if (listed3) f.sege[b] = n;        // + the raw values of penalized ids, below
            if (rel2 || rel3) l23 = max(l23, b);
        }
        F_TS(9);
        if (l23 >= 0) atomicMax(&f.last3, l23);
        __syncthreads();
        f_thresholds(sm, c2, m0, s2lo, s2hi);
        // list segments of the bins listed in pass 3 (room for raw values of
        // penalized ids too)
        if (has_pen) {
            for (int s = t; s < kHashSlots; s += kThreads) {
                const uint32_t id = sm.hkey[s];
                if (id == kEmpty) continue;
                const float dr = ydiv(ldg(row + id)) - m0;
                if (dr <= kFDUp && dr >= -kFDLo) {
                    const int b = f_bin(dr);
                    if (f.w23[b] & kW3Listed) atomicAdd(&f.sege[b], 1u);
                }
            }
        }
        __syncthreads();
        uint32_t capv[kPer], capl = 0;
#pragma unroll
        for (int q = 0; q < kPer; q++) {
            const int b = kPer * t + q;
            capv[q] = (f.w23[b] & kW3Listed) ? f.sege[b] : 0u;
            capl += capv[q];
        }
        uint32_t ltot;
        uint32_t o = block_excl_u32(capl, &ltot, sm) + f.list_end;
#pragma unroll
        for (int q = 0; q < kPer; q++) {
            const int b = kPer * t + q;
            if (capv[q]) { f.seg[b] = o; f.sege[b] = o; }
            o += capv[q];
        }
        __syncthreads();
        if (t == 0) f.list_end += ltot;
        __syncthreads();
        if (f.fail || f.list_end > lsz) F_FAIL();
    }
    GS_STAMP(17);

    // ---- pass 3 (cache): seq-2 and seq-3 record counts, bins listed, seq-3
    // deferrals ---------------------------------------------------------------
    auto visit3 = [&](int i, float y, uint32_t flag) {
        const float dp = y - m0;
        if (!(dp <= kFDUp) || dp < -kFDLo) return;
        const int b = f_bin(dp);
        const uint32_t w = f.w23[b];
        if (!(w & kW3Visit)) return;
        if (w & kW3Listed) {
            const uint32_t slot = atomicAdd(&f.sege[b], 1u);
            if (slot < lsz) stg(gl + slot, f_entry(y, (uint32_t)i));
            return;
        }
        if ((w & 7u) == kCRec) {
            FullRec &rc = f.u.rec[(w >> 6) & kNoRec];
            if (y >= rc.up) atomicAdd(&rc.hi, 1u);
            else if (y >= rc.thr) atomicAdd(&rc.tie, 1u);
        }
        if (((w >> 3) & 7u) == kCRec) {
            FullRec &rc = f.u.rec[(w >> 16) & kNoRec];
            if (y >= rc.up) atomicAdd(&rc.hi, 1u);
            else if (y >= rc.thr) {
                if (!nuc) atomicAdd(&rc.tie, 1u);
                else {
                    const uint32_t slot = atomicAdd((uint32_t *)&f.ndefer, 1u);
                    if (slot < kFDeferCap) stg(defer + slot, (uint32_t)i | flag);
                }
            }
        }
    };
    // (the row's last pass: non-temporal loads, so the row does not push the
    // partly written list lines out of L2)
    if (t_one) row_for_each_any<true>(row, V, [&](int i, float y) { visit3(i, y, 0u); });
    else row_for_each_any<true>(row, V, [&](int i, float x) { visit3(i, x / T, 0u); });
    __syncthreads();
    if (has_pen) {
        for (int s = t; s < kHashSlots; s += kThreads) {
            const uint32_t id = sm.hkey[s];
            if (id == kEmpty) continue;
            const float y = ydiv(ldg(row + id));
            const float dp = y - m0;
            if (!(dp <= kFDUp) || dp < -kFDLo) continue;
            const int b = f_bin(dp);
            const uint32_t w = f.w23[b];
            if (!(w & kW3Visit)) continue;
            if (w & kW3Listed) {
                for (uint32_t p = f.seg[b]; p < f.sege[b]; p++)
                    if (ldg(gl + p) != 0ull && f_entry_id(ldg(gl + p)) == id) stg(gl + p, (uint64_t)0);
                continue;
            }
            if ((w & 7u) == kCRec) {
                FullRec &rc = f.u.rec[(w >> 6) & kNoRec];
                if (y >= rc.up) atomicSub(&rc.hi, 1u);
                else if (y >= rc.thr) atomicSub(&rc.tie, 1u);
            }
            if (((w >> 3) & 7u) == kCRec) {   // a deferred raw value is skipped when the deferrals are resolved
                FullRec &rc = f.u.rec[(w >> 16) & kNoRec];
                if (y >= rc.up) atomicSub(&rc.hi, 1u);
                else if (y >= rc.thr && !nuc) atomicSub(&rc.tie, 1u);
            }
        }
        __threadfence_block();
        __syncthreads();
        for (int s = t; s < kHashSlots; s += kThreads)
            if (sm.hkey[s] != kEmpty) visit3((int)sm.hkey[s], pen_y(s), kFPen);
        __threadfence_block();
        __syncthreads();
    }
    GS_STAMP(18);
    if ((uint32_t)f.ndefer > kFDeferCap) F_FAIL();
    f_bags(sm, gl, c2, 2, 1.0f);
    if (!nuc) f_bags(sm, gl, c2, 3, 1.0f);
    if (f.fail) F_FAIL();
    GS_STAMP(19);

    // ---- walk seq 2: the cut and s2 (src/sampler.rs:59-67) -------------------
    const int nb23 = f.last3 + 1;
    auto lst23 = [&](int b) {
        const uint32_t w = f.w23[b];
        return (w & 7u) == kCLst || ((w >> 3) & 7u) == kCLst;
    };
    N = f_items(sm, gl, items, isz, nb23, nov, lst23, [&](int b) {
        const uint32_t w = f.w23[b];
        return (w & 7u) != kCNone || ((w >> 3) & 7u) != kCNone;
    }, reinterpret_cast<uint64_t *>(f.w1), kFBins / 2, 48);   // w1: unused after plan B until walk 2
    GS_STAMP(20);
    if (N < 0) F_FAIL();
    F_STAT(4, N);
    F_STAT(5, f.list_end);
    F_STAT(6, f.ndefer);
    F_STAT(7, f.nrec);
    float s2 = 1.0f;
    int n3 = N;
    uint32_t cut_id = 0u;
    if (nuc) {
        f_cache_fns(sm, 2, f.w1, f.v1);
        WArgs wa{c2, 2, 1.0f, 1, top_p, f.w1, f.v1};
        const int jc = f_walk(sm, items, N, wa, &s2, 9);
        if (jc < 0 || jc >= N) F_FAIL();
        cut_id = f_entry_id(ldg(items + jc));
        n3 = jc + 1;
        F_STAT(12, __float_as_int(s2));
        F_STAT(13, cut_id);
        // deferred seq-3 elements: exact increments now that s2 is exact
        const int nd = f.ndefer;
        for (int j = t; j < nd; j += kThreads) {
            const uint32_t en = ldg(defer + j);
            const uint32_t id = en & ~kFPen;
            float y;
            if (en & kFPen) {
                const int hs = hash_find(sm, id);
                if (hs < 0) { f.fail = 1; continue; }
                y = pen_y(hs);
            } else {
                if (has_pen && hash_find(sm, id) >= 0) continue;   // its raw value left the row
                y = ydiv(ldg(row + id));
            }
            const int b = f_bin(y - m0);
            const uint32_t w = f.w23[b];
            if (((w >> 3) & 7u) != kCRec) { f.fail = 1; continue; }
            const uint32_t r3 = (w >> 16) & kNoRec;
            const uint32_t lvl = f.v3[b];
            uint32_t dn, up;
            f_incs(f_val(c2, 3, y, s2), (int)f.ex[b][1] - 128, &dn, &up);
            if (dn == lvl + 1u) atomicAdd(&f.u.rec[r3].hi, 1u);
            else if (up == lvl + 1u) atomicAdd(&f.u.rec[r3].tie, 1u);
            else if (dn != lvl || up != lvl) f.fail = 1;
        }
        __syncthreads();
        f_bags(sm, gl, c2, 3, s2);
        if (f.fail) F_FAIL();
    }
    GS_STAMP(21);

    // ---- walk seq 3: the draw (src/sampler.rs:71-78) ---------------------------
    {
        f_cache_fns(sm, 3, f.w1, f.v1);
        WArgs wa{c2, 3, s2, 2, r, f.w1, f.v1};
        float c3;
        const int jd = f_walk(sm, items, n3, wa, &c3, 10);
        if (jd < 0) F_FAIL();
        if (jd < n3) *tok = (int)f_entry_id(ldg(items + jd));
        else if (nuc) *tok = (int)cut_id;
        else F_FAIL();   // the last element of the whole order: sort path
    }
    GS_STAMP(22);
    return true;
}
