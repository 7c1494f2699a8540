// gs_bins.hpp -- exact full-vocabulary sampling without sorting the row.
// (Included inside namespace gs by gs_kernels.hip, after RowSmem and the
// block helpers.)
//
// The reference (src/sampler.rs:44-78) sorts all V scaled logits y, then runs
// three sequential f32 accumulations in sorted order:
//   seq 1  S = sum of e_j = expf(y_j - max)                  (:54)
//   seq 2  cum of p_j = e_j / S until cum >= top_p: cut, s2   (:61-67)
//   seq 3  cum of q_j = p_j / s2 (or p_j) until r < cum       (:74-75)
// Inside one binade of the running sum an f32 add is integer arithmetic on
// multiples of the grid g (block_seqsum, gs_block.hpp), so the contribution
// of a set of elements is order independent -- unless the running sum leaves
// the binade inside the set, or an element is an exact rounding tie (its
// rounding then depends on the parity of the sum before it).  So:
//   pass 1 (HBM)   counts the elements of each bin of d' = y - m0 (m0 = max
//                  of the first round of loads); the exact max; NaNs.
//   plan (LDS)     predicts from the counts the binade of each accumulation
//                  at each bin; bins where an accumulation may change binade,
//                  reach top_p or r, or meet likely ties are "collected".
//                  Every bin owns a segment of a per-row list in global
//                  scratch, in bin order.
//   pass 2 (cache) collected bins write (key, index) to their segment; every
//                  other element adds its integer increment of each
//                  accumulation to its bin.  Elements whose increment the fast
//                  exp cannot decide are deferred.
//   resolve (LDS)  deferred elements get exact increments from the exact
//                  expf; S is bracketed by two walks (ties rounded down /
//                  up); bins holding a tie, or an increment the brackets of S
//                  and s2 cannot decide, are marked for collection.
//   pass 3 (cache) only if bins were marked: collects them.
//   walk (LDS)     replays each accumulation: consecutive collected bins form
//                  a group replayed exactly by block_seqsum over its sorted
//                  segments; the bulk bins between two groups form a run that
//                  is one integer add.
// Every prediction is checked; a failed check returns false and the caller
// uses the sort-based path.  Elements with d < -18.5 (e < 2^-26) add +0 to
// all three sums (below half a grid step of every running sum).

constexpr float kDUp = 3.0f;
constexpr float kDLo = 18.5f;
constexpr float kInvW = (float)kBins / (kDUp + kDLo);
// Bins b < kMassBins (d' > 3 - kMassBins/kInvW, about -3) get exact masses
// in pass 1: their elements are few and large, so count times the bin's
// central value is too coarse for the running-sum plan there.
constexpr int kMassBins = 1143;
constexpr float kMassScale = 4294967296.0f;       // fixed point 2^32
constexpr float kDelta = 1.0f / 4096.0f;          // relative margin of the plan
constexpr float kExpErr = 1.0f / 4194304.0f;      // bound on |fast_exp / expf - 1| (2^-22)
constexpr float kTieThr = 1.0f / 8.0f;            // expected ties that force collection
constexpr int kNoRun = 0x7fffffff;
constexpr int kMaxSeg = 512;                      // largest collected bin (wave sort)
constexpr uint32_t kNow = 0x80000000u;            // cnt[] flag: collect in the next pass
constexpr uint32_t kMetaCol = 1u, kMetaNow = 0x80u;  // meta flags: collected / collect in the next pass
constexpr uint32_t kDeferCapG = 65536;            // deferred elements per row
constexpr uint32_t kWalkCap = 65536;              // items of the walk array per row
// deferred entry: id | bit 31 penalized value | bit 30 seq-2 done (its
// increment added) | bit 29 seq-3 increment pending (merged pass 3)
constexpr uint32_t kDone2 = 0x40000000u, kPend3 = 0x20000000u, kIdMask = 0x1fffffffu;

__device__ __forceinline__ int bin_of(float dp)
{
    int b = (int)((kDUp - dp) * kInvW);
    return b > kBins - 1 ? kBins - 1 : b;
}

// bin_of for any dp (out-of-range values land in the end bins).
__device__ __forceinline__ int bin_clamp(float dp)
{
    const int b = (int)((kDUp - dp) * kInvW);
    return min(max(b, 0), kBins - 1);
}

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

// meta: bit0 collected, bit1 seq-2 increments needed, bit2 seq-3 increments
// needed, bit3 nonempty, bits 4..6 seq-1 ties, bit7 collect in the next pass;
// bytes 1..3 = b1, b2, b3 + 128.
__device__ __forceinline__ int meta_b(uint32_t mt, int which) { return (int)((mt >> (8 * which)) & 255u) - 128; }

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

// Exact increment of an exact summand at grid exponent b.  Returns 0 on a
// rounding tie (*k = the lower choice), 1 otherwise, -1 if out of range.
__device__ __forceinline__ int inc_exact(float a, int b, uint32_t *k)
{
    float m = ldexpf(a, 23 - b);
    if (!(m < 16777216.0f)) return -1;
    float fl = floorf(m);
    float fr = m - fl;
    *k = (uint32_t)fl + (fr > 0.5f ? 1u : 0u);
    return fr != 0.5f ? 1 : 0;
}

// Failure exit of the binned path (development builds record the line).
__device__ __forceinline__ bool bins_fail(int line)
{
#ifdef GS_TIMING
    if (threadIdx.x == 0) atomicAdd((unsigned long long *)&g_stamp[24], 1ull);
    if (threadIdx.x == 0 && blockIdx.x == g_row) g_stamp[25] = (uint64_t)line;
    if (threadIdx.x == 0 && blockIdx.x < 1024) g_fails[blockIdx.x] = line;
#endif
    (void)line;
    return false;
}
#define BINS_FAIL() return bins_fail(__LINE__)

// ---------------------------------------------------------------------------
__device__ float block_max_f(float v, RowSmem &sm)
{
    for (int d = 32; d > 0; d >>= 1) v = fmaxf(v, __shfl_xor(v, d, 64));
    if (lane_id() == 0) sm.red_f32[wave_id()] = v;
    __syncthreads();
    float r = sm.red_f32[0];
    for (int i = 1; i < kWaves; i++) r = fmaxf(r, sm.red_f32[i]);
    __syncthreads();
    return r;
}

__device__ double block_excl_f64(double v, double *tot, RowSmem &sm)
{
    const int lane = lane_id(), w = wave_id();
    double incl = v;
    for (int d = 1; d < 64; d <<= 1) {
        double o = __shfl_up(incl, d, 64);
        if (lane >= d) incl += o;
    }
    if (lane == 63) sm.red_f64[w] = incl;
    __syncthreads();
    double pre = 0.0, all = 0.0;
    for (int i = 0; i < kWaves; i++) { if (i < w) pre += sm.red_f64[i]; all += sm.red_f64[i]; }
    __syncthreads();
    *tot = all;
    return pre + incl - v;
}

__device__ double block_sum_f64(double v, RowSmem &sm)
{
    double tot;
    block_excl_f64(v, &tot, sm);
    return tot;
}

// Exclusive scan with "last nonzero value" (0 = none), `init` before the
// first thread.
__device__ int block_excl_last(int v, int init, RowSmem &sm)
{
    const int lane = lane_id(), w = wave_id();
    int incl = v;
    for (int d = 1; d < 64; d <<= 1) {
        int o = __shfl_up(incl, d, 64);
        if (lane >= d && incl == 0) incl = o;
    }
    if (lane == 63) sm.red_i32[w] = incl;
    __syncthreads();
    int pre = init;
    for (int i = 0; i < w; i++) if (sm.red_i32[i]) pre = sm.red_i32[i];
    __syncthreads();
    int ex = __shfl_up(incl, 1, 64);
    if (lane == 0 || ex == 0) ex = pre;
    return ex;
}

// Sort the segment g[0..n) descending with one wave: the segment is loaded
// into registers (C entries per lane), ranks come from v_readlane broadcasts,
// one scatter.  Removed entries (0) go last.
template <int C>
__device__ void wave_sort_c(uint64_t *g, int n)
{
    const int lane = lane_id();
    uint64_t mine[C];
    int rank[C];
#pragma unroll
    for (int c = 0; c < C; c++) {
        const int j = c * 64 + lane;
        mine[c] = j < n ? ldg(g + j) : 0ull;
        rank[c] = 0;
    }
#pragma unroll
    for (int cj = 0; cj < C; cj++) {
        const int lim = min(64, n - cj * 64);
        const uint32_t lo = (uint32_t)mine[cj], hi = (uint32_t)(mine[cj] >> 32);
        for (int l = 0; l < lim; l++) {
            const uint64_t o = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)hi, l) << 32) |
                               (uint32_t)__builtin_amdgcn_readlane((int)lo, l);
            const int j = cj * 64 + l;
#pragma unroll
            for (int c = 0; c < C; c++)
                rank[c] += (o > mine[c]) | ((o == mine[c]) & (j < c * 64 + lane));
        }
    }
#pragma unroll
    for (int c = 0; c < C; c++) {
        const int j = c * 64 + lane;
        if (j < n) stg(g + rank[c], mine[c]);
    }
}

// False if n > kMaxSeg.
__device__ bool wave_sort_segment(uint64_t *g, int n)
{
    if (n <= 1) return true;
    if (n <= 64) wave_sort_c<1>(g, n);
    else if (n <= 128) wave_sort_c<2>(g, n);
    else if (n <= 256) wave_sort_c<4>(g, n);
    else if (n <= kMaxSeg) wave_sort_c<8>(g, n);
    else return false;
    return true;
}

__device__ __forceinline__ uint64_t list_entry(float y, uint32_t i)
{
    return ((uint64_t)f2key(y) << 32) | (uint64_t)(~i);
}

// Groups and runs from the collected flags: a collected bin starts a group if
// the last nonempty bin before it is bulk; the overflow segment opens group 0.
// Bulk bins get their run index in cnt[].  Returns false on inconsistency.
__device__ bool build_groups(RowSmem &sm)
{
    BinsSmem &bn = sm.x.bn;
    const int t = threadIdx.x;
    constexpr int kPer = kBins / kThreads;
    int kind[kPer];
    int lastk = 0;
#pragma unroll
    for (int c = 0; c < kPer; c++) {
        const int b = kPer * t + c;
        const bool ne = bn.off[b + 1] > bn.off[b];
        kind[c] = !ne ? 0 : ((bn.meta[b] & 1u) ? 2 : 1);
        if (kind[c]) lastk = kind[c];
    }
    int prevk = block_excl_last(lastk, 2, sm);
    int starts[kPer];
    uint32_t nstart = 0;
#pragma unroll
    for (int c = 0; c < kPer; c++) {
        starts[c] = (kind[c] == 2 && prevk == 1) ? 1 : 0;
        if (kind[c]) prevk = kind[c];
        nstart += starts[c];
    }
    uint32_t tstart;
    const uint32_t xstart = block_excl_u32(nstart, &tstart, sm);
    const int G = 1 + (int)tstart;
    if (G > kMaxGroups) return false;
    for (int g = t; g < kMaxGroups; g += kThreads) { bn.gbeg[g] = 0xffffffffu; bn.gend[g] = 0u; }
    for (int g = t; g <= kMaxGroups; g += kThreads) { bn.runb[g] = kNoRun; bn.runt[g] = 0u; }
    __syncthreads();
    uint32_t gb = xstart;
#pragma unroll
    for (int c = 0; c < kPer; c++) {
        const int b = kPer * t + c;
        gb += starts[c];
        if (kind[c] == 2) {
            atomicMin(&bn.gbeg[gb], bn.off[b]);
            atomicMax(&bn.gend[gb], bn.off[b + 1]);
        } else if (kind[c] == 1) {
            const uint32_t mt = bn.meta[b];
            bn.cnt[b] = gb + 1;            // run between group gb and group gb+1
            const int packed = (int)(((mt >> 8) & 0xffffffu) | ((mt & 2u) << 23) | ((mt & 4u) << 23));
            const int old = atomicCAS(&bn.runb[gb + 1], kNoRun, packed);
            if (old != kNoRun && old != packed) bn.fail = 1;
            const uint32_t ties = (mt >> 4) & 7u;
            if (ties) atomicAdd(&bn.runt[gb + 1], ties);
        }
    }
    if (t == 0) {
        bn.ngroups = G;
        atomicMin(&bn.gbeg[0], 0u);
        atomicMax(&bn.gend[0], (uint32_t)bn.nover);
    }
    __syncthreads();
    return bn.fail == 0;
}

// Sum the bulk increments of accumulation `which` per run.
// (seq 3: from acc3 when given -- the merged pass 3 -- else from esum.)
__device__ void gather_runs(RowSmem &sm, int which, const uint32_t *acc3 = nullptr)
{
    BinsSmem &bn = sm.x.bn;
    const int t = threadIdx.x;
    for (int i = t; i <= bn.ngroups; i += kThreads) bn.run[i] = 0ull;
    __syncthreads();
    const uint32_t *src = which == 2 ? bn.k2 : (acc3 ? acc3 : bn.esum);   // seq 3 reuses esum
    for (int b = t; b < kBins; b += kThreads) {
        const uint32_t mt = bn.meta[b];
        if ((mt & 1u) || bn.off[b + 1] == bn.off[b]) continue;     // nonempty bulk bins only
        const uint32_t v = src[b];
        if (v) atomicAdd((unsigned long long *)&bn.run[bn.cnt[b]], (unsigned long long)v);
    }
    __syncthreads();
}

// ---------------------------------------------------------------------------
// Block-wide exact replay of one accumulation over the flat walk array:
// items are f32 summands, or run markers (a NaN whose payload is the run
// index) standing for a run's integer increment at the run's grid exponent.
// runfn(r, e, &f) gives the increment function of run r at grid exponent e,
// or false if the run cannot be applied there (wrong binade, missing
// increments).  Returns the stop index (first item after which pred holds),
// n if none, or -1 when an event falls on a run (the plan was wrong).
// Generalises block_seqsum (gs_block.hpp) to run items.
__device__ __forceinline__ bool is_marker(float v) { return isnan(v); }
__device__ __forceinline__ int marker_run(float v) { return (int)(__float_as_uint(v) & 0xffffu); }
__device__ __forceinline__ float make_marker(int r) { return __uint_as_float(0x7fc00000u | (uint32_t)r); }

// Run tables of one walk, built block-wide by make_walk_tab: per run r,
// inc[r] = (increment with seq-1 ties rounded up << 32) | increment with ties
// rounded down, each capped at kSat, or kBadInc if the run has no increments
// for this accumulation; ex[r] = packed planned grid exponents (rounded down
// | rounded up << 16, each + 512), kAnyEx where the increment is 0.
constexpr uint32_t kBadInc = 0xffffffffu;
constexpr int kAnyEx = 0xffff;
struct WalkTab {
    const uint64_t *inc;
    const int *ex;
    int G;
    int hi;                        // 1: use the ties-rounded-up half
};
__device__ void make_walk_tab(RowSmem &sm, int which)
{
    BinsSmem &bn = sm.x.bn;
    const int G = bn.ngroups;
    for (int r = threadIdx.x; r <= G; r += kThreads) {
        uint32_t lo = 0u, hi = 0u;
        int exl = kAnyEx, exh = kAnyEx;
        const int packed = bn.runb[r];
        if (r > 0 && packed != kNoRun) {
            const bool have = which == 1 || (which == 2 && (packed & (1 << 24))) || (which == 3 && (packed & (1 << 25)));
            if (!have) {
                lo = hi = kBadInc;
            } else {
                const uint64_t R = bn.run[r], Rh = R + (which == 1 ? bn.runt[r] : 0u);
                const int eb = ((packed >> (8 * (which - 1))) & 255) - 128;
                lo = R > kSat ? kSat : (uint32_t)R;
                hi = Rh > kSat ? kSat : (uint32_t)Rh;
                if (lo) exl = eb + 512;
                if (hi) exh = eb + 512;
            }
        }
        bn.run[r] = ((uint64_t)hi << 32) | lo;
        bn.wbase[r] = (uint32_t)(exl | (exh << 16));
    }
    __syncthreads();
}
__device__ __forceinline__ WalkTab walk_tab(const BinsSmem &bn, bool hi)
{
    return WalkTab{bn.run, reinterpret_cast<const int *>(bn.wbase), bn.ngroups, hi ? 1 : 0};
}
// Increment of a marker item at grid exponent e; *bad if the run cannot be
// applied there.  Reads the tables for any item (the index is clamped).
__device__ __forceinline__ uint32_t tab_inc(const WalkTab &T, float v, int e, bool *bad)
{
    const int r = min(marker_run(v), T.G);
    const uint64_t pk = T.inc[r];
    const int exw = T.ex[r];
    const uint32_t inc = T.hi ? (uint32_t)(pk >> 32) : (uint32_t)pk;
    const int ex = T.hi ? (int)((uint32_t)exw >> 16) : (exw & 0xffff);
    *bad = inc == kBadInc || (ex != kAnyEx && ex != e + 512);
    return inc == kBadInc ? 0u : inc;
}

// Exact replay of one accumulation over the walk array by a single wave,
// kWalkK consecutive items per lane (kWalkK * 64 items per step).  Items are
// f32 summands, or run markers (a NaN whose payload is the run index) that
// stand for a run's integer increment (tables from make_walk_tab).  Each
// step composes the lanes' increment functions with a DPP scan and checks
// each item in order for an event: a binade crossing, the predicate, or a
// run that does not apply.  Windows without rounding ties use plain integer
// sums at grids e and e + 1 and take one crossing within the step; windows
// with ties compose parity functions (ParFn) and restart after each event.
// The event's element is added with the reference's own f32 add.  Returns
// the first item after which pred holds, n if none, or -1 when an event
// falls on a run.  Wave-uniform result.
constexpr int kWalkK = 4;
template <class Pred>
__device__ int wave_walk(const float *W, int n, const WalkTab &T, Pred pred, float *s_out)
{
    const int lane = lane_id();
    float s = 0.0f;
    int pos = 0;
    while (pos < n && s == 0.0f) {               // 0 + a == a exactly
        const float v = ldg(W + pos);
        if (is_marker(v)) {
            bool bad;
            if (tab_inc(T, v, -126, &bad) != 0u || bad) { *s_out = s; return -1; }
        } else {
            s = s + v;
            if (pred(s)) { *s_out = s; return pos; }
        }
        pos++;
    }
    constexpr int kStep = 64 * kWalkK;
    float vn[kWalkK];
#pragma unroll
    for (int q = 0; q < kWalkK; q++) {
        const int i = pos + kWalkK * lane + q;
        vn[q] = i < n ? ldg(W + i) : 0.0f;
    }
    for (; pos < n; pos += kStep) {
        float v[kWalkK];
#pragma unroll
        for (int q = 0; q < kWalkK; q++) {
            v[q] = vn[q];
            const int i = pos + kStep + kWalkK * lane + q;   // prefetch the next window
            vn[q] = i < n ? ldg(W + i) : 0.0f;
        }
        const int lim = min(kStep, n - pos);
        int start = 0;
        while (start < lim) {
            const int e = grid_exp(s);
            const uint32_t M = (uint32_t)ldexpf(s, 23 - e);
            uint32_t k0[kWalkK], k1[kWalkK];
            bool bad0[kWalkK], bad1[kWalkK], valid[kWalkK], t0[kWalkK];
            bool anytie = false;
#pragma unroll
            for (int q = 0; q < kWalkK; q++) {
                const int idx = kWalkK * lane + q;
                valid[q] = idx >= start && idx < lim;
                const bool mk = is_marker(v[q]);
                bool rb0, rb1, et0, et1;
                const uint32_t r0 = tab_inc(T, v[q], e, &rb0), r1 = tab_inc(T, v[q], e + 1, &rb1);
                const uint32_t e0 = elem_inc(v[q], e, &et0), e1 = elem_inc(v[q], e + 1, &et1);
                k0[q] = !valid[q] ? 0u : (mk ? r0 : e0);
                k1[q] = !valid[q] ? 0u : (mk ? r1 : e1);
                bad0[q] = valid[q] && mk && rb0;
                bad1[q] = valid[q] && mk && rb1;
                t0[q] = valid[q] && !mk && et0;
                anytie |= valid[q] && !mk && (et0 || et1);
            }
            if (!__any(anytie)) {
                // ---- fast step: integer sums at grids e and e + 1 ----
                uint32_t l0 = 0, l1 = 0;
#pragma unroll
                for (int q = 0; q < kWalkK; q++) { l0 = sat_add(l0, k0[q]); l1 = sat_add(l1, k1[q]); }
                const uint32_t i0 = wave_scan_add(l0), i1 = wave_scan_add(l1);
                uint32_t b = i0 - l0;                        // grid-e increments before this lane's items
                uint32_t c1[kWalkK];                         // inclusive grid-(e+1) sums
                {
                    uint32_t acc = i1 - l1;
#pragma unroll
                    for (int q = 0; q < kWalkK; q++) { acc += k1[q]; c1[q] = acc; }
                }
                int qev = kWalkK;
#pragma unroll
                for (int q = 0; q < kWalkK; q++) {
                    if (qev == kWalkK) {
                        const uint32_t a = b + k0[q];
                        const bool ev = valid[q] && ((M + a) >= (1u << 24) || bad0[q] ||
                                                     pred(ldexpf((float)(M + a), e - 23)));
                        if (ev) qev = q;
                        else b = a;
                    }
                }
                const uint64_t mask = __ballot(qev < kWalkK);
                if (mask == 0) {
                    s = ldexpf((float)(M + (uint32_t)__builtin_amdgcn_readlane((int)b, (lim - 1) / kWalkK)), e - 23);
                    break;
                }
                const int L = __ffsll((unsigned long long)mask) - 1;
                const int q = __builtin_amdgcn_readlane(qev, L);
                float vq = v[0];
                uint32_t cq = c1[0];
#pragma unroll
                for (int k = 1; k < kWalkK; k++) if (q == k) { vq = v[k]; cq = c1[k]; }
                const float vL = rdl(vq, L);
                if (is_marker(vL)) { *s_out = s; return -1; }   // event on a run
                const int idx = kWalkK * L + q;
                const float sc = ldexpf((float)(M + (uint32_t)__builtin_amdgcn_readlane((int)b, L)), e - 23) + vL;
                s = sc;
                if (pred(sc)) { *s_out = s; return pos + idx; }
                start = idx + 1;
                if (grid_exp(sc) != e + 1) continue;         // not a one-binade crossing: restart
                // the rest of the window on the grid-(e+1) sums
                const uint32_t C = (uint32_t)__builtin_amdgcn_readlane((int)cq, L);
                const uint32_t M1 = (uint32_t)ldexpf(sc, 22 - e);
                int qev2 = kWalkK;
                uint32_t prev = i1 - l1;
#pragma unroll
                for (int q2 = 0; q2 < kWalkK; q2++) {
                    const int idx2 = kWalkK * lane + q2;
                    if (qev2 == kWalkK && idx2 > idx && valid[q2]) {
                        const uint32_t a = M1 + (c1[q2] - C);
                        if (a >= (1u << 24) || bad1[q2] || pred(ldexpf((float)a, e + 1 - 23))) qev2 = q2;
                    }
                    if (qev2 == kWalkK) prev = c1[q2];
                }
                const uint64_t mask2 = __ballot(qev2 < kWalkK);
                if (mask2 == 0) {
                    const uint32_t last = (uint32_t)__builtin_amdgcn_readlane((int)c1[kWalkK - 1], (lim - 1) / kWalkK);
                    s = ldexpf((float)(M1 + (last - C)), e + 1 - 23);
                    break;
                }
                const int L2 = __ffsll((unsigned long long)mask2) - 1;
                const int q2 = __builtin_amdgcn_readlane(qev2, L2);
                float v2 = v[0];
#pragma unroll
                for (int k = 1; k < kWalkK; k++) if (q2 == k) v2 = v[k];
                const float vL2 = rdl(v2, L2);
                if (is_marker(vL2)) { *s_out = s; return -1; }
                const int idx2 = kWalkK * L2 + q2;
                // prev: grid-(e+1) sum up to the item before idx2 (C right after the crossing)
                const uint32_t before2 = (uint32_t)__builtin_amdgcn_readlane((int)prev, L2);
                const float sc2 = ldexpf((float)(M1 + (before2 - C)), e + 1 - 23) + vL2;
                s = sc2;
                if (pred(sc2)) { *s_out = s; return pos + idx2; }
                start = idx2 + 1;
                continue;
            }
            // ---- step with ties: parity functions at grid e ----
            ParFn f[kWalkK];
#pragma unroll
            for (int q = 0; q < kWalkK; q++) {
                // a tie element: K + ((p + K) & 1), K the lower choice (elem_inc's value)
                const uint32_t K = k0[q];
                f[q].f0 = t0[q] ? K + (K & 1u) : k0[q];
                f[q].f1 = t0[q] ? K + ((K + 1u) & 1u) : k0[q];
            }
            ParFn loc = f[0];
#pragma unroll
            for (int q = 1; q < kWalkK; q++) loc = par_compose(loc, f[q]);
            const ParFn incl = wave_scan_incl(loc);
            ParFn ex;
            ex.f0 = __shfl_up(incl.f0, 1, 64);
            ex.f1 = __shfl_up(incl.f1, 1, 64);
            if (lane == 0) ex.f0 = ex.f1 = 0u;
            uint32_t b = par_apply(ex, M & 1u);
            int qev = kWalkK;
#pragma unroll
            for (int q = 0; q < kWalkK; q++) {
                if (qev == kWalkK) {
                    const uint32_t a = sat_add(b, par_apply(f[q], (M + b) & 1u));
                    const bool cross = (M + a) >= (1u << 24);
                    const bool ev = valid[q] && (cross || bad0[q] || pred(ldexpf((float)(M + a), e - 23)));
                    if (ev) qev = q;
                    else b = a;
                }
            }
            const uint64_t mask = __ballot(qev < kWalkK);
            if (mask == 0) {
                s = ldexpf((float)(M + (uint32_t)__builtin_amdgcn_readlane((int)b, (lim - 1) / kWalkK)), e - 23);
                break;
            }
            const int L = __ffsll((unsigned long long)mask) - 1;
            const int q = __builtin_amdgcn_readlane(qev, L);
            float vq = v[0];
#pragma unroll
            for (int k = 1; k < kWalkK; k++) if (q == k) vq = v[k];
            const float vL = rdl(vq, L);
            if (is_marker(vL)) { *s_out = s; return -1; }
            const uint32_t before = (uint32_t)__builtin_amdgcn_readlane((int)b, L);
            const float na = ldexpf((float)(M + before), e - 23) + vL;   // the reference's f32 add
            s = na;
            const int idx = kWalkK * L + q;
            if (pred(na)) { *s_out = s; return pos + idx; }
            start = idx + 1;
        }
    }
    *s_out = s;
    return n;
}

// Run wave_walk on wave 0 and hand the result to the whole block.
template <class Pred>
__device__ int walk(RowSmem &sm, const float *W, int n, int which, Pred pred, float *s_out)
{
    make_walk_tab(sm, which);
    if (wave_id() == 0) {
        float sv;
        const int r = wave_walk(W, n, walk_tab(sm.x.bn, false), pred, &sv);
        if (lane_id() == 0) { sm.seq.first = r; sm.seq.s = sv; }
    }
    __syncthreads();
    const int r = sm.seq.first;
    *s_out = sm.seq.s;
    __syncthreads();
    return r;
}

// Clear the unused tail of the collected segments selected by `sel` and sort
// them.
template <class Sel>
__device__ bool finish_segments(RowSmem &sm, uint64_t *gl, Sel sel)
{
    BinsSmem &bn = sm.x.bn;
    const int t = threadIdx.x;
    for (int b = t; b < kBins; b += kThreads) {
        if (!sel(b)) continue;
        for (uint32_t j = bn.cnt[b] & ~kNow; j < bn.off[b + 1]; j++) stg(gl + j, (uint64_t)0);
    }
    __threadfence_block();
    __syncthreads();
    bool ok = true;
    for (int b = wave_id(); b < kBins; b += kWaves)
        if (sel(b)) ok &= wave_sort_segment(gl + bn.off[b], (int)(bn.off[b + 1] - bn.off[b]));
    if (!ok) bn.fail = 1;
    __threadfence_block();
    __syncthreads();
    return bn.fail == 0;
}


// The flat walk array: per group g, a marker of run g, then the group's
// sorted entries as exact summands expf(y - m) (0 for removed entries);
// a final marker for the run after the last group.  WT holds token ids.
// Returns the item count, or -1 if it does not fit.
__device__ int build_walk(RowSmem &sm, const uint64_t *gl, float *W, uint32_t *WT, float m, float m0, bool mass)
{
    BinsSmem &bn = sm.x.bn;
    const int t = threadIdx.x;
    const int G = bn.ngroups;
    const uint32_t sz = (t < G) ? 1u + (bn.gend[t] - bn.gbeg[t]) : 0u;
    uint32_t tot;
    const uint32_t wb = block_excl_u32(sz, &tot, sm);
    if (t < G) bn.wbase[t] = wb;
    if (t == 0) bn.wbase[G] = tot;
    __syncthreads();
    const uint32_t N = tot + 1;
    if (N > kWalkCap) return -1;
    // one item per thread: group by binary search over the marker positions
    for (uint32_t w = t; w < N; w += kThreads) {
        int lo = 0, hi = G;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (bn.wbase[mid] <= w) lo = mid;
            else hi = mid - 1;
        }
        const uint32_t w0 = bn.wbase[lo];
        if (w == w0) {
            stg(W + w, make_marker(lo));
            stg(WT + w, 0xffffffffu);
            continue;
        }
        const uint64_t en = ldg(gl + bn.gbeg[lo] + (w - w0 - 1));
        const float y = key2f((uint32_t)(en >> 32));
        const float e = en ? glibc_expf(y - m) : 0.0f;
        stg(W + w, e);
        stg(WT + w, ~(uint32_t)en);
        // masses of collected bins (plan B); overflow entries are summed there
        if (mass && en && y - m0 <= kDUp) atomicAdd(reinterpret_cast<float *>(&bn.k2[bin_clamp(y - m0)]), e);
    }
    __threadfence_block();
    __syncthreads();
    return (int)N;
}

__device__ __forceinline__ float next_up(float v) { return __uint_as_float(__float_as_uint(v) + 1u); }

// Increment of p = e / S (src/sampler.rs:56) over every f32 S in [Slo, Shi]
// (at most 8 values).  Returns 2 if some value is a rounding tie, out of
// range, or the range is too wide; 0 if all give the same increment (*k);
// 1 if they differ (the increment waits for the exact S).
__device__ __forceinline__ int inc_s_range(float e, float Slo, float Shi, int b, uint32_t *k)
{
    int n = 0;
    uint32_t k0 = 0;
    bool same = true;
    for (float S = Slo; S <= Shi; S = next_up(S)) {
        if (++n > 8) return 2;
        uint32_t kk;
        if (inc_exact(e / S, b, &kk) != 1) return 2;
        if (n == 1) k0 = kk;
        else same &= kk == k0;
    }
    *k = k0;
    return same ? 0 : 1;
}

// Pass constants, kept in registers by the pass loops.
struct PassK {
    float m0, m, inv_s, inv_s2, hw2;
    int ixlim;                     // pass 3: record indices of bins <= ixlim
    float inv_s2c, hw3;            // merged pass 3: 1 / (centre of the s2 range), seq-3 tolerance
};
// Classification of one element: cl 0 nothing to do, 1 list it, 2 defer it,
// 3 add increment k to bin b.  Branch-free; one LDS read (meta).
struct Cls {
    int b, cl;
    uint32_t k;
    bool wix;                      // record the element index in its bin's segment
    uint32_t k3 = 0u;              // merged pass 3: seq-3 increment to add now
    uint32_t dfl = 0u;             // flags of a deferred entry (kDone2: k is added now; kPend3)
};
// Pass 2: accumulation 1 (src/sampler.rs:54).
__device__ __forceinline__ Cls classify1(const BinsSmem &bn, const PassK &K, float y)
{
    const float dp = y - K.m0;
    const bool inr = (dp <= kDUp) && (dp >= -kDLo);
    Cls c;
    c.b = bin_clamp(dp);
    const uint32_t mt = bn.meta[c.b];
    const bool ok = inc_of(ldexpf(fast_exp(y - K.m), 23 - meta_b(mt, 1)), 2.0f * kExpErr, &c.k);
    c.cl = !inr ? 0 : ((mt & kMetaCol) ? 1 : (ok ? 3 : 2));
    c.wix = false;
    return c;
}
// Pass 3: accumulation 2, p = e / S (src/sampler.rs:56, :61-63).
__device__ __forceinline__ Cls classify3(const BinsSmem &bn, const PassK &K, float y)
{
    const float dp = y - K.m0;
    const bool inr = (dp <= kDUp) && (dp >= -kDLo);
    Cls c;
    c.b = bin_clamp(dp);
    const uint32_t mt = bn.meta[c.b];
    const float p = fast_exp(y - K.m) * K.inv_s;
    const bool ok = inc_of(ldexpf(p, 23 - meta_b(mt, 2)), K.hw2, &c.k);
    c.cl = !inr ? 0 : ((mt & kMetaNow) ? 1 : (((mt & kMetaCol) || !(mt & 2u)) ? 0 : (ok ? 3 : 2)));
    c.wix = inr && c.b <= K.ixlim;
    return c;
}
// Pass 3 merged with pass 4 (rows with a nucleus cut and no penalty):
// accumulation 2 as classify3 and, in the bins before the predicted draw
// (meta bit 2), accumulation 3 with q = p / s2 for s2 known to a range
// (tolerance hw3).  An element either increment of which cannot be decided
// is deferred; the decided one is added now (dfl says which is pending).
__device__ __forceinline__ Cls classify3m(const BinsSmem &bn, const PassK &K, float y)
{
    const float dp = y - K.m0;
    const bool inr = (dp <= kDUp) && (dp >= -kDLo);
    Cls c;
    c.b = bin_clamp(dp);
    const uint32_t mt = bn.meta[c.b];
    const float p = fast_exp(y - K.m) * K.inv_s;
    const bool ok2 = inc_of(ldexpf(p, 23 - meta_b(mt, 2)), K.hw2, &c.k);
    uint32_t k3;
    const bool ok3 = inc_of(ldexpf(p * K.inv_s2c, 23 - meta_b(mt, 3)), K.hw3, &k3);
    const bool want3 = (mt & 4u) != 0u;
    const bool bulk2 = inr && !(mt & kMetaNow) && !(mt & kMetaCol) && (mt & 2u);
    const bool d2 = !ok2, d3 = want3 && !ok3;
    c.cl = !inr ? 0 : ((mt & kMetaNow) ? 1 : (!bulk2 ? 0 : ((d2 || d3) ? 2 : 3)));
    c.dfl = c.cl == 2 ? ((d2 ? 0u : kDone2) | (d3 ? kPend3 : 0u)) : 0u;
    c.k3 = (bulk2 && want3 && !d3) ? k3 : 0u;
    c.wix = inr && c.b <= K.ixlim;
    return c;
}
// Pass 4: accumulation 3, q = p / s2 (src/sampler.rs:68, :74-75).
__device__ __forceinline__ Cls classify4(const BinsSmem &bn, const PassK &K, float y)
{
    const float dp = y - K.m0;
    const bool inr = (dp <= kDUp) && (dp >= -kDLo);
    Cls c;
    c.b = bin_clamp(dp);
    const uint32_t mt = bn.meta[c.b];
    const float q = fast_exp(y - K.m) * K.inv_s * K.inv_s2;
    const bool ok = inc_of(ldexpf(q, 23 - meta_b(mt, 3)), 2.0f * kExpErr + 0x1p-22f, &c.k);
    c.cl = !inr ? 0 : ((mt & kMetaNow) ? 1 : (((mt & kMetaCol) || !(mt & 4u)) ? 0 : (ok ? 3 : 2)));
    c.wix = false;
    return c;
}

// One cached pass over the row, then over the penalized values: each element
// is listed (bins flagged kNow), deferred, or adds its increment to acc[b],
// as cls says.  Raw contributions of penalized ids are undone first.
template <class ClsF>
__device__ void bins_pass(RowSmem &sm, const float *row, int V, bool t_one, float T, bool has_pen,
                          uint64_t *gl, uint32_t *defer, uint32_t dcap, uint32_t *acc, uint32_t *ix, ClsF cls,
                          uint32_t *acc3 = nullptr)
{
    BinsSmem &bn = sm.x.bn;
    const int t = threadIdx.x;
    auto act = [&](int i, float y, const Cls &c, uint32_t flag) {
        if (c.wix) stg(ix + atomicAdd(&bn.icur[c.b], 1u), (uint32_t)i);
        if (c.cl == 1) {
            const uint32_t slot = atomicAdd(&bn.cnt[c.b], 1u) & ~kNow;
            stg(gl + slot, list_entry(y, (uint32_t)i));
        } else if (c.cl == 2) {
            const int slot = atomicAdd(&bn.ndefer, 1);
            if ((uint32_t)slot < dcap) stg(defer + slot, (uint32_t)i | flag | c.dfl);
            if ((c.dfl & kDone2) && c.k) atomicAdd(&acc[c.b], c.k);
        } else if (c.cl == 3 && c.k) {
            atomicAdd(&acc[c.b], c.k);
        }
        if (acc3 && c.k3) atomicAdd(&acc3[c.b], c.k3);
    };
    auto act0 = [&](int i, float y, const Cls &c) { act(i, y, c, 0u); };
    if (t_one) row_for_each_cls(row, V, [](float x) { return x; }, cls, act0);
    else row_for_each_cls(row, V, [T](float x) { return x / T; }, cls, act0);
    __syncthreads();
    if (!has_pen) return;
    for (int s = t; s < kHashSlots; s += kThreads) {
        const uint32_t id = sm.hkey[s];
        if (id == kEmpty) continue;
        const float x = ldg(row + id);
        const Cls c = cls(t_one ? x : x / T);
        if (c.cl == 3 && c.k) atomicAdd(&acc[c.b], 0u - c.k);
    }
    for (int b = t; b < kBins; b += kThreads) {
        if (!(bn.cnt[b] & kNow)) continue;
        for (uint32_t j = bn.off[b]; j < (bn.cnt[b] & ~kNow); j++)
            if (hash_find(sm, ~(uint32_t)ldg(gl + j)) >= 0) stg(gl + j, (uint64_t)0);
    }
    const int nd = min((uint32_t)bn.ndefer, dcap);
    for (int j = t; j < nd; j += kThreads)
        if (hash_find(sm, ldg(defer + j) & kIdMask) >= 0) stg(defer + j, 0xffffffffu);
    __threadfence_block();
    __syncthreads();
    for (int s = t; s < kHashSlots; s += kThreads) {
        const uint32_t id = sm.hkey[s];
        if (id == kEmpty) continue;
        const float yp = __uint_as_float(sm.hval[s]);
        const float y = t_one ? yp : yp / T;
        act((int)id, y, cls(y), 0x80000000u);
    }
    __syncthreads();
}

// List the elements of the bins flagged kNow (one pass over the row, then the
// penalized values), sort those segments and clear the flag.
__device__ bool collect_now(RowSmem &sm, const float *row, int V, bool t_one, float T, bool has_pen, uint64_t *gl)
{
    BinsSmem &bn = sm.x.bn;
    const int t = threadIdx.x;
    auto visit = [&](int i, float y) {
        const float dp = y - bn.m0;
        if (!(dp <= kDUp) || dp < -kDLo) return;
        const int b = bin_of(dp);
        if (bn.cnt[b] & kNow) {
            const uint32_t slot = atomicAdd(&bn.cnt[b], 1u) & ~kNow;
            stg(gl + slot, list_entry(y, (uint32_t)i));
        }
    };
    if (t_one) row_for_each(row, V, true, visit);
    else row_for_each(row, V, true, [&](int i, float x) { visit(i, x / T); });
    __syncthreads();
    if (has_pen) {
        for (int b = t; b < kBins; b += kThreads) {
            if (!(bn.cnt[b] & kNow)) continue;
            for (uint32_t j = bn.off[b]; j < (bn.cnt[b] & ~kNow); j++)
                if (hash_find(sm, ~(uint32_t)gl[j]) >= 0) gl[j] = 0ull;
        }
        __threadfence_block();
        __syncthreads();
        for (int s = t; s < kHashSlots; s += kThreads) {
            const uint32_t id = sm.hkey[s];
            if (id == kEmpty) continue;
            const float yp = __uint_as_float(sm.hval[s]);
            visit((int)id, t_one ? yp : yp / T);
        }
        __syncthreads();
    }
    return true;
}

// collect_now for rows whose bins were indexed in pass 3 (ix[off[b],
// icur[b]) holds every element of bin b <= ixlim): the flagged bins are
// listed from their index segments, one wave per bin, without a pass over
// the row.  Returns false if a flagged bin was not indexed.
__device__ bool collect_now_ix(RowSmem &sm, const float *row, bool t_one, float T, uint64_t *gl,
                               const uint32_t *ix)
{
    BinsSmem &bn = sm.x.bn;
    const int t = threadIdx.x, lane = lane_id();
    constexpr int kPer = kBins / kThreads;
    uint32_t nk = 0;
    bool bad = false;
#pragma unroll
    for (int c = 0; c < kPer; c++) {
        const int b = kPer * t + c;
        if (bn.cnt[b] & kNow) {
            nk++;
            bad |= b > bn.ixlim || bn.icur[b] != bn.off[b + 1];
        }
    }
    if (block_or((int)bad, sm)) return false;
    uint32_t tot;
    uint32_t ex = block_excl_u32(nk, &tot, sm);
#pragma unroll
    for (int c = 0; c < kPer; c++) {
        const int b = kPer * t + c;
        if (bn.cnt[b] & kNow) bn.nzc[ex++] = (uint32_t)b;
    }
    __syncthreads();
    for (uint32_t k = wave_id(); k < tot; k += kWaves) {
        const int b = (int)bn.nzc[k];
        for (uint32_t p = bn.off[b] + lane; p < bn.off[b + 1]; p += 64) {
            const uint32_t id = ldg(ix + p);
            const float x = ldg(row + id);
            const float y = t_one ? x : x / T;
            const uint32_t slot = atomicAdd(&bn.cnt[b], 1u) & ~kNow;
            stg(gl + slot, list_entry(y, id));
        }
    }
    __threadfence_block();
    __syncthreads();
    return true;
}

// Sort the segments of the kNow bins descending (entries are distinct; removed
// entries are 0), zero their unused tails and clear the flag.  Bins are
// monotone in the key, so a run of consecutive kNow bins (empty bins between
// them included) sorts as one range, and the position of a nonzero entry in
// its run is the number of nonzero entries of the run's earlier bins plus its
// rank inside its own bin; zeros take the slots after the last nonzero
// entry.  Work items are 64-entry chunks of the runs, spread over all waves;
// entries go to tmp (room for kWalkCap entries), then back.  False if a run
// exceeds kMaxRun entries or tmp is too small.  Uses gbeg/gend/wbase/runt/run
// as run tables (build_groups and build_walk rebuild them).
constexpr uint32_t kMaxRun = 16384;
__device__ bool finish_now(RowSmem &sm, uint64_t *gl, uint64_t *tmp)
{
    BinsSmem &bn = sm.x.bn;
    const int t = threadIdx.x, lane = lane_id();
    const float m0 = bn.m0;
    constexpr int kPer = kBins / kThreads;
    // kind: 0 empty (transparent), 1 other nonempty, 2 kNow
    int kind[kPer], lastk = 0;
#pragma unroll
    for (int c = 0; c < kPer; c++) {
        const int b = kPer * t + c;
        const uint32_t cb = bn.cnt[b];
        const bool ne = bn.off[b + 1] > bn.off[b];
        kind[c] = !ne ? 0 : ((cb & kNow) ? 2 : 1);
        if (cb & kNow)
            for (uint32_t j = cb & ~kNow; j < bn.off[b + 1]; j++) stg(gl + j, (uint64_t)0);
        if (kind[c]) lastk = kind[c];
        bn.nzc[b] = 0u;
    }
    int prevk = block_excl_last(lastk, 1, sm);
    uint32_t nst = 0;
    int starts[kPer];
#pragma unroll
    for (int c = 0; c < kPer; c++) {
        starts[c] = (kind[c] == 2 && prevk != 2) ? 1 : 0;
        if (kind[c]) prevk = kind[c];
        nst += starts[c];
    }
    uint32_t nruns;
    uint32_t r = block_excl_u32(nst, &nruns, sm);
    if (nruns > (uint32_t)kMaxGroups) return false;
    for (int g = t; g < kMaxGroups; g += kThreads) { bn.gbeg[g] = 0xffffffffu; bn.gend[g] = 0u; bn.run[g] = 0ull; }
    __syncthreads();
    r -= 1;                                   // run index of the current kNow bin
#pragma unroll
    for (int c = 0; c < kPer; c++) {
        const int b = kPer * t + c;
        r += starts[c];
        if (kind[c] == 2) {
            atomicMin(&bn.gbeg[r], bn.off[b]);
            atomicMax(&bn.gend[r], bn.off[b + 1]);
        }
        if (starts[c]) bn.runt[r] = (uint32_t)b;      // the run's first bin
    }
    __threadfence_block();
    __syncthreads();
    // items per run and their prefix (wbase[r] = first item of run r)
    const uint32_t nit = (t < (int)nruns) ? (bn.gend[t] - bn.gbeg[t] + 63u) >> 6 : 0u;
    if (t < (int)nruns && bn.gend[t] - bn.gbeg[t] > kMaxRun) bn.fail = 1;
    uint32_t tot;
    const uint32_t ib = block_excl_u32(nit, &tot, sm);
    if (t < (int)nruns) bn.wbase[t] = ib;
    __syncthreads();
    if (bn.fail || tot * 64u > kWalkCap) return false;
    auto item_run = [&](uint32_t it) {
        int lo = 0, hi = (int)nruns - 1;            // largest r with wbase[r] <= it
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (bn.wbase[mid] <= it) lo = mid;
            else hi = mid - 1;
        }
        return lo;
    };
    auto bin_of_entry = [&](uint64_t en) { return bin_clamp(key2f((uint32_t)(en >> 32)) - m0); };
    // nonzero entries per bin
    for (uint32_t it = wave_id(); it < tot; it += kWaves) {
        const int rr = item_run(it);
        const uint32_t o = bn.gbeg[rr], n = bn.gend[rr] - o;
        const uint32_t j = 64u * (it - bn.wbase[rr]) + lane;
        const uint64_t en = j < n ? ldg(gl + o + j) : 0ull;
        if (en) atomicAdd(&bn.nzc[bin_of_entry(en)], 1u);
    }
    __syncthreads();
    // exclusive prefix of the nonzero counts in bin order
    {
        uint32_t v[kPer], loc = 0;
#pragma unroll
        for (int c = 0; c < kPer; c++) { v[c] = bn.nzc[kPer * t + c]; loc += v[c]; }
        uint32_t all;
        uint32_t ex = block_excl_u32(loc, &all, sm);
#pragma unroll
        for (int c = 0; c < kPer; c++) { bn.nzc[kPer * t + c] = ex; ex += v[c]; }
    }
    __syncthreads();
    // run r: nonzero prefix at its first bin (runt[r])
    if (t < (int)nruns) {
        // (not from the run's first entry: that slot may hold a zero, such as
        // a penalized id's raw value taken out of the list)
        bn.runt[t] = bn.nzc[bn.runt[t]];
    }
    __syncthreads();
    for (uint32_t it = wave_id(); it < tot; it += kWaves) {
        const int rr = item_run(it);
        const uint32_t o = bn.gbeg[rr], n = bn.gend[rr] - o, base = bn.wbase[rr];
        const uint32_t j = 64u * (it - base) + lane;
        if (j >= n) continue;
        const uint64_t mine = ldg(gl + o + j);
        uint32_t pos;
        if (mine) {
            const int b = bin_of_entry(mine);
            const uint32_t bo = bn.off[b], bc = bn.cnt[b] & ~kNow;
            uint32_t rank = 0;
            uint32_t i = bo;
            for (; i + 4 <= bc; i += 4) {
                const uint64_t a0 = ldg(gl + i), a1 = ldg(gl + i + 1), a2 = ldg(gl + i + 2), a3 = ldg(gl + i + 3);
                rank += (a0 > mine) + (a1 > mine) + (a2 > mine) + (a3 > mine);
            }
            for (; i < bc; i++) rank += ldg(gl + i) > mine;
            pos = bn.nzc[b] - bn.runt[rr] + rank;
        } else {
            // zeros after the run's nonzero entries; the run's nonzero total is
            // its size minus its zeros, which the zero counter reaches last
            pos = 0xffffffffu;
            const uint32_t zi = (uint32_t)atomicAdd((unsigned long long *)&bn.run[rr], 1ull);
            pos = n - 1u - zi;
        }
        stg(tmp + 64u * base + pos, mine);
    }
    __threadfence_block();
    __syncthreads();
    for (uint32_t it = wave_id(); it < tot; it += kWaves) {
        const int rr = item_run(it);
        const uint32_t o = bn.gbeg[rr], n = bn.gend[rr] - o, base = bn.wbase[rr];
        const uint32_t j = 64u * (it - base) + lane;
        if (j < n) stg(gl + o + j, ldg(tmp + 64u * base + j));
    }
    __threadfence_block();
    __syncthreads();
    for (int b = t; b < kBins; b += kThreads)
        if (bn.cnt[b] & kNow) { bn.cnt[b] = bn.off[b + 1]; bn.meta[b] &= ~kMetaNow; }
    __syncthreads();
    return true;
}

// ---------------------------------------------------------------------------
// The binned path.  Returns true with *tok / *status set, or false to ask for
// the sort-based path.  Needs a 16-byte aligned row and `gl`, a per-row list
// of lcap u64 entries in global memory.
__device__ bool full_bins_row(RowSmem &sm, const float *row, int V, float T, float top_p,
                              bool has_pen, float r, uint64_t *gl, uint32_t lcap, int *tok,
                              int *status)
{
    // deferred ids and the walk arrays live after the list
    const uint32_t lneed = (uint32_t)V + (uint32_t)(kOverCap + 2 * kHashSlots);
    if (lcap < lneed + kDeferCapG / 2 + kWalkCap) BINS_FAIL();
    uint32_t *defer = reinterpret_cast<uint32_t *>(gl + lneed);
    const uint32_t dcap = kDeferCapG;
    float *W = reinterpret_cast<float *>(gl + lneed + kDeferCapG / 2);
    uint32_t *WT = reinterpret_cast<uint32_t *>(W + kWalkCap);
    uint64_t *tmp = reinterpret_cast<uint64_t *>(W);       // segment sort staging (W is dead then)
    // element indices by bin (same positions as the list), recorded in pass 3
    // for bins up to the cut when the row has no penalty and a nucleus cut;
    // later stages read the elements of a few bins from them instead of
    // passing over the row again
    uint32_t *ix = reinterpret_cast<uint32_t *>(gl + lneed + kDeferCapG / 2 + kWalkCap);
    if (lcap < lneed + kDeferCapG / 2 + kWalkCap + (lneed + 1) / 2) BINS_FAIL();
    const bool use_ix = (top_p < 1.0f) && !has_pen;
    BinsSmem &bn = sm.x.bn;
    const int t = threadIdx.x;
    const bool t_one = (T == 1.0f);
    const bool nucleus = top_p < 1.0f;
    // Rows with a nucleus cut, no penalty and a draw predicted beyond a fifth
    // of the row compute the seq-3 increments in pass 3 (no pass 4, which
    // would otherwise pass over the row); their per-bin sums use the penalty
    // hash's LDS (4096 words), which such rows leave unused.  Set in plan B.
    bool merge3 = false;
    static_assert(2 * kHashSlots == kBins && offsetof(RowSmem, hval) == offsetof(RowSmem, hkey) + 4 * kHashSlots,
                  "hkey and hval form one array of kBins words");
    uint32_t *acc3 = nullptr;
    const float4 *r4 = reinterpret_cast<const float4 *>(row);
    const int n4 = V >> 2;
    if (n4 == 0) BINS_FAIL();

    uint64_t *mass64 = reinterpret_cast<uint64_t *>(bn.esum);   // aliases esum + k2 until plan A
    for (int b = t; b < kBins; b += kThreads) { bn.cnt[b] = 0; mass64[b] = 0ull; }
    if (t == 0) { bn.nover = 0; bn.ndefer = 0; bn.fail = 0; bn.ncollect = 0; bn.nties = 0; }

    // ---- pass 1 (HBM): counts, max, NaN -------------------------------------
    float tmax = -INFINITY;
    int nan = 0;
    float m0 = 0.0f;
    auto visit = [&](int i, float y) {
        nan |= (int)isnan(y);
        if (y > tmax && !(has_pen && hash_find(sm, (uint32_t)i) >= 0)) tmax = y;
        const float dp = y - m0;
        if (dp > kDUp) {
            const int slot = atomicAdd(&bn.nover, 1);
            if (slot < kOverCap) bn.over[slot] = list_entry(y, (uint32_t)i);
        } else if (dp >= -kDLo) {
            const int b = bin_of(dp);
            atomicAdd(&bn.cnt[b], 1u);
            if (b < kMassBins) atomicAdd((unsigned long long *)&mass64[b], (unsigned long long)(fast_exp(dp) * kMassScale));
        }
    };
    for (int base = 0; base < n4; base += kThreads * kUnroll) {
        float4 v[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; u++)
            v[u] = ldg(r4 + min(base + u * kThreads + t, n4 - 1));   // unconditional: no wait between loads
        if (base == 0) {
            float lm = -INFINITY;
#pragma unroll
            for (int u = 0; u < kUnroll; u++) {
                const int q = u * kThreads + t;
                if (q < n4) lm = fmaxf(lm, fmaxf(fmaxf(v[u].x, v[u].y), fmaxf(v[u].z, v[u].w)));
            }
            const float bm = block_max_f(lm, sm);
            m0 = t_one ? bm : bm / T;
            if (!isfinite(m0)) BINS_FAIL();
        }
        if (t_one) {
#pragma unroll
            for (int u = 0; u < kUnroll; u++) {
                const int q = base + u * kThreads + t;
                if (q < n4) {
                    visit(4 * q + 0, v[u].x);
                    visit(4 * q + 1, v[u].y);
                    visit(4 * q + 2, v[u].z);
                    visit(4 * q + 3, v[u].w);
                }
            }
        } else {
#pragma unroll
            for (int u = 0; u < kUnroll; u++) {
                const int q = base + u * kThreads + t;
                if (q < n4) {
                    visit(4 * q + 0, v[u].x / T);
                    visit(4 * q + 1, v[u].y / T);
                    visit(4 * q + 2, v[u].z / T);
                    visit(4 * q + 3, v[u].w / T);
                }
            }
        }
    }
    for (int i = (n4 << 2) + t; i < V; i += kThreads) visit(i, t_one ? row[i] : row[i] / T);
    if (has_pen) {
        for (int s = t; s < kHashSlots; s += kThreads) {
            if (sm.hkey[s] == kEmpty) continue;
            const float y = t_one ? __uint_as_float(sm.hval[s]) : __uint_as_float(sm.hval[s]) / T;
            nan |= (int)isnan(y);
            tmax = fmaxf(tmax, y);
        }
    }
    if (block_or(nan, sm) || sm.flag_nan) { *status = GS_ERR_NAN; *tok = 0; return true; }
    const float m = block_max_f(tmax, sm);
    if (t == 0) { bn.m = m; bn.m0 = m0; }
    *status = GS_OK;
    // Infinite max: some y - max is NaN and so is every probability; that
    // rare case (the reference returns its last candidate) takes the sort path.
    if (!isfinite(m)) BINS_FAIL();
    // bins must cover [m - 18.5, m]; a first-round max above m (penalized) breaks that
    if (bn.nover > kOverCap || m0 > m) BINS_FAIL();
    GS_STAMP(9);

    // ---- penalty: penalized values join the counts and the overflow --------
    if (has_pen) {
        for (int j = t; j < bn.nover; j += kThreads)
            if (hash_find(sm, ~(uint32_t)bn.over[j]) >= 0) bn.over[j] = 0ull;
        __syncthreads();
        for (int s = t; s < kHashSlots; s += kThreads) {
            const uint32_t id = sm.hkey[s];
            if (id == kEmpty) continue;
            // the raw value leaves the plan's mass: its exact mass (added in
            // pass 1) from a mass bin; from a bulk bin, one element of the
            // count the mass is estimated from (mass64 of bulk bins counts
            // them).  Counts stay: segment sizes are upper bounds.
            {
                const float xr = ldg(row + id);
                const float dr = (t_one ? xr : xr / T) - m0;
                if (dr <= kDUp && dr >= -kDLo) {
                    const int b = bin_of(dr);
                    if (b < kMassBins) atomicAdd((unsigned long long *)&mass64[b], 0ull - (unsigned long long)(fast_exp(dr) * kMassScale));
                    else atomicAdd((unsigned long long *)&mass64[b], 1ull);
                }
            }
            const float yp = t_one ? __uint_as_float(sm.hval[s]) : __uint_as_float(sm.hval[s]) / T;
            const float dq = yp - m0;
            if (dq > kDUp) {
                const int slot = atomicAdd(&bn.nover, 1);
                if (slot < kOverCap) bn.over[slot] = list_entry(yp, id);
            } else if (dq >= -kDLo) {
                // raw counts stay (segment sizes are upper bounds); masses are a plan only
                const int b = bin_of(dq);
                atomicAdd(&bn.cnt[b], 1u);
                if (b < kMassBins) atomicAdd((unsigned long long *)&mass64[b], (unsigned long long)(fast_exp(dq) * kMassScale));
            }
        }
        __syncthreads();
        if (bn.nover > kOverCap) BINS_FAIL();
    }
    const int nover = bn.nover;

    // ---- plan A: accumulation 1 ----------------------------------------------
    // The running sum before bin b is predicted from counts times the bin's
    // central value; its binade gives the bin's grid.  Collected: the bin that
    // opens the sum, bins where it may change binade, bins with likely
    // rounding ties, and bins whose increment sum might not fit 32 bits.
    constexpr int kPer = kBins / kThreads;
    static_assert(kPer * kThreads == kBins, "bins per thread");
    const float wbin = (kDUp + kDLo) / (float)kBins;
    const float shift = m0 - m;            // e = exp(d' + shift)
    auto e_at = [&](float bpos) { return (double)fast_exp(kDUp - bpos * wbin + shift); };
    const double dl = 1.0 - kDelta, dh = 1.0 + kDelta;
    {
        double osum = 0.0;
        for (int j = t; j < nover; j += kThreads) {
            const uint64_t en = bn.over[j];
            if (en) osum += (double)fast_exp(key2f((uint32_t)(en >> 32)) - m);
        }
        osum = block_sum_f64(osum, sm);
        uint32_t cntv[kPer];
        double eb[kPer];
        double loc = 0.0;
        uint32_t ctot = 0;
        const double mscale = (double)fast_exp(shift) / (double)kMassScale;   // mass rel. m0 -> rel. m
#pragma unroll
        for (int c = 0; c < kPer; c++) {
            const int b = kPer * t + c;
            cntv[c] = bn.cnt[b];
            eb[c] = b < kMassBins ? (double)mass64[b] * mscale
                                  : (double)(cntv[c] - (uint32_t)mass64[b]) * e_at((float)b + 0.5f);
            loc += eb[c];
            ctot += cntv[c];
        }
        double stot;
        const double pre = block_excl_f64(loc, &stot, sm) + osum;
        uint32_t call;
        const uint32_t cpre = block_excl_u32(ctot, &call, sm);
        if ((uint32_t)nover + call > lneed) BINS_FAIL();
        if (t == 0) bn.off[kBins] = (uint32_t)nover + call;
        uint32_t o = (uint32_t)nover + cpre;
        double lo = pre;
#pragma unroll
        for (int c = 0; c < kPer; c++) {
            const int b = kPer * t + c;
            const double hi = lo + eb[c];
            const double ehi = e_at((float)b) * 1.001;
            const double cn = (double)cntv[c];
            bool col = !(lo > 0.0);
            int b1 = 0;
            if (cntv[c] && !col) {
                b1 = grid_exp((float)lo);
                const bool cx = grid_exp((float)(lo * dl)) != grid_exp((float)(hi * dh));
                col |= cx;
                const int c1 = ilogb(ehi);
                const bool ct = (c1 < b1) && cn * ldexp(1.0, c1 - b1) > kTieThr;
                col |= ct;
                const bool co = cn * (ldexp(ehi, 23 - b1) + 1.0) >= 4.0e9;
                col |= co;
#ifdef GS_TIMING
                if (blockIdx.x == g_row) { if (cx) atomicAdd(&g_fails[1010], (int)cntv[c]); if (ct) atomicAdd(&g_fails[1011], (int)cntv[c]); if (co) atomicAdd(&g_fails[1012], (int)cntv[c]); g_fails[1013] = __float_as_int((float)lo); }
#endif
            }
            if (cntv[c] == 0) col = false;
            bn.meta[b] = (col ? kMetaCol | kMetaNow : 0u) | (cntv[c] ? 8u : 0u) | ((uint32_t)(b1 + 128) << 8) |
                         (128u << 16) | (128u << 24);
            bn.off[b] = o;
            bn.cnt[b] = col ? o | kNow : o;  // list cursor of collected bins
            bn.esum[b] = 0u;
            bn.k2[b] = 0u;                  // collected masses accumulate here (f32)
            o += cntv[c];
            lo = hi;
        }
    }
    for (int j = t; j < nover; j += kThreads) stg(gl + j, bn.over[j]);
    __syncthreads();
    GS_STAMP(10);

    // ---- pass 2 (cache): accumulation-1 increments, collected bins listed ----
    PassK K;
    K.m0 = m0;
    K.m = m;
    K.inv_s = 1.0f;
    K.inv_s2 = 1.0f;
    K.hw2 = 0.0f;
    K.ixlim = -1;
    bins_pass(sm, row, V, t_one, T, has_pen, gl, defer, dcap, bn.esum, nullptr,
              [&bn, K](float y) { return classify1(bn, K, y); });
    GS_STAMP(11);
    if ((uint32_t)bn.ndefer > dcap) BINS_FAIL();
    if (!finish_now(sm, gl, tmp)) BINS_FAIL();
    if (wave_id() == 0 && !wave_sort_segment(gl, nover)) bn.fail = 1;
    __threadfence_block();
    __syncthreads();
    if (bn.fail) BINS_FAIL();
    GS_STAMP(12);

    // ---- exact accumulation-1 increments of the deferred elements ------------
    auto def_y = [&](uint32_t en) {
        const uint32_t id = en & kIdMask;
        float x = ldg(row + id);
        if (en & 0x80000000u) {
            const int s = hash_find(sm, id);
            if (s >= 0) x = __uint_as_float(sm.hval[s]);
        }
        return t_one ? x : x / T;
    };
    {
        const int nd = bn.ndefer;
        for (int j = t; j < nd; j += kThreads) {
            const uint32_t en = ldg(defer + j);
            if (en == 0xffffffffu) continue;
            const float y = def_y(en);
            const int b = bin_of(y - m0);
            uint32_t k;
            const int rc = inc_exact(glibc_expf(y - m), meta_b(bn.meta[b], 1), &k);
            if (rc < 0) { bn.fail = 1; continue; }
            if (k) atomicAdd(&bn.esum[b], k);
            if (rc == 0) {                  // tie: the lower choice is added, the tie counted
                const uint32_t old = atomicAdd(&bn.meta[b], 16u);
                if (((old >> 4) & 7u) == 7u) bn.fail = 1;
                atomicAdd(&bn.nties, 1);
            }
        }
    }
    __syncthreads();
    if (bn.fail) BINS_FAIL();

    // ---- S, bracketed by the ties rounded down / up --------------------------
    if (!build_groups(sm)) BINS_FAIL();
    gather_runs(sm, 1);
    int N = build_walk(sm, gl, W, WT, m, m0, true);
    if (N < 0) BINS_FAIL();
    GS_STAMP(13);
    GS_DIAG(26, N);
    GS_DIAG(28, bn.ndefer);
    GS_DIAG(30, bn.nties);
    // ties rounded down (wave 0) and, if there are ties, rounded up (wave 1),
    // concurrently
    float Slo, Shi;
    const bool s_exact = bn.nties == 0;
    {
        make_walk_tab(sm, 1);
        const int w = wave_id();
        if (w == 0 || (w == 1 && !s_exact)) {
            float sv;
            const int rr = wave_walk(W, N, walk_tab(bn, w == 1), [](float) { return false; }, &sv);
            if (lane_id() == 0) {
                if (w == 0) { sm.seq.first = rr; sm.seq.s = sv; }
                else { sm.seq.start = rr; bn.Shi = sv; }
            }
        }
        __syncthreads();
#ifdef GS_TIMING
        if (t == 0 && (sm.seq.first != N || (!s_exact && sm.seq.start != N))) { g_fails[1000] = blockIdx.x; g_fails[1001] = sm.seq.first; g_fails[1002] = sm.seq.start; g_fails[1003] = N; g_fails[1004] = bn.nties; }
#endif
        if (sm.seq.first != N || (!s_exact && sm.seq.start != N)) BINS_FAIL();
        Slo = sm.seq.s;
        Shi = s_exact ? Slo : bn.Shi;
        __syncthreads();
    }
    if (!(Slo > 0.0f) || !(Shi >= Slo) || !isfinite(Shi)) BINS_FAIL();
    GS_STAMP(14);

    // ---- plan B: accumulations 2 and 3 ---------------------------------------
    // Masses: bulk bins from their exact seq-1 increments, collected bins and
    // the overflow from their exact summands.  With S bracketed, the seq-2
    // running sum before each bin is known to the rounding of the increments:
    // bulk bins before the cut get seq-2 increments in pass 3; bins where it
    // may change binade or reach top_p are collected.
    double osum = 0.0;
    for (int j = t; j < nover; j += kThreads) {
        const uint64_t en = ldg(gl + j);
        if (en) osum += (double)glibc_expf(key2f((uint32_t)(en >> 32)) - m);
    }
    osum = block_sum_f64(osum, sm);          // contains barriers
    const double Sc = 0.5 * ((double)Slo + (double)Shi);
    const double iSc = 1.0 / Sc;
    {
        uint32_t mtv[kPer];
        double mass[kPer];
        double loc = 0.0;
#pragma unroll
        for (int c = 0; c < kPer; c++) {
            const int b = kPer * t + c;
            mtv[c] = bn.meta[b];
            if (mtv[c] & 1u) mass[c] = (double)__uint_as_float(bn.k2[b]);
            else mass[c] = ldexp((double)bn.esum[b] + 0.5 * (double)((mtv[c] >> 4) & 7u), meta_b(mtv[c], 1) - 23);
            if (!(mtv[c] & 8u)) mass[c] = 0.0;
            loc += mass[c];
        }
        double stot;
        const double pre = block_excl_f64(loc, &stot, sm) + osum;
        stot += osum;
        double s2lo = 1.0, s2hi = 1.0;
        if (t == 0) { bn.cut_g = kBins; bn.ixlim = -1; bn.ixlast = -1; }
        __syncthreads();
        if (nucleus) {
            if (stot / Sc < (double)top_p * (1.0 + 2.0 * kDelta)) BINS_FAIL();   // the cut may not happen
            double lo = pre;
#pragma unroll
            for (int c = 0; c < kPer; c++) {
                const double hi = lo + mass[c];
                if (mass[c] > 0.0 && hi * iSc * dh >= (double)top_p) { atomicMin(&bn.cut_g, kPer * t + c); break; }
                lo = hi;
            }
            __syncthreads();
            const int cb = bn.cut_g;
            if (cb >= kBins) BINS_FAIL();
            // the cut element lies in bin cb, or anywhere from the max (e = 1)
            // on if the overflow segment may already reach top_p
            const double ehc = (osum / Sc * dh >= (double)top_p) ? 1.0 : e_at((float)cb) * 1.001;
            s2lo = (double)top_p;
            s2hi = (double)top_p + ehc / Sc * (1.0 + 4.0 * kDelta) + 0x1p-24;
        }
        if (t == 0) {
            bn.Slo = Slo;
            bn.Shi = Shi;
            bn.inv_s = (float)(1.0 / Sc);
            bn.hw2 = 2.0f * kExpErr + (float)(((double)Shi - (double)Slo) / (double)Slo) + 0x1p-22f;
            bn.s2lo = (float)s2lo;
            bn.s2hi = (float)s2hi;
            bn.inv_s2c = (float)(2.0 / (s2lo + s2hi));
            bn.hw3 = bn.hw2 + (float)((s2hi - s2lo) / s2lo) + 0x1p-22f;
        }
        const double s2c = 0.5 * (s2lo + s2hi);
        // The bins that may precede the draw (seq 3): indexed in pass 3 when
        // they hold at most a fifth of the row, else the merged pass 3.
        if (nucleus) {
            double lo = pre;
#pragma unroll
            for (int c = 0; c < kPer; c++) {
                const double hi = lo + mass[c];
                const uint32_t mt = mtv[c];
                const double plo_ = lo * iSc;
                if ((mt & 8u) && !(mt & 1u) && plo_ * dl < (double)top_p && plo_ / s2c * dl <= (double)r)
                    atomicMax(&bn.ixlim, kPer * t + c);
                lo = hi;
            }
        }
        __syncthreads();
        merge3 = nucleus && !has_pen && bn.ixlim >= 0 && bn.off[bn.ixlim + 1] - bn.off[0] > (uint32_t)V / 5u;
        if (merge3) acc3 = reinterpret_cast<uint32_t *>(sm.hkey);
        double lo = pre;
#pragma unroll
        for (int c = 0; c < kPer; c++) {
            const int b = kPer * t + c;
            const double hi = lo + mass[c];
            const uint32_t mt = mtv[c];
            if ((mt & 8u) && !(mt & 1u)) {
                const double cn = (double)(bn.off[b + 1] - bn.off[b]);
                bool col = ((mt >> 4) & 7u) != 0u;            // seq-1 ties need the order for S
                const double ehi = e_at((float)b) * 1.001;
                const double plo_ = lo * iSc, phi_ = hi * iSc, pe = ehi * iSc;
                bool k2 = false, k3 = false;
                int b2 = 0, b3 = 0;
                if (nucleus) {
                    k2 = plo_ * dl < (double)top_p;
                    if (k2) {
                        b2 = grid_exp((float)plo_);
                        col |= !(plo_ > 0.0);
                        col |= grid_exp((float)(plo_ * dl)) != grid_exp((float)(phi_ * dh));
                        col |= phi_ * dh >= (double)top_p;
                        const int c2 = ilogb(pe);
                        if (c2 < b2) col |= cn * ldexp(1.0, c2 - b2) > kTieThr;
                        col |= cn * (ldexp(pe, 23 - b2) + 1.0) >= 4.0e9;
                        // merged pass 3: the seq-3 decisions of plan C, with S
                        // and s2 known to their ranges (far inside the margin)
                        const double qlo = plo_ / s2c, qhi = phi_ / s2c;
                        if (merge3 && qlo * dl <= (double)r) {
                            k3 = true;
                            b3 = grid_exp((float)qlo);
                            col |= !(qlo > 0.0);
                            col |= grid_exp((float)(qlo * dl)) != grid_exp((float)(qhi * dh));
                            col |= qhi * dh > (double)r;
                            const double qe = pe / s2c;
                            const int c3 = ilogb(qe);
                            if (c3 < b3) col |= cn * ldexp(1.0, c3 - b3) > kTieThr;
                            col |= cn * (ldexp(qe, 23 - b3) + 1.0) >= 4.0e9;
                            atomicMax(&bn.ixlast, b);
                        }
                    }
                }
                bn.meta[b] = (mt & 0xff00u) | (mt & 0x78u) | (col ? 0x81u : 0u) | (k2 ? 2u : 0u) |
                             (k3 ? 4u : 0u) | ((uint32_t)(b2 + 128) << 16) | ((uint32_t)(b3 + 128) << 24);
                if (col) {
                    bn.cnt[b] = bn.off[b] | kNow;
                    atomicAdd(&bn.ncollect, 1);
                }
            }
            bn.k2[b] = 0u;
            if (merge3) acc3[b] = 0u;
            bn.icur[b] = bn.off[b];
            bn.pre_e[b] = (float)lo;
            lo = hi;
        }
        if (t == kThreads - 1) bn.pre_e[kBins] = (float)lo;
    }
    __syncthreads();
    if (t == 0) {
        bn.ndefer = 0;
        // a large region is cheaper as passes over the row than as gathers
        if (bn.ixlim >= 0 && bn.off[bn.ixlim + 1] - bn.off[0] > (uint32_t)V / 5u) bn.ixlim = -1;
    }
    __syncthreads();
    GS_STAMP(16);

    // ---- pass 3 (cache): accumulation-2 increments, new bins listed ----------
    K.inv_s = bn.inv_s;
    K.hw2 = bn.hw2;
    K.ixlim = use_ix ? bn.ixlim : -1;
    K.inv_s2c = bn.inv_s2c;
    K.hw3 = bn.hw3;
    if (merge3)
        bins_pass(sm, row, V, t_one, T, has_pen, gl, defer, dcap, bn.k2, ix,
                  [&bn, K](float y) { return classify3m(bn, K, y); }, acc3);
    else
        bins_pass(sm, row, V, t_one, T, has_pen, gl, defer, dcap, bn.k2, ix,
                  [&bn, K](float y) { return classify3(bn, K, y); });
    GS_STAMP(17);
    GS_DIAG(29, bn.ndefer | ((uint64_t)bn.ncollect << 32));
    if ((uint32_t)bn.ndefer > dcap) BINS_FAIL();
    if (!finish_now(sm, gl, tmp)) BINS_FAIL();

    // ---- deferred accumulation-2 elements over the reachable S ---------------
    // A possible tie needs the exact order (the bin is collected in pass 4); a
    // unique increment is added now; otherwise it waits for the exact S.
    auto mark = [&](int b) {
        const uint32_t old = atomicOr(&bn.meta[b], kMetaCol | kMetaNow);
        if (!(old & 1u)) { bn.cnt[b] = bn.off[b] | kNow; atomicAdd(&bn.ncollect, 0x10000); }
    };
    const int nd = bn.ndefer;
    for (int j = t; j < nd; j += kThreads) {
        const uint32_t en = ldg(defer + j);
        if (en == 0xffffffffu || (en & kDone2)) continue;
        const float y = def_y(en);
        const int b = bin_of(y - m0);
        const uint32_t mt = bn.meta[b];
        if (mt & 1u) continue;
        uint32_t k;
        const int rc = inc_s_range(glibc_expf(y - m), Slo, Shi, meta_b(mt, 2), &k);
        if (rc == 2) { mark(b); continue; }
        if (rc == 0) {
            if (k) atomicAdd(&bn.k2[b], k);
            defer[j] = en | kDone2;
        }
    }
    __syncthreads();
    GS_STAMP(18);

    // ---- pass 4 (cache, rare): collect the bins of possible ties -------------
#ifdef GS_TIMING
    if (t == 0 && blockIdx.x < 256) g_fails[512 + blockIdx.x] = ((bn.ncollect >> 16) ? 1 : 0) | (s_exact ? 0 : 4);
#endif
    if (bn.ncollect >> 16) {
        if (!use_ix || !collect_now_ix(sm, row, t_one, T, gl, ix)) {
#ifdef GS_TIMING
            if (t == 0 && blockIdx.x < 256) g_fails[512 + blockIdx.x] |= 16;
#endif
            collect_now(sm, row, V, t_one, T, has_pen, gl);
        }
        if (!finish_now(sm, gl, tmp)) BINS_FAIL();
    }
    // runs carry the accumulation-2 grids now: always regroup; the walk array
    // changes only if bins were collected
    if (!build_groups(sm)) BINS_FAIL();
    if (bn.ncollect) {
        N = build_walk(sm, gl, W, WT, m, m0, false);
        if (N < 0) BINS_FAIL();
    }
    GS_STAMP(19);
    GS_DIAG(27, N | ((uint64_t)bn.ncollect << 32));

    // ---- exact walks ----------------------------------------------------------
    float S = Slo;
    if (!s_exact) {
        gather_runs(sm, 1);
        if (walk(sm, W, N, 1, [](float) { return false; }, &S) != N) BINS_FAIL();
        if (!(S >= Slo && S <= Shi)) BINS_FAIL();
    }
    GS_STAMP(20);
    // late seq-2 increments, now that S is exact (no reachable value was a tie)
    for (int j = t; j < nd; j += kThreads) {
        const uint32_t en = ldg(defer + j);
        if (en == 0xffffffffu || (en & kDone2)) continue;
        const float y = def_y(en);
        const int b = bin_of(y - m0);
        const uint32_t mt = bn.meta[b];
        if (mt & 1u) continue;
        uint32_t k;
        if (inc_exact(glibc_expf(y - m) / S, meta_b(mt, 2), &k) != 1) { bn.fail = 1; continue; }
        if (k) atomicAdd(&bn.k2[b], k);
    }
    // summands of seq 2: p = e / S (src/sampler.rs:56)
    for (int j = t; j < N; j += kThreads) { const float v = W[j]; if (!is_marker(v)) W[j] = v / S; }
    __threadfence_block();
    __syncthreads();
    if (bn.fail) BINS_FAIL();
    int js = -1;
    float s2 = 1.0f;
    uint32_t cut_tok = 0;
    if (nucleus) {
        gather_runs(sm, 2);
        js = walk(sm, W, N, 2, [top_p](float c) { return c >= top_p; }, &s2);
        if (js < 0 || js >= N || !(s2 >= bn.s2lo && s2 <= bn.s2hi)) BINS_FAIL();
        cut_tok = WT[js];
    }
    GS_STAMP(21);

    if (!merge3) {
    // ---- plan C: accumulation 3, with S and s2 exact -------------------------
    // q = p / s2 (src/sampler.rs:68); the seq-3 running sum before bin b is
    // the bin's mass prefix / (S s2) to the rounding of the increments.  Bulk
    // bins before the draw get seq-3 increments in pass 4 (in esum, free now);
    // bins where it may change binade or pass r are collected.
    {
        const double inv_ss = 1.0 / ((double)S * (double)s2);
#pragma unroll
        for (int c = 0; c < kPer; c++) {
            const int b = kPer * t + c;
            const uint32_t mt = bn.meta[b];
            bn.esum[b] = 0u;
            if (!(mt & 8u) || (mt & 1u) || (nucleus && !(mt & 2u))) continue;
            const double qlo = (double)bn.pre_e[b] * inv_ss, qhi = (double)bn.pre_e[b + 1] * inv_ss;
            if (!(qlo * dl <= (double)r)) continue;
            const double cn = (double)(bn.off[b + 1] - bn.off[b]);
            const double qe = e_at((float)b) * 1.001 * inv_ss;
            const int b3 = grid_exp((float)qlo);
            bool col = !(qlo > 0.0);
            col |= grid_exp((float)(qlo * dl)) != grid_exp((float)(qhi * dh));
            col |= qhi * dh > (double)r;
            const int c3 = ilogb(qe);
            if (c3 < b3) col |= cn * ldexp(1.0, c3 - b3) > kTieThr;
            col |= cn * (ldexp(qe, 23 - b3) + 1.0) >= 4.0e9;
            bn.meta[b] = (mt & 0x00ffffffu) | 4u | (col ? kMetaCol | kMetaNow : 0u) | ((uint32_t)(b3 + 128) << 24);
            if (col) bn.cnt[b] = bn.off[b] | kNow;
            atomicMax(&bn.ixlast, b);
        }
        if (t == 0) {
            bn.ndefer = 0;
            bn.ncollect = 0;
            bn.inv_s = 1.0f / S;
            bn.inv_s2 = 1.0f / s2;
        }
        __syncthreads();
    }

    // ---- pass 4 (cache): accumulation-3 increments, new bins listed ----------
    K.inv_s = bn.inv_s;
    K.inv_s2 = bn.inv_s2;
    K.ixlim = -1;
    {
        // with indexed bins, only the elements of bins up to the last seq-3
        // bin are visited, through their indices; otherwise a pass over the row
        // gathers win only for small regions: about one fifth of the row
        // costs as much as a streaming pass
        bool gather = use_ix && bn.ixlast <= bn.ixlim &&
                      (bn.ixlast < 0 || bn.off[bn.ixlast + 1] - bn.off[0] <= (uint32_t)V / 5u);
        if (gather) {
            bool bad = false;
            for (int b = t; b <= bn.ixlim; b += kThreads) bad |= bn.icur[b] != bn.off[b + 1];
            gather = !block_or((int)bad, sm);
        }
        if (gather) {
#ifdef GS_TIMING
            if (t == 0 && blockIdx.x < 256) g_fails[512 + blockIdx.x] |= 8;
#endif
            const uint32_t p0 = bn.off[0], p1 = bn.ixlast >= 0 ? bn.off[bn.ixlast + 1] : p0;
            auto act = [&](uint32_t i, float y, const Cls &c) {
                if (c.cl == 1) {
                    const uint32_t slot = atomicAdd(&bn.cnt[c.b], 1u) & ~kNow;
                    stg(gl + slot, list_entry(y, i));
                } else if (c.cl == 2) {
                    const int slot = atomicAdd(&bn.ndefer, 1);
                    if ((uint32_t)slot < dcap) stg(defer + slot, i);
                } else if (c.cl == 3 && c.k) {
                    atomicAdd(&bn.esum[c.b], c.k);
                }
            };
            constexpr int kG = 8;
            for (uint32_t p = p0 + t; p < p1; p += kThreads * kG) {
                uint32_t id[kG];
                float x[kG];
#pragma unroll
                for (int g = 0; g < kG; g++) id[g] = ldg(ix + min(p + (uint32_t)(g * kThreads), p1 - 1));
#pragma unroll
                for (int g = 0; g < kG; g++) x[g] = ldg(row + id[g]);
#pragma unroll
                for (int g = 0; g < kG; g++) {
                    if (p + (uint32_t)(g * kThreads) < p1) {
                        const float y = t_one ? x[g] : x[g] / T;
                        act(id[g], y, classify4(bn, K, y));
                    }
                }
            }
            __syncthreads();
        } else {
            bins_pass(sm, row, V, t_one, T, has_pen, gl, defer, dcap, bn.esum, ix,
                      [&bn, K](float y) { return classify4(bn, K, y); });
        }
    }
    GS_STAMP(22);
    if ((uint32_t)bn.ndefer > dcap) BINS_FAIL();
    if (!finish_now(sm, gl, tmp)) BINS_FAIL();
    // deferred seq-3 elements: exact increments; a tie needs the bin's order
    {
        const int nd4 = bn.ndefer;
        for (int j = t; j < nd4; j += kThreads) {
            const uint32_t en = ldg(defer + j);
            if (en == 0xffffffffu) continue;
            const float y = def_y(en);
            const int b = bin_of(y - m0);
            const uint32_t mt = bn.meta[b];
            if (mt & 1u) continue;
            const float p = glibc_expf(y - m) / S;
            uint32_t k;
            const int rc = inc_exact(nucleus ? p / s2 : p, meta_b(mt, 3), &k);
            if (rc < 0) { bn.fail = 1; continue; }
            if (rc == 0) { mark(b); continue; }
            if (k) atomicAdd(&bn.esum[b], k);
        }
    }
    __syncthreads();
    if (bn.fail) BINS_FAIL();
    } else {
        // merged pass 3: the pending seq-3 increments, now that S and s2 are
        // exact; a rounding tie marks its bin for collection (its order
        // decides the tie)
        if (t == 0) bn.ncollect = 0;
        __syncthreads();
        for (int j = t; j < nd; j += kThreads) {
            const uint32_t en = ldg(defer + j);
            if (en == 0xffffffffu || !(en & kPend3)) continue;
            const float y = def_y(en);
            const int b = bin_of(y - m0);
            const uint32_t mt = bn.meta[b];
            if (mt & 1u) continue;
            uint32_t k;
            const int rc = inc_exact(glibc_expf(y - m) / S / s2, meta_b(mt, 3), &k);
            if (rc < 0) { bn.fail = 1; continue; }
            if (rc == 0) { mark(b); continue; }
            if (k) atomicAdd(&acc3[b], k);
        }
        __syncthreads();
        if (bn.fail) BINS_FAIL();
        GS_STAMP(22);
    }
#ifdef GS_TIMING
    if (t == 0 && blockIdx.x < 256 && bn.ncollect) g_fails[512 + blockIdx.x] |= 2;
#endif
    if (bn.ncollect) {
        if (!use_ix || !collect_now_ix(sm, row, t_one, T, gl, ix)) {
#ifdef GS_TIMING
            if (t == 0 && blockIdx.x < 256) g_fails[512 + blockIdx.x] |= 32;
#endif
            collect_now(sm, row, V, t_one, T, has_pen, gl);
        }
        if (!finish_now(sm, gl, tmp)) BINS_FAIL();
    }
    if (!build_groups(sm)) BINS_FAIL();
    N = build_walk(sm, gl, W, WT, m, m0, false);
    if (N < 0) BINS_FAIL();
    // summands of seq 3 (src/sampler.rs:56, :68); the walk ends at the cut
    if (t == 0) bn.cut_g = N;
    __syncthreads();
    for (int j = t; j < N; j += kThreads) {
        const float v = W[j];
        if (is_marker(v)) continue;
        const float p = v / S;
        W[j] = nucleus ? p / s2 : p;
        if (nucleus && WT[j] == cut_tok) atomicMin(&bn.cut_g, j);
    }
    __threadfence_block();
    __syncthreads();
    const int n3 = nucleus ? bn.cut_g + 1 : N;
    if (n3 > N) BINS_FAIL();
    GS_STAMP(23);
    gather_runs(sm, 3, acc3);
    float c3;
    const int jd = walk(sm, W, n3, 3, [r](float c) { return r < c; }, &c3);
    if (jd < 0) BINS_FAIL();
    if (jd < n3) *tok = (int)WT[jd];
    else if (nucleus) *tok = (int)WT[n3 - 1];
    else BINS_FAIL();   // the last element of the whole order: sort path
    return true;
}
