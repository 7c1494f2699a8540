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
constexpr float kDelta = 1.0f / 4096.0f;          // relative margin of the plan
constexpr float kDeltaS = 1.0f / 4096.0f;         // accepted |S / Spred - 1|
constexpr float kExpErr = 1.0f / 2097152.0f;      // bound on |fast_exp / expf - 1| (2^-21)
constexpr float kTieThr = 1.0f / 256.0f;          // expected ties that force collection
constexpr int kNoRun = 0x7fffffff;
constexpr int kMaxSeg = 512;                      // largest collected bin (wave sort)
constexpr uint32_t kNow = 0x80000000u;            // cnt[] flag: collect in pass 3
constexpr uint32_t kDeferCapG = 65536;            // deferred elements per row
constexpr uint32_t kWalkCap = 65536;              // items of the walk array per row
// deferred entry: id | bit 31 penalized value | bit 30 seq-2 done | bit 29 seq-3 done
constexpr uint32_t kDone2 = 0x40000000u, kDone3 = 0x20000000u, kIdMask = 0x1fffffffu;

__device__ __forceinline__ int bin_of(float dp)
{
    int b = (int)((kDUp - dp) * kInvW);
    return b > kBins - 1 ? kBins - 1 : b;
}

// exp(d) via v_exp_f32 with the rounding error of d*log2(e) compensated:
// t = RN(d*L), err = d*L - t (exact by fma) + d*(log2(e) - L), then
// exp2(t) * (1 + err*ln2).  Measured on gfx950 against glibc expf over every
// f32 d in [-30, 0]: max relative error 1.19e-7 (2^-23); kExpErr allows 4x.
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
// needed, bit3 nonempty, bits 4..7 seq-1 ties; bytes 1..3 = b1, b2, b3 + 128.
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

// Increment of every float in [lo, hi] (at most 8 of them): true if all give
// the same increment and none is a tie.
__device__ __forceinline__ bool inc_range(float lo, float hi, int b, uint32_t *k)
{
    uint32_t k0;
    if (inc_exact(lo, b, &k0) != 1) return false;
    float v = lo;
    for (int i = 0; i < 8 && v < hi; i++) {
        v = __uint_as_float(__float_as_uint(v) + 1u);   // next float (v > 0)
        uint32_t kk;
        if (inc_exact(v, b, &kk) != 1 || kk != k0) return false;
    }
    if (v < hi) return false;
    *k = k0;
    return true;
}

__device__ __forceinline__ float next_up(float v) { return __uint_as_float(__float_as_uint(v) + 1u); }

// Increment over every reachable value of a summand: p = e / S for every f32
// S in [Slo, Shi], and (with s2) q = p / s2 for every f32 s2 in [s2lo, s2hi].
// Returns 2 if some reachable value is a rounding tie (or the sets are too
// large to enumerate), 0 if all give the same increment (*k), 1 otherwise.
__device__ int inc_combos(float e, float Slo, float Shi, bool with_s2, float s2lo, float s2hi, int b, uint32_t *k)
{
    int n = 0;
    uint32_t k0 = 0;
    bool same = true;
    int ns = 0;
    for (float S = Slo; S <= Shi; S = next_up(S)) {
        if (++ns > 8) return 2;
        const float p = e / S;
        int nq = 0;
        for (float s2 = s2lo; s2 <= s2hi; s2 = next_up(s2)) {
            if (++nq > 96) return 2;
            uint32_t kk;
            if (inc_exact(with_s2 ? p / s2 : p, b, &kk) != 1) return 2;
            if (n++ == 0) k0 = kk;
            else same &= kk == k0;
            if (!with_s2) break;
        }
    }
    *k = k0;
    return same ? 0 : 1;
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
        mine[c] = j < n ? g[j] : 0ull;
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
        if (j < n) g[rank[c]] = mine[c];
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

// ---------------------------------------------------------------------------
// Pass-2 classification of one element (shared with the penalty fix-ups).
// Returns 0 negligible/overflow, 1 collected, 2 deferred, 3 bulk.
__device__ __forceinline__ int classify2(const BinsSmem &bn, float y, int *bin, uint32_t *k1, uint64_t *k23)
{
    const float dp = y - bn.m0;
    if (!(dp <= kDUp) || dp < -kDLo) return 0;
    const int b = bin_of(dp);
    *bin = b;
    const uint32_t mt = bn.meta[b];
    if (mt & 1u) return 1;
    const float e = fast_exp(y - bn.m);
    uint32_t a1, a2 = 0, a3 = 0;
    bool ok = inc_of(ldexpf(e, 23 - meta_b(mt, 1)), 2.0f * kExpErr, &a1);
    const float p = e * bn.inv_spred;
    if (mt & 2u) ok &= inc_of(ldexpf(p, 23 - meta_b(mt, 2)), bn.hw2, &a2);
    if (mt & 4u) ok &= inc_of(ldexpf(p * bn.inv_s2c, 23 - meta_b(mt, 3)), bn.hw3, &a3);
    if (!ok) return 2;
    *k1 = a1;
    *k23 = (uint64_t)a2 | ((uint64_t)a3 << 32);
    return 3;
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
            const uint32_t ties = (mt >> 4) & 15u;
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
__device__ void gather_runs(RowSmem &sm, int which)
{
    BinsSmem &bn = sm.x.bn;
    const int t = threadIdx.x;
    for (int i = t; i <= bn.ngroups; i += kThreads) bn.run[i] = 0ull;
    __syncthreads();
    for (int b = t; b < kBins; b += kThreads) {
        const uint32_t mt = bn.meta[b];
        if ((mt & 1u) || bn.off[b + 1] == bn.off[b]) continue;     // nonempty bulk bins only
        uint64_t v;
        if (which == 1) v = bn.esum[b];
        else if (which == 2) v = bn.k23[b] & 0xffffffffull;
        else v = bn.k23[b] >> 32;
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

// Exact replay of one accumulation over the walk array by a single wave,
// 64 items per step, DPP scans (see block_walk for the item encoding and the
// return values).  Wave-uniform: every lane returns the same result.
template <class RunFn, class Pred>
__device__ int wave_walk(const float *W, int n, RunFn runfn, Pred pred, float *s_out)
{
    const int lane = lane_id();
    float s = 0.0f;
    int pos = 0;
    while (pos < n && s == 0.0f) {               // 0 + a == a exactly
        const float v = W[pos];
        if (is_marker(v)) {
            ParFn f;
            if (!runfn(marker_run(v), -126, &f) || f.f0 != 0u) { *s_out = s; return -1; }
        } else {
            s = s + v;
            if (pred(s)) { *s_out = s; return pos; }
        }
        pos++;
    }
    float vnext = (pos + lane < n) ? W[pos + lane] : 0.0f;
    for (; pos < n; pos += 64) {
        const float v = vnext;
        vnext = (pos + 64 + lane < n) ? W[pos + 64 + lane] : 0.0f;   // prefetch
        const int lim = min(64, n - pos);
        const bool mk = is_marker(v);
        int start = 0;
        while (start < lim) {
            const int e = grid_exp(s);
            const uint32_t M = (uint32_t)ldexpf(s, 23 - e);
            ParFn f = {0u, 0u};
            bool bad = false;
            const bool valid = lane >= start && lane < lim;
            if (valid) {
                if (mk) bad = !runfn(marker_run(v), e, &f);
                else f = elem_fn(v, e);
            }
            const ParFn incl = wave_scan_incl(f);
            const uint32_t after = par_apply(incl, M & 1u);
            const bool cross = (M + after) >= (1u << 24);
            const float sa = ldexpf((float)(M + after), e - 23);
            const bool ev = valid && (cross || bad || pred(sa));
            const uint64_t mask = __ballot(ev);
            if (mask == 0) {
                s = rdl(sa, lim - 1);
                break;
            }
            const int first = __ffsll((unsigned long long)mask) - 1;
            if (__builtin_amdgcn_readlane((int)mk, first)) { *s_out = s; return -1; }   // event on a run
            const float prev = (first == start) ? s : rdl(sa, first - 1);
            const float na = prev + rdl(v, first);   // the reference's f32 add
            s = na;
            if (pred(na)) { *s_out = s; return pos + first; }
            start = first + 1;
        }
    }
    *s_out = s;
    return n;
}

// Run wave_walk on wave 0 and hand the result to the whole block.
template <class RunFn, class Pred>
__device__ int walk(RowSmem &sm, const float *W, int n, RunFn runfn, Pred pred, float *s_out)
{
    if (wave_id() == 0) {
        float sv;
        const int r = wave_walk(W, n, runfn, pred, &sv);
        if (lane_id() == 0) { sm.seq.first = r; sm.seq.s = sv; }
    }
    __syncthreads();
    const int r = sm.seq.first;
    *s_out = sm.seq.s;
    __syncthreads();
    return r;
}

template <class RunFn, class Pred>
__device__ int block_walk(const float *W, int n, RunFn runfn, Pred pred, float *s_out, SeqSmem &sm)
{
    const int t = threadIdx.x;
    float s = 0.0f;
    int pos = 0;
    // leading steps from s == 0: one at a time (0 + a == a exactly)
#ifdef GS_TIMING
    if (threadIdx.x == 0 && blockIdx.x == g_row) { g_fails[601] += n; g_fails[602]++; }
#endif
    while (pos < n && s == 0.0f) {
#ifdef GS_TIMING
        if (threadIdx.x == 0 && blockIdx.x == g_row) g_fails[603]++;
#endif
        const float v = W[pos];
        if (is_marker(v)) {
            ParFn f;
            if (!runfn(marker_run(v), -126, &f)) { *s_out = s; return -1; }
            if (f.f0 != 0u) { *s_out = s; return -1; }   // a run cannot open the sum
        } else {
            s = s + v;
            if (pred(s)) { *s_out = s; return pos; }
        }
        pos++;
    }
    const int tile = kThreads * kSeqPer;
    while (pos < n) {
        const int tend = min(pos + tile, n);
        float av[kSeqPer];
#pragma unroll
        for (int q = 0; q < kSeqPer; q++) {
            const int j = pos + t * kSeqPer + q;
            av[q] = (j < tend) ? W[j] : 0.0f;
        }
        int start = pos;
        for (;;) {
#ifdef GS_TIMING
            if (threadIdx.x == 0 && blockIdx.x == g_row) {
                int it = g_fails[600]++;
                if (it < 64) { g_fails[700 + 2 * it] = (int)__builtin_amdgcn_s_memrealtime(); g_fails[701 + 2 * it] = start - pos; }
            }
#endif
            const int e = grid_exp(s);
            const uint32_t M = (uint32_t)ldexpf(s, 23 - e);
            ParFn fn[kSeqPer];
            bool badq[kSeqPer];
            ParFn loc = {0u, 0u};
#pragma unroll
            for (int q = 0; q < kSeqPer; q++) {
                const int j = pos + t * kSeqPer + q;
                badq[q] = false;
                fn[q].f0 = 0u;
                fn[q].f1 = 0u;
                if (j >= start && j < tend) {
                    if (is_marker(av[q])) badq[q] = !runfn(marker_run(av[q]), e, &fn[q]);
                    else fn[q] = elem_fn(av[q], e);
                }
                loc = par_compose(loc, fn[q]);
            }
            if (t == 0) sm.first = 0x7fffffff;
            const ParFn ex = block_scan_excl(loc, sm);   // contains a barrier
            const uint32_t pM = M & 1u;
            uint32_t before = par_apply(ex, pM);
            int my_first = 0x7fffffff;
#pragma unroll
            for (int q = 0; q < kSeqPer; q++) {
                const int j = pos + t * kSeqPer + q;
                const uint32_t inc = par_apply(fn[q], (pM + before) & 1u);
                const uint32_t after = sat_add(before, inc);
                if (j >= start && j < tend && my_first == 0x7fffffff) {
                    const bool cross = (M + after) >= (1u << 24);
                    const bool stop = !cross && pred(ldexpf((float)(M + after), e - 23));
                    if (cross || stop || badq[q]) my_first = j;
                }
                before = after;
            }
            if (my_first != 0x7fffffff) atomicMin(&sm.first, my_first);
            __syncthreads();
            const int first = sm.first;
            if (first == 0x7fffffff) {
                const int last = tend - 1;
                const int owner = (last - pos) / kSeqPer;
                if (t == owner) {
                    uint32_t b2 = par_apply(ex, pM);
#pragma unroll
                    for (int q = 0; q < kSeqPer; q++) {
                        const int j = pos + t * kSeqPer + q;
                        if (j <= last) b2 = sat_add(b2, par_apply(fn[q], (pM + b2) & 1u));
                    }
                    sm.s = ldexpf((float)(M + b2), e - 23);
                }
                __syncthreads();
                s = sm.s;
                __syncthreads();
                break;
            }
            const int owner = (first - pos) / kSeqPer;
            if (t == owner) {
                uint32_t b2 = par_apply(ex, pM);
                float sa = s;
                int nxt = first + 1;
#pragma unroll
                for (int q = 0; q < kSeqPer; q++) {
                    const int j = pos + t * kSeqPer + q;
                    if (j >= start && j < first) b2 = sat_add(b2, par_apply(fn[q], (pM + b2) & 1u));
                    if (j == first) {
                        if (is_marker(av[q])) nxt = -1;            // event on a run
                        else {
                            const float sb = ldexpf((float)(M + b2), e - 23);
                            sa = sb + av[q];                        // the reference's f32 add
                            if (pred(sa)) nxt = -2 - first;
                        }
                    }
                }
                sm.s = sa;
                sm.start = nxt;
            }
            __syncthreads();
            s = sm.s;
            const int nxt = sm.start;
            __syncthreads();
            if (nxt == -1) { *s_out = s; return -1; }
            if (nxt < -1) { *s_out = s; return -2 - nxt; }
            start = nxt;
            if (start >= tend) break;
        }
        pos = tend;
    }
    *s_out = s;
    return n;
}

// One accumulation over runs and groups (all threads call).  With last_g >= 0
// it stops after the first last_n elements of group last_g.  tie_up adds the
// run's seq-1 tie count (ties rounded up instead of down).  Returns false on
// a failed check; *stop_g = -1 if the predicate never held.
template <class A, class P>
__device__ bool walk_seq(RowSmem &sm, const uint64_t *gl, int which, bool tie_up, int last_g, int last_n,
                         A a_of, P pred, float *s_out, int *stop_g, int *stop_j)
{
    BinsSmem &bn = sm.x.bn;
    const int G = bn.ngroups;
    float s = 0.0f;
    *stop_g = -1;
    *stop_j = -1;
    for (int g = 0; g <= G; g++) {
        if (last_g >= 0 && g > last_g) break;
        if (g > 0 && bn.runb[g] != kNoRun) {
            const int packed = bn.runb[g];
            if (which == 2 && !(packed & (1 << 24))) return false;
            if (which == 3 && !(packed & (1 << 25))) return false;
            const uint64_t R = bn.run[g] + (tie_up ? bn.runt[g] : 0u);
            if (R) {
                if (!(s > 0.0f)) return false;
                const int eb = ((packed >> (8 * (which - 1))) & 255) - 128;
                const int e = grid_exp(s);
                if (e != eb) return false;
                const uint64_t M = (uint64_t)ldexpf(s, 23 - e);
                if (M + R >= (1ull << 24)) return false;
                s = ldexpf((float)(M + R), e - 23);
                if (pred(s)) return false;   // the event lies inside the run
            }
        }
        if (g == G) break;
        const uint32_t b0 = bn.gbeg[g];
        const int n = (g == last_g) ? last_n : (int)(bn.gend[g] - b0);
        float so;
        const int stop = block_seqsum([&](int j) { return a_of(gl[b0 + j]); }, n, s, pred, &so, sm.seq);
        s = so;
        if (stop < n) { *stop_g = g; *stop_j = stop; break; }
    }
    *s_out = s;
    return true;
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
        for (uint32_t j = bn.cnt[b] & ~kNow; j < bn.off[b + 1]; j++) gl[j] = 0ull;
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

// Increment functor of the runs for accumulation `which` (tie_up: the run's
// seq-1 ties round up).
struct RunFn {
    const BinsSmem *bn;
    int which;
    bool tie_up;
    __device__ bool operator()(int r, int e, ParFn *f) const
    {
        f->f0 = f->f1 = 0u;
        if (r == 0 || bn->runb[r] == kNoRun) return true;
        const int packed = bn->runb[r];
        if (which == 2 && !(packed & (1 << 24))) return false;
        if (which == 3 && !(packed & (1 << 25))) return false;
        const uint64_t R = bn->run[r] + (tie_up ? bn->runt[r] : 0u);
        if (R == 0) return true;
        if (e != ((packed >> (8 * (which - 1))) & 255) - 128) return false;
        const uint32_t R32 = R > kSat ? kSat : (uint32_t)R;
        f->f0 = f->f1 = R32;
        return true;
    }
};
__device__ __forceinline__ RunFn run_fn(const BinsSmem &bn, int which, bool tie_up) { return RunFn{&bn, which, tie_up}; }

// The flat walk array: per group g, a marker of run g, then the group's
// sorted entries as exact summands expf(y - m) (0 for removed entries);
// a final marker for the run after the last group.  WT holds token ids.
// Returns the item count, or -1 if it does not fit.
__device__ int build_walk(RowSmem &sm, const uint64_t *gl, float *W, uint32_t *WT, float m)
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
    for (int g = t; g <= G; g += kThreads) { W[bn.wbase[g]] = make_marker(g); WT[bn.wbase[g]] = 0xffffffffu; }
    for (int g = 0; g < G; g++) {
        const uint32_t b0 = bn.gbeg[g], n = bn.gend[g] - b0, w0 = bn.wbase[g] + 1;
        for (uint32_t p = t; p < n; p += kThreads) {
            const uint64_t en = gl[b0 + p];
            W[w0 + p] = en ? glibc_expf(key2f((uint32_t)(en >> 32)) - m) : 0.0f;
            WT[w0 + p] = ~(uint32_t)en;
        }
    }
    __threadfence_block();
    __syncthreads();
    return (int)N;
}

// ---------------------------------------------------------------------------
// The binned path.  Returns true with *tok / *status set, or false to ask for
// the sort-based path.  Needs a 16-byte aligned row and `gl`, a per-row list
// of lcap >= V + kOverCap + 2*kHashSlots u64 entries in global memory.
__device__ bool full_bins_row(RowSmem &sm, const float *row, int V, float T, float top_p,
                              bool has_pen, float r, uint64_t *gl, uint32_t lcap, int *tok,
                              int *status)
{
    // deferred ids live in the upper part of the scratch row
    const uint32_t lneed = (uint32_t)V + (uint32_t)(kOverCap + 2 * kHashSlots);
    if (lcap < lneed + kDeferCapG / 2 + kWalkCap) BINS_FAIL();
    uint32_t *defer = reinterpret_cast<uint32_t *>(gl + lneed);
    const uint32_t dcap = kDeferCapG;
    float *W = reinterpret_cast<float *>(gl + lneed + kDeferCapG / 2);
    uint32_t *WT = reinterpret_cast<uint32_t *>(W + kWalkCap);
    BinsSmem &bn = sm.x.bn;
    const int t = threadIdx.x;
    const bool t_one = (T == 1.0f);
    const float4 *r4 = reinterpret_cast<const float4 *>(row);
    const int n4 = V >> 2;
    if (n4 == 0) BINS_FAIL();

    for (int b = t; b < kBins; b += kThreads) bn.cnt[b] = 0;
    if (t == 0) { bn.nover = 0; bn.ndefer = 0; bn.fail = 0; bn.ncollect = 0; }

    // ---- pass 1: counts, max, NaN ------------------------------------------
    float tmax = -INFINITY;
    int nan = 0;
    float m0 = 0.0f;
    auto visit = [&](int i, float x) {
        const float y = t_one ? x : x / T;
        nan |= (int)isnan(y);
        if (y > tmax && !(has_pen && hash_find(sm, (uint32_t)i) >= 0)) tmax = y;
        const float dp = y - m0;
        if (dp > kDUp) {
            const int slot = atomicAdd(&bn.nover, 1);
            if (slot < kOverCap) bn.over[slot] = list_entry(y, (uint32_t)i);
        } else if (dp >= -kDLo) {
            atomicAdd(&bn.cnt[bin_of(dp)], 1u);
        }
    };
    for (int base = 0; base < n4; base += kThreads * kUnroll) {
        float4 v[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; u++) {
            const int q = base + u * kThreads + t;
            if (q < n4) v[u] = r4[q];
        }
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
    }
    for (int i = (n4 << 2) + t; i < V; i += kThreads) visit(i, row[i]);
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
    GS_STAMP(10);

    // ---- penalty: penalized values join the counts and the overflow --------
    if (has_pen) {
        for (int j = t; j < bn.nover; j += kThreads)
            if (hash_find(sm, ~(uint32_t)bn.over[j]) >= 0) bn.over[j] = 0ull;
        __syncthreads();
        for (int s = t; s < kHashSlots; s += kThreads) {
            const uint32_t id = sm.hkey[s];
            if (id == kEmpty) continue;
            const float yp = t_one ? __uint_as_float(sm.hval[s]) : __uint_as_float(sm.hval[s]) / T;
            const float dq = yp - m0;
            if (dq > kDUp) {
                const int slot = atomicAdd(&bn.nover, 1);
                if (slot < kOverCap) bn.over[slot] = list_entry(yp, id);
            } else if (dq >= -kDLo) {
                atomicAdd(&bn.cnt[bin_of(dq)], 1u);   // raw counts stay: segment sizes are upper bounds
            }
        }
        __syncthreads();
        if (bn.nover > kOverCap) BINS_FAIL();
    }
    const int nover = bn.nover;

    // ---- plan ---------------------------------------------------------------
    constexpr int kPer = kBins / kThreads;
    static_assert(kPer * kThreads == kBins, "bins per thread");
    const float wbin = (kDUp + kDLo) / (float)kBins;
    const float shift = m0 - m;            // e = exp(d' + shift)
    auto e_at = [&](float bpos) { return (double)fast_exp(kDUp - bpos * wbin + shift); };
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
#pragma unroll
    for (int c = 0; c < kPer; c++) {
        const int b = kPer * t + c;
        cntv[c] = bn.cnt[b];
        eb[c] = (double)cntv[c] * e_at((float)b + 0.5f);
        loc += eb[c];
        ctot += cntv[c];
    }
    double stot;
    const double pre = block_excl_f64(loc, &stot, sm) + osum;
    stot += osum;
    uint32_t call;
    const uint32_t cpre = block_excl_u32(ctot, &call, sm);
    if ((uint32_t)nover + call > lcap) BINS_FAIL();
    double plo[kPer + 1];
    plo[0] = pre;
#pragma unroll
    for (int c = 0; c < kPer; c++) plo[c + 1] = plo[c] + eb[c];
    // Predicted seq-1 result: in a bulk bin every summand is rounded to the
    // grid of the running sum (src/sampler.rs:54); with the bin's summands
    // between its edge values, a bin inside one rounding cell contributes
    // count * k exactly, a bin across one cell boundary is split by the
    // position of the boundary (summands uniform in d), and wide bins
    // contribute their mean.
    double spred = 0.0;
#pragma unroll
    for (int c = 0; c < kPer; c++) {
        const int b = kPer * t + c;
        if (cntv[c] == 0) continue;
        if (plo[c] <= 0.0) { spred += eb[c]; continue; }
        const double g = ldexp(1.0, grid_exp((float)plo[c]) - 23);
        const double mlo = e_at((float)b + 1.0f) / g, mhi = e_at((float)b) / g;
        const double klo = floor(mlo + 0.5), khi = floor(mhi + 0.5);
        double k;
        if (klo == khi) k = klo;
        else if (khi == klo + 1.0) {
            const double h = klo + 0.5;
            const double f = (log(mhi) - log(h)) / (log(mhi) - log(mlo));
            k = klo + f;
        } else k = eb[c] / ((double)cntv[c] * g);
        spred += (double)cntv[c] * k * g;
    }
    spred = block_sum_f64(spred, sm) + osum;
    const double lost = stot - spred;
    const double Spred = stot - lost;
    const bool nucleus = top_p < 1.0f;
    if (t == 0) { bn.cut_g = kBins; bn.Spred = (float)Spred; }
    __syncthreads();
    double s2lo = 1.0, s2hi = 1.0;
    if (nucleus) {
        if (stot / Spred < (double)top_p * (1.0 + 2.0 * kDelta)) BINS_FAIL();   // the cut may not happen
#pragma unroll
        for (int c = 0; c < kPer; c++) {
            if (cntv[c] == 0) continue;
            if (plo[c + 1] / Spred * (1.0 + kDelta) >= (double)top_p) { atomicMin(&bn.cut_g, kPer * t + c); break; }
        }
        __syncthreads();
        const int cb = bn.cut_g;
        if (cb >= kBins) BINS_FAIL();
        // the cut element lies in bin cb, or anywhere from the max (e = 1) on
        // if the overflow segment may already reach top_p
        const double ehc = (osum / Spred * (1.0 + kDelta) >= (double)top_p) ? 1.0 : e_at((float)cb) * 1.001;
        s2lo = (double)top_p;
        s2hi = (double)top_p + ehc / Spred * (1.0 + 4.0 * kDelta);
    }
    const double s2c = 0.5 * (s2lo + s2hi);
    const float hw2 = kDeltaS + 2.0f * kExpErr + 4.0f / 16777216.0f;
    const float hw3 = hw2 + (float)((s2hi - s2lo) / (2.0 * s2c)) + 4.0f / 16777216.0f;
    if (t == 0) {
        bn.inv_spred = (float)(1.0 / Spred);
        bn.inv_s2c = nucleus ? (float)(1.0 / s2c) : 1.0f;
        bn.hw2 = hw2;
        bn.hw3 = hw3;
        bn.s2lo = (float)s2lo;
        bn.s2hi = (float)s2hi;
        bn.off[kBins] = (uint32_t)nover + call;
    }
    {
        uint32_t o = (uint32_t)nover + cpre;
#pragma unroll
        for (int c = 0; c < kPer; c++) {
            const int b = kPer * t + c;
            const double lo = plo[c], hi = plo[c + 1];
            const double ehi = e_at((float)b) * 1.001;
            const double dl = 1.0 - kDelta, dh = 1.0 + kDelta;
            const double cn = (double)cntv[c];
            bool col = !(lo > 0.0);
            int b1 = 0, b2 = 0, b3 = 0;
            bool k2 = false, k3 = false;
            if (cntv[c] && !col) {
                b1 = grid_exp((float)lo);
                col |= grid_exp((float)(lo * dl)) != grid_exp((float)(hi * dh));
                const int c1 = ilogb(ehi);
                if (c1 < b1) col |= cn * ldexp(1.0, c1 - b1) > kTieThr;
                col |= cn * (ldexp(ehi, 23 - b1) + 1.0) >= 4.0e9;
                const double plo_ = lo / Spred, phi_ = hi / Spred;
                const double pe = ehi / Spred;
                bool reach3 = true;
                if (nucleus) {
                    k2 = plo_ * dl < (double)top_p;
                    reach3 = k2;
                    if (k2) {
                        b2 = grid_exp((float)plo_);
                        col |= grid_exp((float)(plo_ * dl)) != grid_exp((float)(phi_ * dh));
                        col |= phi_ * dh >= (double)top_p;
                        const int c2 = ilogb(pe);
                        if (c2 < b2) col |= cn * ldexp(1.0, c2 - b2) > kTieThr;
                        col |= cn * (ldexp(pe, 23 - b2) + 1.0) >= 4.0e9;
                    }
                }
                if (reach3) {
                    const double qlo = plo_ / s2c, qhi = phi_ / s2c;
                    k3 = qlo * dl <= (double)r;
                    if (k3) {
                        b3 = grid_exp((float)qlo);
                        col |= grid_exp((float)(qlo * dl)) != grid_exp((float)(qhi * dh));
                        col |= qhi * dh > (double)r;
                        const int c3 = ilogb(pe / s2c);
                        if (c3 < b3) col |= cn * ldexp(1.0, c3 - b3) > kTieThr;
                        col |= cn * (ldexp(pe / s2c, 23 - b3) + 1.0) >= 4.0e9;
                    }
                }
            }
            if (cntv[c] == 0) col = false;
            bn.meta[b] = (col ? 1u : 0u) | (k2 ? 2u : 0u) | (k3 ? 4u : 0u) | (cntv[c] ? 8u : 0u) |
                         ((uint32_t)(b1 + 128) << 8) | ((uint32_t)(b2 + 128) << 16) |
                         ((uint32_t)(b3 + 128) << 24);
            bn.off[b] = o;
            bn.cnt[b] = o;                  // cursor of collected bins
            bn.esum[b] = 0ull;
            bn.k23[b] = 0ull;
            o += cntv[c];
        }
    }
    for (int j = t; j < nover; j += kThreads) gl[j] = bn.over[j];
    __syncthreads();
    GS_STAMP(11);

    // ---- pass 2 -------------------------------------------------------------
    auto visit2 = [&](int i, float x) {
        const float y = t_one ? x : x / T;
        int b;
        uint32_t k1;
        uint64_t k23;
        const int cl = classify2(bn, y, &b, &k1, &k23);
        if (cl == 1) {
            const uint32_t slot = atomicAdd(&bn.cnt[b], 1u);
            gl[slot] = list_entry(y, (uint32_t)i);
        } else if (cl == 2) {
            const int slot = atomicAdd(&bn.ndefer, 1);
            if ((uint32_t)slot < dcap) defer[slot] = (uint32_t)i;
        } else if (cl == 3) {
            if (k1) atomicAdd((unsigned long long *)&bn.esum[b], (unsigned long long)k1);
            if (k23) atomicAdd((unsigned long long *)&bn.k23[b], (unsigned long long)k23);
        }
    };
    row_for_each(row, V, true, visit2);
    __syncthreads();
    GS_STAMP(12);
    if (has_pen) {
        // undo raw contributions of penalized ids, then add the penalized values
        for (int s = t; s < kHashSlots; s += kThreads) {
            const uint32_t id = sm.hkey[s];
            if (id == kEmpty) continue;
            const float yr = t_one ? row[id] : row[id] / T;
            int b;
            uint32_t k1;
            uint64_t k23;
            if (classify2(bn, yr, &b, &k1, &k23) == 3) {
                if (k1) atomicAdd((unsigned long long *)&bn.esum[b], (unsigned long long)(0ull - (uint64_t)k1));
                if (k23) atomicAdd((unsigned long long *)&bn.k23[b], (unsigned long long)(0ull - k23));
            }
        }
        for (int b = t; b < kBins; b += kThreads) {
            if (!(bn.meta[b] & 1u)) continue;
            for (uint32_t j = bn.off[b]; j < bn.cnt[b]; j++)
                if (hash_find(sm, ~(uint32_t)gl[j]) >= 0) gl[j] = 0ull;
        }
        const int nd = min((uint32_t)bn.ndefer, dcap);
        for (int j = t; j < nd; j += kThreads)
            if (hash_find(sm, defer[j] & kIdMask) >= 0) defer[j] = 0xffffffffu;
        __threadfence_block();
        __syncthreads();
        for (int s = t; s < kHashSlots; s += kThreads) {
            const uint32_t id = sm.hkey[s];
            if (id == kEmpty) continue;
            const float yp = t_one ? __uint_as_float(sm.hval[s]) : __uint_as_float(sm.hval[s]) / T;
            int b;
            uint32_t k1;
            uint64_t k23;
            const int cl = classify2(bn, yp, &b, &k1, &k23);
            if (cl == 1) {
                const uint32_t slot = atomicAdd(&bn.cnt[b], 1u);
                gl[slot] = list_entry(yp, id);
            } else if (cl == 2) {
                const int slot = atomicAdd(&bn.ndefer, 1);
                if ((uint32_t)slot < dcap) defer[slot] = id | 0x80000000u;
            } else if (cl == 3) {
                if (k1) atomicAdd((unsigned long long *)&bn.esum[b], (unsigned long long)k1);
                if (k23) atomicAdd((unsigned long long *)&bn.k23[b], (unsigned long long)k23);
            }
        }
        __syncthreads();
    }
#ifdef GS_TIMING
    if (t == 0 && blockIdx.x == g_row) g_stamp[28] = (uint64_t)bn.ndefer;
#endif
    if ((uint32_t)bn.ndefer > dcap) BINS_FAIL();
    if (!finish_segments(sm, gl, [&](int b) { return (bn.meta[b] & 1u) != 0u; })) BINS_FAIL();
    if (wave_id() == 0 && !wave_sort_segment(gl, nover)) bn.fail = 1;
    __threadfence_block();
    __syncthreads();
    if (bn.fail) BINS_FAIL();
    GS_STAMP(13);

    // ---- resolve deferred elements -------------------------------------------
    const int nd = bn.ndefer;
    auto def_y = [&](uint32_t en) {
        const uint32_t id = en & kIdMask;
        float x = row[id];
        if (en & 0x80000000u) {
            const int s = hash_find(sm, id);
            if (s >= 0) x = __uint_as_float(sm.hval[s]);
        }
        return t_one ? x : x / T;
    };
    auto mark = [&](int b) {
        const uint32_t old = atomicOr(&bn.meta[b], 1u);
        if (!(old & 1u)) { bn.cnt[b] = bn.off[b] | kNow; atomicAdd(&bn.ncollect, 1); }
    };
    // seq 1: exact increments; a tie adds its lower choice and is counted
    for (int j = t; j < nd; j += kThreads) {
        const uint32_t en = defer[j];
        if (en == 0xffffffffu) continue;
        const float y = def_y(en);
        const int b = bin_of(y - m0);
        uint32_t k;
        const int rc = inc_exact(glibc_expf(y - m), meta_b(bn.meta[b], 1), &k);
        if (rc < 0) { bn.fail = 1; continue; }
        if (k) atomicAdd((unsigned long long *)&bn.esum[b], (unsigned long long)k);
        if (rc == 0) {
            const uint32_t old = atomicAdd(&bn.meta[b], 16u);
            if (((old >> 4) & 15u) == 15u) bn.fail = 1;
        }
    }
    __syncthreads();
    if (bn.fail) BINS_FAIL();
    GS_STAMP(16);
    if (!build_groups(sm)) BINS_FAIL();
    gather_runs(sm, 1);
    int N = build_walk(sm, gl, W, WT, m);
    if (N < 0) BINS_FAIL();
    GS_STAMP(17);
    float Slo, Shi;
    if (walk(sm, W, N, run_fn(bn, 1, false), [](float) { return false; }, &Slo) != N) BINS_FAIL();
    GS_STAMP(18);
    if (walk(sm, W, N, run_fn(bn, 1, true), [](float) { return false; }, &Shi) != N) BINS_FAIL();
    GS_STAMP(19);
#ifdef GS_TIMING
    if (t == 0 && blockIdx.x == g_row) { g_stamp[30] = __float_as_uint(Slo); g_stamp[31] = ((uint64_t)__float_as_uint(Shi) << 32) | __float_as_uint(bn.Spred); }
#endif
    if (!(Slo >= bn.Spred * (1.0f - kDeltaS) && Shi <= bn.Spred * (1.0f + kDeltaS))) BINS_FAIL();
    GS_STAMP(14);
    // bins with a seq-1 tie need the exact order
    for (int b = t; b < kBins; b += kThreads)
        if (!(bn.meta[b] & 1u) && ((bn.meta[b] >> 4) & 15u)) mark(b);
    __syncthreads();
    // seq 2 and seq 3 over the reachable values of S and s2: a possible tie
    // needs the exact order (collect the bin); a unique increment is added
    // now; otherwise the increment waits for the exact S or s2 (kDone bits).
    for (int j = t; j < nd; j += kThreads) {
        const uint32_t en = defer[j];
        if (en == 0xffffffffu) continue;
        const float y = def_y(en);
        const int b = bin_of(y - m0);
        const uint32_t mt = bn.meta[b];
        if (mt & 1u) continue;
        const float e = glibc_expf(y - m);
        uint32_t k, st = 0;
        if (mt & 2u) {
            const int rc = inc_combos(e, Slo, Shi, false, 1.0f, 1.0f, meta_b(mt, 2), &k);
            if (rc == 2) { mark(b); continue; }
            if (rc == 0) { st |= kDone2; if (k) atomicAdd((unsigned long long *)&bn.k23[b], (unsigned long long)k); }
        } else st |= kDone2;
        if (mt & 4u) {
            const int rc = inc_combos(e, Slo, Shi, nucleus, bn.s2lo, bn.s2hi, meta_b(mt, 3), &k);
            if (rc == 2) { mark(b); continue; }
            if (rc == 0) { st |= kDone3; if (k) atomicAdd((unsigned long long *)&bn.k23[b], (unsigned long long)k << 32); }
        } else st |= kDone3;
        defer[j] = en | st;
    }
    __syncthreads();
#ifdef GS_TIMING
    if (t == 0 && blockIdx.x == g_row) g_stamp[29] = (uint64_t)bn.ncollect;
#endif

    // ---- pass 3: collect the marked bins ------------------------------------
    if (bn.ncollect > 0) {
        auto visit3 = [&](int i, float x) {
            const float y = t_one ? x : x / T;
            const float dp = y - m0;
            if (!(dp <= kDUp) || dp < -kDLo) return;
            const int b = bin_of(dp);
            if (bn.cnt[b] & kNow) {
                const uint32_t slot = atomicAdd(&bn.cnt[b], 1u) & ~kNow;
                gl[slot] = list_entry(y, (uint32_t)i);
            }
        };
        row_for_each(row, V, true, visit3);
        __syncthreads();
        GS_STAMP(20);
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
                const float yp = t_one ? __uint_as_float(sm.hval[s]) : __uint_as_float(sm.hval[s]) / T;
                const float dq = yp - m0;
                if (!(dq <= kDUp) || dq < -kDLo) continue;
                const int b = bin_of(dq);
                if (bn.cnt[b] & kNow) {
                    const uint32_t slot = atomicAdd(&bn.cnt[b], 1u) & ~kNow;
                    gl[slot] = list_entry(yp, id);
                }
            }
            __syncthreads();
        }
        if (!finish_segments(sm, gl, [&](int b) { return (bn.cnt[b] & kNow) != 0u; })) BINS_FAIL();
        if (!build_groups(sm)) BINS_FAIL();
        N = build_walk(sm, gl, W, WT, m);
        if (N < 0) BINS_FAIL();
        GS_STAMP(21);
    }

    // ---- exact walks --------------------------------------------------------
    float S = Slo;
    if (bn.ncollect > 0) {
        gather_runs(sm, 1);
        if (walk(sm, W, N, run_fn(bn, 1, false), [](float) { return false; }, &S) != N) BINS_FAIL();
        if (!(S >= Slo && S <= Shi)) BINS_FAIL();
    } else if (Slo != Shi) BINS_FAIL();
    GS_STAMP(22);
    // late seq-2 increments, now that S is exact
    for (int j = t; j < nd; j += kThreads) {
        const uint32_t en = defer[j];
        if (en == 0xffffffffu || (en & kDone2)) continue;
        const float y = def_y(en);
        const int b = bin_of(y - m0);
        const uint32_t mt = bn.meta[b];
        if (mt & 1u) continue;
        uint32_t k;
        if (inc_exact(glibc_expf(y - m) / S, meta_b(mt, 2), &k) != 1) { bn.fail = 1; continue; }
        if (k) atomicAdd((unsigned long long *)&bn.k23[b], (unsigned long long)k);
    }
    __syncthreads();
    if (bn.fail) BINS_FAIL();
    // summands of seq 2: p = e / S (src/sampler.rs:56)
    for (int j = t; j < N; j += kThreads) { const float v = W[j]; if (!is_marker(v)) W[j] = v / S; }
    __threadfence_block();
    __syncthreads();
    int n3 = N, js = -1;
    float s2 = 1.0f;
    if (nucleus) {
        gather_runs(sm, 2);
        js = walk(sm, W, N, run_fn(bn, 2, false), [top_p](float c) { return c >= top_p; }, &s2);
        if (js < 0 || js >= N || !(s2 >= bn.s2lo && s2 <= bn.s2hi)) BINS_FAIL();
        // summands of seq 3: q = p / s2 (src/sampler.rs:68)
        for (int j = t; j <= js; j += kThreads) { const float v = W[j]; if (!is_marker(v)) W[j] = v / s2; }
        __threadfence_block();
        __syncthreads();
        n3 = js + 1;
    }
    // late seq-3 increments, now that S and s2 are exact
    for (int j = t; j < nd; j += kThreads) {
        const uint32_t en = defer[j];
        if (en == 0xffffffffu || (en & kDone3)) continue;
        const float y = def_y(en);
        const int b = bin_of(y - m0);
        const uint32_t mt = bn.meta[b];
        if ((mt & 1u) || !(mt & 4u)) continue;
        const float p = glibc_expf(y - m) / S;
        uint32_t k;
        if (inc_exact(nucleus ? p / s2 : p, meta_b(mt, 3), &k) != 1) { bn.fail = 1; continue; }
        if (k) atomicAdd((unsigned long long *)&bn.k23[b], (unsigned long long)k << 32);
    }
    __syncthreads();
    if (bn.fail) BINS_FAIL();
    GS_STAMP(23);
    gather_runs(sm, 3);
    float c3;
    const int jd = walk(sm, W, n3, run_fn(bn, 3, false), [r](float c) { return r < c; }, &c3);
    if (jd < 0) BINS_FAIL();
    if (jd < n3) *tok = (int)WT[jd];
    else if (nucleus) *tok = (int)WT[js];
    else BINS_FAIL();   // the last element of the whole order: sort path
    return true;
}
