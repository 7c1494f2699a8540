// gs_full3.hpp -- the exact full-vocabulary path by increment histograms.
// (Included inside namespace gs by gs_kernels.hip after gs_full.hpp, whose
// bins of d' = y - m0, pass-1 masses, fast exp and block helpers it shares.)
//
// The reference (src/sampler.rs:44-78) sorts all V scaled logits y
// (descending, ties by index here) and runs three sequential f32
// accumulations in sorted order:
//   seq 1  S  = sum of a_j = expf(y_j - max)                    (:53-54)
//   seq 2  cum of p_j = a_j / S until cum >= top_p: cut, s2      (:56, :59-67)
//   seq 3  cum of q_j = p_j / s2 (or p_j) until r < cum          (:68, :71-78)
// While a running f32 sum s stays in one binade [2^e, 2^(e+1)) each add is
// s + g k with g = 2^(e-23) and k = the summand in units of g rounded to
// nearest; only a summand at exactly k + 1/2 (a rounding tie) depends on s,
// through the parity of s / g.
//
// Here every element computes its own k in the pass: k = rint(a~ F) with a~
// a fast exp accurate to 2^-22 and F = 2^(23-e) (seq 1) or the grid-scaled
// 1/S, 1/(S s2) (seqs 2, 3).  When a~ F lies within the error band of a
// half-integer the element is set aside and resolved with glibc's expf
// (then it is either an exact k or a rounding tie).  The k are counted in a
// histogram per run of bins (a "level" array): a run is a stretch of the
// sorted order that a plan, from pass-1 masses, predicts to stay in one
// binade.  Elements of the same k commute, and a tie sits between levels k+1
// and k, so a run's contribution is its level sum plus one parity step per
// tie.  The stretches where the sum may change binade (windows), the nucleus
// cut, the draw, and the head of the row (large summands whose level counts
// would not fit) are listed instead: their elements are sorted by (y, index)
// and added one by one with the reference's own f32 adds.  Every prediction
// is checked; a failed check returns false and the row goes to the next
// path (the same result, slower).
//
// Passes over the row: pass 1 (HBM) bins and masses, pass 2 (cache) seq 1,
// pass 3 (cache) seqs 2 and 3 for the elements above the cut.

// Development builds record per row (< 1024) the failing line ([0]) and
// statistics, and per row (< 256) stage timestamps.
#if defined(GS_TIMING) || defined(GS_DIAG)
__device__ int g_v3diag[1024 * 32];
__device__ uint32_t g_v3t[256 * 32];
#define F3_STAT(k, v) do { if (threadIdx.x == 0 && blockIdx.x < 1024) g_v3diag[blockIdx.x * 32 + (k)] = (int)(v); } while (0)
__device__ int g_v3dump[64 * 256];
#define F3_DUMP(k, v) do { if (blockIdx.x < 64) g_v3dump[blockIdx.x * 256 + (k)] = (int)(v); } while (0)
#define F3_TS(k) do { if (threadIdx.x == 0 && blockIdx.x < 256) g_v3t[blockIdx.x * 32 + (k)] = (uint32_t)__builtin_amdgcn_s_memrealtime(); } while (0)
#else
#define F3_STAT(k, v) do { } while (0)
#define F3_DUMP(k, v) do { } while (0)
#define F3_TS(k) do { } while (0)
#endif
#ifdef GS_TIMING
#define F3_CLK(v) const uint64_t v = clock64()
#define F3_CSTAT(k, v) F3_STAT(k, v)
#else
#define F3_CLK(v) do { } while (0)
#define F3_CSTAT(k, v) do { } while (0)
#endif
#define F3_FAIL() do { F3_STAT(0, __LINE__); return false; } while (0)

constexpr uint32_t kF3Listed = 0x80000000u;   // role word: a listed bin; bits 0-23: its list cursor
constexpr uint32_t kF3Cur = 0x00ffffffu;
constexpr uint32_t kF3In2 = 0x40000000u;      // in a run of seq 1 (pass 2) / seq 2 (pass 3): bits 8-13 the run
constexpr uint32_t kF3In3 = 0x20000000u;      // in a run of seq 3: bits 0-5 the run
// Role words of the passes (f.w, f.u.w23): bit 31 listed (bits 0-23 its
// cursor), else bit 30 (seqs 1 and 2) or bit 31 of the seq-3 word: counted,
// bits 24-29 the scale shift sh = 23 - e, bits 0-23 the level offset + 2^23.
constexpr uint32_t kF3W3 = 0x80000000u;
constexpr uint32_t kF3L2Bit = 0x10000000u, kF3L3Bit = 0x08000000u;   // per-bin roles of seqs 2 / 3 (global table): listed
constexpr uint32_t kF3KeyListed = 0xffffffffu, kF3KeyNone = 0xfffffffeu;
// a~ = exp2(RN(d log2 e)) is within 2^-18.5 of expf(d) for |d| <= 32
// (the product's rounding, the constant's and v_exp_f32's 1 ulp); beyond,
// every scaled summand is far below 1/2.  The bands hold that error, and for
// seqs 2 and 3 the roundings of 1/S, of the products and of p and q.
constexpr float kF3Band1 = 7.62939453125e-6f;      // 2^-17
constexpr float kF3Band23 = 1.52587890625e-5f;     // 2^-16
constexpr double kF3Lo = 1.0 - 1.0 / 65536.0, kF3Hi = 1.0 + 1.0 / 65536.0;   // level range margins (2^-16)

// A list entry (key << 32 | ~index) whose element left the list (the raw
// value of a penalized id): the low word becomes the index itself, which
// ranks it below the live entries of its key and keeps it unique.
__device__ __forceinline__ bool f3_live(uint64_t en) { return ((uint32_t)en & 0x80000000u) != 0u; }
__device__ __forceinline__ uint64_t f3_dead(uint64_t en) { return (en & 0xffffffff00000000ull) | (uint64_t)(~(uint32_t)en); }

// 16-bit level counters, two per LDS word: slot j is the low (j even) or
// high half of word j / 2.  f.lcount[s] counts every increment, so that a
// counter that wrapped shows as a total that does not match.
__device__ __forceinline__ void f3_lvl_add(Full3Smem &f, int slot, uint32_t n)
{
    atomicAdd(&f.lvl[slot >> 1], n << ((slot & 1) << 4));
}
__device__ __forceinline__ uint32_t f3_lvl_get(const Full3Smem &f, uint32_t slot)
{
    return (f.lvl[slot >> 1] >> ((slot & 1u) << 4)) & 0xffffu;
}
// Add every thread's count n to f.lcount[s] (one atomic per wave; all
// threads call).
__device__ __forceinline__ void f3_lcount(Full3Smem &f, int s, uint32_t n)
{
    for (int d = 32; d > 0; d >>= 1) n += __shfl_xor(n, d, 64);
    if (lane_id() == 0 && n) atomicAdd(&f.lcount[s], n);
}

// Wave64 inclusive scan of ParFn with DPP moves, without branches (the
// lower lane's value is always the left operand).
template <int CTRL>
__device__ __forceinline__ void f3_dpp_step(ParFn &v, bool take)
{
    ParFn o;
    o.f0 = dpp_mov<CTRL>(v.f0);
    o.f1 = dpp_mov<CTRL>(v.f1);
    const ParFn c = par_compose(o, v);
    v.f0 = take ? c.f0 : v.f0;
    v.f1 = take ? c.f1 : v.f1;
}
__device__ __forceinline__ ParFn f3_wave_scan(ParFn v)
{
    const int lane = lane_id(), rl = lane & 15;
    f3_dpp_step<0x111>(v, rl >= 1);      // row_shr:1
    f3_dpp_step<0x112>(v, rl >= 2);      // row_shr:2
    f3_dpp_step<0x114>(v, rl >= 4);      // row_shr:4
    f3_dpp_step<0x118>(v, rl >= 8);      // row_shr:8
    f3_dpp_step<0x142>(v, (lane & 31) >= 16);   // row_bcast:15
    f3_dpp_step<0x143>(v, lane >= 32);          // row_bcast:31
    return v;
}

// Stop conditions of a walk (monotone in the sum).  thr(e): the smallest
// sum P 2^(e-23) (P an integer, in units of the grid 2^(e-23)) for which
// the condition holds, as P, or at least 2^25 if it holds for none below
// 2^24 units.  A multiple of the grid with P < 2^24 is an exact float and
// v 2^(23-e) is exact (a power-of-two scaling), so P >= thr(e) is the
// condition itself.
struct F3Never {
    __device__ bool operator()(float) const { return false; }
    __device__ uint32_t thr(int) const { return kSat; }
};
struct F3AtLeast {      // cum >= v
    float v;
    __device__ bool operator()(float cc) const { return cc >= v; }
    __device__ uint32_t thr(int e) const
    {
        const float q = ceilf(ldexpf(v, 23 - e));
        return q < (float)kSat ? (uint32_t)fmaxf(q, 0.0f) : kSat;
    }
};
struct F3Above {        // v < cum
    float v;
    __device__ bool operator()(float cc) const { return v < cc; }
    __device__ uint32_t thr(int e) const
    {
        const float q = floorf(ldexpf(v, 23 - e)) + 1.0f;
        return q < (float)kSat ? (uint32_t)fmaxf(q, 0.0f) : kSat;
    }
};

// Exact sequential f32 adds cum = RN(cum + v[j]) over LDS values v[beg, end)
// on one wave (every lane calls with the same arguments), stopping at the
// first j after which pred(cum) holds (pred is monotone: the sums only
// grow).  256 values per step, four consecutive ones per lane: while the sum
// stays in one binade each add is an integer increment at its grid (elem_fn,
// a rounding tie as a function of the parity before it); a lane composes its
// four, a wave scan composes the lanes.  The first value whose add leaves
// the binade is added with the reference's own f32 add and the next step
// starts after it.  Returns j (or end); *cum_io receives the sum there (or
// at the end).
//
// The first nseq values are added one by one instead (every lane runs the
// same chain, reading broadcasts): the sum crosses binades often while it is
// small (at the head of the row), and each crossing would cost a step.
template <class P>
__device__ uint32_t f3_chain(const float *v, uint32_t beg, uint32_t end, float *cum_io, P pred, uint32_t nseq = 0)
{
    const int lane = lane_id();
    float cum = *cum_io;
    uint32_t j0 = beg;
    {
        // eight values per group; the next group's LDS reads are issued
        // before the current group's adds
        const uint32_t js = (beg & 3u) ? beg : beg + (min(end - beg, nseq) & ~7u);
        if (j0 < js) {
            float4 n0 = *reinterpret_cast<const float4 *>(v + j0), n1 = *reinterpret_cast<const float4 *>(v + j0 + 4);
            for (; j0 < js; j0 += 8u) {
                const float cur[8] = {n0.x, n0.y, n0.z, n0.w, n1.x, n1.y, n1.z, n1.w};
                if (j0 + 8u < js) {
                    n0 = *reinterpret_cast<const float4 *>(v + j0 + 8);
                    n1 = *reinterpret_cast<const float4 *>(v + j0 + 12);
                }
                float c[8];
                float x = cum;
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    x = x + cur[i];
                    c[i] = x;
                }
                if (pred(c[7])) {          // pred is monotone: the first of the 8 that holds
                    int i = 0;
                    while (!pred(c[i])) i++;
                    *cum_io = c[i];
                    return j0 + (uint32_t)i;
                }
                cum = c[7];
            }
            j0 = js;
        }
    }
    while (j0 < end) {
        const uint32_t jl = j0 + 4u * (uint32_t)lane;
        // this lane's live values: [jl, jl + nl); the reads past them stay
        // inside the workgroup's LDS and are replaced by 0
        const uint32_t nl = jl < end ? min(end - jl, 4u) : 0u;
        float a[4];
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const float x = v[jl + c];
            a[c] = (uint32_t)c < nl ? x : 0.0f;
        }
        const int e = grid_exp(cum);
        const uint32_t P0 = (uint32_t)ldexpf(cum, 23 - e);      // cum = P0 2^(e-23), P0 < 2^24
        // The common step (no rounding tie, no value of 2^22 grid units or
        // more) adds k = rint(a 2^(23-e)) per value whatever the parities:
        // an integer wave scan gives the sums.  Otherwise each value's
        // increment is a function of the parity before it (elem_fn) and the
        // functions are composed.
        uint32_t k[4];
        bool spec = false;
#pragma unroll
        for (int c = 0; c < 4; c++) {
            const float m = ldexpf(a[c], 23 - e);
            spec |= !(m < 4194304.0f) || m - floorf(m) == 0.5f;
            k[c] = (uint32_t)rintf(m);
        }
        uint32_t Pc[5];                                           // the sums before value c, and after the last
        if (!__any(spec)) {
            const uint32_t ks = k[0] + k[1] + k[2] + k[3];        // < 2^24: the scan stays below 2^30
            Pc[0] = P0 + (wave_incl_u32(ks) - ks);
#pragma unroll
            for (int c = 0; c < 4; c++) Pc[c + 1] = Pc[c] + k[c];
        } else {
            ParFn fc[4];
#pragma unroll
            for (int c = 0; c < 4; c++) fc[c] = elem_fn(a[c], e);
            ParFn loc = fc[0];
#pragma unroll
            for (int c = 1; c < 4; c++) loc = par_compose(loc, fc[c]);
            const ParFn incl = f3_wave_scan(loc);
            ParFn ex;
            ex.f0 = __shfl_up(incl.f0, 1, 64);
            ex.f1 = __shfl_up(incl.f1, 1, 64);
            if (lane == 0) ex = ParFn{0u, 0u};
            Pc[0] = P0 + par_apply(ex, P0 & 1u);
#pragma unroll
            for (int c = 0; c < 4; c++) Pc[c + 1] = Pc[c] + par_apply(fc[c], Pc[c] & 1u);
        }
        // per lane: the first live value whose add leaves the binade (a sum
        // of 2^24 grid units or more) or after which pred holds (a sum of
        // pred.thr(e) units or more; the sums only grow, so each event is a
        // threshold on the sums after the values)
        const uint32_t lim = min(pred.thr(e), 1u << 24);
        uint32_t cev = 0;
#pragma unroll
        for (int c = 1; c <= 4; c++) cev += Pc[c] < lim ? 1u : 0u;
        const bool ev = cev < nl;
        uint32_t Pb = Pc[0], Pa = Pc[1], Pl = Pc[0];
#pragma unroll
        for (int c = 1; c < 4; c++) {
            Pb = cev == (uint32_t)c ? Pc[c] : Pb;
            Pa = cev == (uint32_t)c ? Pc[c + 1] : Pa;
        }
#pragma unroll
        for (int c = 1; c <= 4; c++) Pl = nl == (uint32_t)c ? Pc[c] : Pl;
        const bool cross = Pa >= (1u << 24);
        const uint64_t bl = __ballot(ev && cross), bs = __ballot(ev && !cross);
        const int Ll = bl ? (int)__builtin_ctzll(bl) : 64;
        const int Ls = bs ? (int)__builtin_ctzll(bs) : 64;
        if (Ls < Ll) {
            const int c = __builtin_amdgcn_readlane((int)cev, Ls);
            *cum_io = ldexpf((float)(uint32_t)__builtin_amdgcn_readlane((int)Pa, Ls), e - 23);
            return j0 + 4u * (uint32_t)Ls + (uint32_t)c;
        }
        if (Ll == 64) {
            const int last = (int)min(end - j0, 256u) - 1;
            cum = ldexpf((float)(uint32_t)__builtin_amdgcn_readlane((int)Pl, last >> 2), e - 23);
            j0 += 256u;
            continue;
        }
        const int c = __builtin_amdgcn_readlane((int)cev, Ll);
        const uint32_t pb = (uint32_t)__builtin_amdgcn_readlane((int)Pb, Ll);
        const float before = pb >= (1u << 24) ? cum : ldexpf((float)pb, e - 23);
        const uint32_t p = j0 + 4u * (uint32_t)Ll + (uint32_t)c;
        const float after = before + v[p];
        if (pred(after)) {
            *cum_io = after;
            return p;
        }
        cum = after;
        j0 = p + 1u;
    }
    *cum_io = cum;
    return end;
}

// The sum after run r of table s, from the sum *c before it: the run's level
// total at its grid, and each rounding tie (table sorted by run, then k
// descending) to even from the parity before it.  False if *c is not in the
// run's binade or the sum leaves it.
__device__ bool f3_seg(const Full3Smem &f, int s, int r, float *c)
{
    const F3Run &R = f.run[s][r];
    const float c0 = *c;
    if (!(c0 > 0.0f) || grid_exp(c0) != R.e) return false;
    const uint64_t P0 = (uint64_t)ldexpf(c0, 23 - R.e);
    uint64_t extra = 0;
    const int nt = f.ntie[s];
    for (int i = 0; i < nt; i++) {
        const F3Tie T = f.tie[s][i];
        if (T.run != (uint32_t)r) continue;
        const uint64_t before = P0 + T.A + extra;
        extra += (uint64_t)T.k + ((before + T.k) & 1u);
    }
    const uint64_t P = P0 + f.rtot[s][r] + extra;
    if (P >= (1ull << 24)) return false;
    *c = ldexpf((float)P, R.e - 23);
    return true;
}

// The smallest of every thread's v (all threads call; one barrier).
__device__ __forceinline__ int f3_block_min(Full3Smem &f, uint32_t v)
{
    const uint32_t w = wave_min_u32(v);
    if (lane_id() == 0) f.wlast[wave_id()] = w;
    __syncthreads();
    uint32_t r = f.wlast[0];
#pragma unroll
    for (int i = 1; i < kWaves; i++) r = min(r, f.wlast[i]);
    return (int)r;
}

// Level totals of table s: rtot[r] = sum of k * count over run r, and for
// each tie, A = the same sum over its run's levels above it.  Then the ties
// are sorted by run, then k descending (one thread; at most kF3Ties).
__device__ void f3_totals(RowSmem &sm, Full3Smem &f, int s)
{
    const int t = threadIdx.x;
    const int nrun = f.nrun[s], nt = f.ntie[s];
    const uint32_t ltot = f.ltot[s];
    // (rtot[s] was cleared by the run planner, a tie's A when it was made)
    const uint32_t lb = s ? (uint32_t)kF3L23 : 0u;
    const uint32_t per = (ltot + kThreads - 1) / kThreads;
    const uint32_t j0 = lb + min((uint32_t)t * per, ltot), j1 = min(j0 + per, lb + ltot);
    uint32_t ncount = 0;
    if (j0 < j1) {
        int r = 0;
        while (r + 1 < nrun && f.run[s][r + 1].base <= j0) r++;
        uint64_t part = 0;
        for (uint32_t j = j0; j < j1; j++) {
            while (r + 1 < nrun && f.run[s][r + 1].base <= j) {
                if (part) atomicAdd((unsigned long long *)&f.rtot[s][r], (unsigned long long)part);
                part = 0;
                r++;
            }
            const uint32_t k = (uint32_t)((int)j - f.run[s][r].off);
            const uint32_t n = f3_lvl_get(f, j);
            part += (uint64_t)k * n;
            ncount += n;
        }
        if (part) atomicAdd((unsigned long long *)&f.rtot[s][r], (unsigned long long)part);
    }
    ncount = (uint32_t)__builtin_amdgcn_readlane((int)wave_incl_u32(ncount), 63);
    if (lane_id() == 0 && ncount) atomicSub(&f.lcount[s], ncount);
    for (int i = 0; i < nt; i++) {
        const F3Tie T = f.tie[s][i];
        const F3Run &R = f.run[s][T.run];
        const uint32_t a0 = max(j0, (uint32_t)(R.off + (int)T.k + 1)), a1 = min(j1, R.base + R.span);
        uint64_t part = 0;
        for (uint32_t j = a0; j < a1; j++) part += (uint64_t)((int)j - R.off) * f3_lvl_get(f, j);
        part = wave_sum_u64(part);
        if (lane_id() == 0 && part) atomicAdd((unsigned long long *)&f.tie[s][i].A, (unsigned long long)part);
    }
    __syncthreads();
    if (f.lcount[s] != 0u) f.fail = 1;    // a 16-bit counter wrapped
    if (nt < 2) return;
    // the ties ranked by (run, k descending, index), one per thread
    F3Tie mine;
    uint32_t rank = 0;
    if (t < nt) {
        mine = f.tie[s][t];
        for (int i = 0; i < nt; i++) {
            const F3Tie o = f.tie[s][i];
            rank += (o.run < mine.run || (o.run == mine.run && (o.k > mine.k || (o.k == mine.k && i < t)))) ? 1u : 0u;
        }
    }
    __syncthreads();
    if (t < nt) f.tie[s][rank] = mine;
    __syncthreads();
}

// Regions of a walk over bins [bH, kFBins): maximal stretches of bins with
// the same key (a run id, kF3KeyListed or kF3KeyNone).  False if more than
// kF3Regs.
template <class K>
__device__ bool f3_regions(RowSmem &sm, Full3Smem &f, int bH, const uint32_t *segst, K key)
{
    constexpr int kPer = kFBins / kThreads;
    const int t = threadIdx.x;
    uint32_t kk[kPer];
#pragma unroll
    for (int q = 0; q < kPer; q++) {
        const int b = kPer * t + q;
        kk[q] = b >= bH ? key(b) : kF3KeyNone;
    }
    uint32_t prev = __shfl_up(kk[kPer - 1], 1, 64);
    if (lane_id() == 63) f.wlast[wave_id()] = kk[kPer - 1];
    __syncthreads();
    if (lane_id() == 0) prev = wave_id() ? f.wlast[wave_id() - 1] : kF3KeyNone;
    uint32_t st[kPer], n = 0;
#pragma unroll
    for (int q = 0; q < kPer; q++) {
        const int b = kPer * t + q;
        const uint32_t pk = q ? kk[q - 1] : prev;
        st[q] = (b == bH || (b > bH && kk[q] != pk)) ? 1u : 0u;
        n += st[q];
    }
    uint32_t tot;
    uint32_t o = block_excl_u32(n, &tot, sm);
#pragma unroll
    for (int q = 0; q < kPer; q++) {
        if (st[q]) {
            if (o < (uint32_t)kF3Regs)
                f.reg[o] = F3Reg{(uint32_t)(kPer * t + q), kk[q],
                                 kk[q] == kF3KeyListed ? ldg(segst + kPer * t + q) : 0u};
            o++;
        }
    }
    if (t == 0) f.nreg = (int)tot;
    __syncthreads();
    return tot <= (uint32_t)kF3Regs;
}

// One walk on wave 0 (every lane calls): the head, then the regions.  The
// summands of the listed entries are staged in LDS (st): the head at
// [0, headend), position p of the regions' sorted list at roff + p.  A
// listed region spans list positions [segst[b0], cend(b1)); a run adds its
// totals (table s).  Stops at the first position after which pred holds (1:
// *arr = 0 in the head, 1 in the regions' list, *pos), or after the limit
// position (lim: 2), or at the end or at a kF3KeyNone region (0); -1 if a
// run's check fails or pred first holds inside a run.
template <class CE, class P>
__device__ int f3_walk(Full3Smem &f, const float *st, uint32_t roff, int s, const uint32_t *segst, CE cend, P pred,
                       bool lim, uint32_t lim_arr, uint32_t lim_pos, float *cum_out, uint32_t *arr, uint32_t *pos)
{
    float cum = 0.0f;
    {
        uint32_t end = f.headend;
        const bool at = lim && lim_arr == 0u;
        if (at) end = lim_pos + 1u;
        const uint32_t p = f3_chain(st, 0u, end, &cum, pred, 64u);
        if (s == 1) F3_TS(16 + 5 * s);
        *cum_out = cum;
        if (p < end) { *arr = 0u; *pos = p; return 1; }
        if (at) return 2;
    }
    const int nreg = f.nreg;
    for (int g = 0; g < nreg; g++) {
        const F3Reg R = f.reg[g];
        if (R.key == kF3KeyNone) break;
        if (R.key == kF3KeyListed) {
            const uint32_t b1 = g + 1 < nreg ? f.reg[g + 1].b0 - 1u : (uint32_t)kFBins - 1u;
            const uint32_t beg = R.beg;
            uint32_t end = cend(b1);
            const bool at = lim && lim_arr == 1u && lim_pos >= beg && lim_pos < end;
            if (at) end = lim_pos + 1u;
            const uint32_t p = f3_chain(st, roff + beg, roff + end, &cum, pred);
            if (s == 1) F3_TS(17 + 5 * s + min(g, 3));
            *cum_out = cum;
            if (p < roff + end) { *arr = 1u; *pos = p - roff; return 1; }
            if (at) return 2;
        } else {
            if (!f3_seg(f, s, (int)R.key, &cum)) return -1;
            *cum_out = cum;
            if (pred(cum)) return -1;
        }
#ifdef GS_TIMING
        {
            // the predicted sums' relative error at region ends (2^-30 units)
            const uint32_t b1 = g + 1 < nreg ? f.reg[g + 1].b0 : (uint32_t)kFBins;
            const double pr = roff == 0u ? (double)f.pre[b1] : (double)f.pre[b1] / (double)f.pre[kFBins];
            const double er = fabs((double)cum / pr - 1.0) * 1073741824.0;
            if (threadIdx.x == 0 && blockIdx.x < 1024 && pr > 0.0) {
                int &slot = g_v3diag[blockIdx.x * 32 + (roff == 0u ? 28 : 29)];
                slot = max(slot, (int)fmin(er, 2e9));
            }
        }
#endif
    }
    return 0;
}

// Table index of scaled logit y: bin b = floor(cb - y / w) at 1 + b, above
// the bins at 0, below at kFBins + 1.  One fma (cb + 1 - y / w, the same
// value in every pass), a clamp to [0, kFBins + 1] and a truncation, which
// is the floor there.  (The bins' edges as f3_range gives them carry a
// margin far above the rounding of this fma.)
__device__ __forceinline__ int f3_tidx(float y, float cb)
{
    const float tb = __builtin_amdgcn_fmed3f(fmaf(y, -kFInvW, cb + 1.0f), 0.0f, (float)(kFBins + 1));
    return (int)tb;
}
// The bin of y clamped to [0, kFBins) (for entries known to lie in a bin).
__device__ __forceinline__ int f3_bin(float y, float cb) { return min(max(f3_tidx(y, cb) - 1, 0), kFBins - 1); }
// A y-interval holding every element of bin b (the index is computed in f32;
// the margin covers its rounding).
__device__ __forceinline__ void f3_range(float cb, int b, float *ylo, float *yhi)
{
    const double iw = 1.0 / (double)kFInvW;
    const double hi = ((double)cb - b) * iw, lo = ((double)cb - b - 1) * iw;
    const double tol = 2e-5 + 4e-6 * fmax(fabs(hi), fabs(lo));
    *yhi = (float)(hi + tol);
    *ylo = (float)(lo - tol);
}

// Sort the entries [0, n) of a pass's list: entry j belongs to the segment
// of its bin ([0, nover) for the overflow entries) and goes to the segment's
// start plus its rank there (the number of greater entries: key descending,
// then index ascending).  sa gets its summand a = expf(y - m), 0 for an
// entry that left the list.  cend(b): the segment's end.
// Every position is checked to lie in [0, n) before it is read or written
// (a segment that the pass did not fill as planned fails the row instead).
template <class CE>
__device__ void f3_sort_list(Full3Smem &f, const uint64_t *lst, uint32_t n, uint32_t nover,
                             const uint32_t *segst, CE cend, uint64_t *se, float *sa, uint32_t *stage, uint32_t scap)
{
    // The last scap / 2 entries (the deep-tail window segments, which are
    // the large ones) are staged in LDS: a rank there costs one 64-bit
    // compare per entry of the segment.  Segments that start before them
    // rank from the list in global memory.
    uint64_t *stage64 = reinterpret_cast<uint64_t *>(stage);
    const uint32_t s0 = n > scap / 2u ? n - scap / 2u : 0u;
    for (uint32_t j = s0 + threadIdx.x; j < n; j += kThreads) stage64[j - s0] = ldg(lst + j);
    __syncthreads();
    for (uint32_t j = threadIdx.x; j < n; j += kThreads) {
        const uint64_t en = j >= s0 ? stage64[j - s0] : ldg(lst + j);
        const float y = f_entry_y(en);
        uint32_t st = 0, end = nover;
        if (j >= nover) {
            const int b = f3_tidx(y, f.cb) - 1;
            if (b < 0 || b >= kFBins) { f.fail = 1; continue; }
            st = ldg(segst + b);
            end = cend(b);
        }
        if (!(st <= j && j < end && end <= n)) { f.fail = 1; continue; }
        uint32_t rank = 0;
        uint32_t q = st;
        if (st >= s0) {
            const uint64_t *sg = stage64 - s0;
            for (; q + 8 <= end; q += 8) {
                uint64_t e8[8];
#pragma unroll
                for (int u = 0; u < 8; u++) e8[u] = sg[q + u];
#pragma unroll
                for (int u = 0; u < 8; u++) rank += e8[u] > en ? 1u : 0u;
            }
            for (; q < end; q++) rank += sg[q] > en ? 1u : 0u;
        } else {
            for (; q + 8 <= end; q += 8) {
                uint64_t e8[8];
#pragma unroll
                for (int u = 0; u < 8; u++) e8[u] = ldg(lst + q + u);
#pragma unroll
                for (int u = 0; u < 8; u++) rank += e8[u] > en ? 1u : 0u;
            }
            for (; q < end; q++) rank += ldg(lst + q) > en ? 1u : 0u;
        }
        if (st + rank >= end) { f.fail = 1; continue; }
        stg(se + st + rank, en);
        stg(sa + st + rank, f3_live(en) ? glibc_expf_tab(y - f.m, f.exptab) : 0.0f);
    }
}

// Increment of a summand x (exact, in grid units): an integer, or a rounding
// tie at floor(x) + 1/2.
__device__ __forceinline__ void f3_exact_k(float x, uint32_t *k, bool *tie)
{
    const float fl = floorf(x);
    *tie = (x - fl) == 0.5f;
    *k = *tie ? (uint32_t)fl : (uint32_t)rintf(x);
}
// Count an exactly known increment of run r (table s): a level, or a tie.
__device__ __forceinline__ void f3_count_exact(Full3Smem &f, int s, int r, float x)
{
    if ((uint32_t)r >= (uint32_t)f.nrun[s]) { f.fail = 1; return; }
    uint32_t k;
    bool tie;
    f3_exact_k(x, &k, &tie);
    const F3Run &R = f.run[s][r];
    if (tie) {
        const int i = atomicAdd(&f.ntie[s], 1);
        if (i < kF3Ties) f.tie[s][i] = F3Tie{(uint32_t)r, k, 0ull};
        return;
    }
    if (k == 0u) return;
    if (k - R.klo >= R.span) { f.fail = 1; return; }
    f3_lvl_add(f, R.off + (int)k, 1u);
    atomicAdd(&f.lcount[s], 1u);
}

// Plan of one accumulation's runs over bins [bH, kFBins).  Per bin (kPer per
// thread, from the caller): key[q] = grid exponent + 256 for a bin of a run,
// kF3KeyListed or kF3KeyNone; KL[b] / KH[b] (LDS, by bin) its level range,
// read at the runs' ends only.  Writes the run
// table s (runs numbered in bin order; level slots from lbase) and rid[q]
// (the bin's run, or -1).  False if there are more than kF3Runs runs or
// their levels exceed lcap.
__device__ bool f3_plan_runs(RowSmem &sm, Full3Smem &f, int s, int bH, const uint32_t *key, const uint32_t *KL,
                             const uint32_t *KH, int *rid, uint32_t lbase, uint32_t lcap)
{
    constexpr int kPer = kFBins / kThreads;
    const int t = threadIdx.x;
    // the neighbouring threads' edge keys (through the free top of lvl)
    uint32_t *kx = f.lvl + 2 * kFBins;
    kx[kPer * t] = key[0];
    kx[kPer * t + kPer - 1] = key[kPer - 1];
    __syncthreads();
    const uint32_t prev = t ? kx[kPer * t - 1] : kF3KeyNone;
    const uint32_t nxt = t + 1 < kThreads ? kx[kPer * t + kPer] : kF3KeyNone;
    uint32_t st[kPer], n = 0;
#pragma unroll
    for (int q = 0; q < kPer; q++) {
        const int b = kPer * t + q;
        const uint32_t pk = q ? key[q - 1] : prev;
        const bool in = b >= bH && key[q] < 512u;
        st[q] = in && (b == bH || pk != key[q]) ? 1u : 0u;
        n += st[q];
    }
    uint32_t tot;
    uint32_t o = block_excl_u32(n, &tot, sm);
    if (s == 1) F3_TS(19);
    if (tot > (uint32_t)kF3Runs) return false;
    int cur = (int)o - 1;
#pragma unroll
    for (int q = 0; q < kPer; q++) {
        const int b = kPer * t + q;
        const bool in = b >= bH && key[q] < 512u;
        if (st[q]) {
            cur++;
            f.run[s][cur].e = (int)key[q] - 256;
            f.run[s][cur].khi = KH[b];
        }
        rid[q] = in ? cur : -1;
        const uint32_t nk = q + 1 < kPer ? key[q + 1] : nxt;
        if (in && (b == kFBins - 1 || nk != key[q])) f.run[s][cur].klo = KL[b];
    }
    __syncthreads();
    if (s == 1) F3_TS(20);
    if (t < 64) {
        uint32_t span = 0;
        if (t < (int)tot) {
            F3Run &R = f.run[s][t];
            span = R.khi >= R.klo ? R.khi - R.klo + 1u : 0u;
            if (span > lcap) span = lcap + 1u;
        }
        uint32_t incl = span;
        for (int d = 1; d < 64; d <<= 1) {
            const uint32_t v = __shfl_up(incl, d, 64);
            if (t >= d) incl += v;
        }
        if (t < (int)tot) {
            F3Run &R = f.run[s][t];
            R.base = lbase + incl - span;
            R.span = span;
            R.off = (int)R.base - (int)R.klo;
        }
        // (the role words hold off + 2^23 in 24 bits)
        const bool big = t < (int)tot && f.run[s][t].klo > (1u << 22);
        if (t == 63) { f.nrun[s] = (int)tot; f.ltot[s] = incl; }
        f.rtot[s][t] = 0ull;
        if (__any(big) && lane_id() == 0) f.ltot[s] = lcap + 1u;
    }
    __syncthreads();
    return f.ltot[s] <= lcap;
}


// The increment every element of a bin adds when its exact summands, in
// grid units, lie in [xl, xh] (up to the bin edges' rounding): the one
// integer that [xl, xh] widened by 2^-15 rounds to, or kF3NoU.
constexpr uint32_t kF3NoU = 0xffffffffu;
__device__ __forceinline__ uint32_t f3_uniform(double xl, double xh)
{
    const double kl = floor(xl * (1.0 - 1.0 / 32768.0) + 0.5), kh = floor(xh * (1.0 + 1.0 / 32768.0) + 0.5);
    return kl == kh && kl < 1073741824.0 ? (uint32_t)kl : kF3NoU;
}

// Pass 2's step for one element from its role word w (table index idx):
// the seq-1 increment k = rint(a~ 2^sh) and its level slot, or a listed or
// ambiguous element (rare).  The same code serves the batched pass and the
// single visits (penalized ids, unaligned ends), so both classify alike.
__device__ __forceinline__ float f3_exp(float d) { return __builtin_amdgcn_exp2f(d * 1.44269504f); }
struct F3K { int slot; bool ok, rare; };
__device__ __forceinline__ F3K f3_k1(uint32_t w, float y, float m)
{
    const float x = ldexpf(f3_exp(y - m), (int)((w >> 24) & 63u));
    const float k = rintf(x);
    const bool amb = fabsf(x - k) >= fmaf(-x, kF3Band1, 0.5f);
    const bool in = (w & kF3In2) != 0u;
    F3K r;
    r.slot = (int)(w & kF3Cur) - (1 << 23) + (int)k;
    r.ok = in && !amb && (uint32_t)r.slot < (uint32_t)kF3H;
    r.rare = (w & kF3Listed) || (in && !r.ok);
    return r;
}
// Pass 3's step: seq 2 (w.x) and seq 3 (w.y, the increment over the range
// of s2: [cS3lo, cS3hi] scale a / (S s2)).
struct F3K23 { int slot2, slot3; bool ok2, ok3, rare; };
__device__ __forceinline__ F3K23 f3_k23(uint2 w, float y, float m, float cS, float cS3lo, float band3)
{
    const float a = f3_exp(y - m);
    F3K23 r;
    {
        const float x = ldexpf(a * cS, (int)((w.x >> 24) & 63u));
        const float k = rintf(x);
        const bool amb = fabsf(x - k) >= fmaf(-x, kF3Band23, 0.5f);
        r.slot2 = (int)(w.x & kF3Cur) - (1 << 23) + (int)k;
        r.ok2 = (w.x & kF3In2) && !amb && (uint32_t)r.slot2 < (uint32_t)kF3H;
    }
    {
        // x over the range of s2 lies in [x0, x0 (1 + band3 - kF3Band23)]
        const float x0 = ldexpf(a * cS3lo, (int)((w.y >> 24) & 63u));
        const float k = rintf(x0);
        const bool amb = fabsf(x0 - k) >= fmaf(-x0, band3, 0.5f);
        r.slot3 = (int)(w.y & kF3Cur) - (1 << 23) + (int)k;
        r.ok3 = (w.y & kF3W3) && !amb && (uint32_t)r.slot3 < (uint32_t)kF3H;
    }
    r.rare = (w.x & kF3Listed) || ((w.x & kF3In2) && !r.ok2) || ((w.y & kF3W3) && !r.ok3);
    return r;
}

// A pass over the row with the elements that need work compacted per wave.
// A wave takes the row in chunks of 64 kUnroll float4s (*ctr: the next free
// chunk); each lane holds 4 kUnroll elements of a chunk; their role words are
// read together (word), those that ask for work (act) are
// appended to the wave's ring in LDS (q, QN entries of (y, index)), and each
// time 64 have gathered every lane of the wave processes one (work).  An
// element of a bin without work costs its bin lookup only.  The 0-3 elements
// before the 16-byte boundary and the ragged end go to work directly.
template <int QN, bool NT, class YF, class WORD, class ACT, class WORK>
__device__ __forceinline__ void f3_qpass(const float *row, int V, YF yf, WORD word, ACT act, WORK work, uint2 *q,
                                         uint32_t *ctr)
{
    static_assert(QN >= 128 && (QN & (QN - 1)) == 0, "ring");
    const int t = threadIdx.x, lane = lane_id();
    const int h0 = min(V, (int)(((16u - ((uint32_t)reinterpret_cast<uintptr_t>(row) & 15u)) & 15u) >> 2));
    const float4 *r4 = reinterpret_cast<const float4 *>(row + h0);
    const int n4 = (V - h0) >> 2;
    constexpr int kE = 4 * kUnroll;
    uint32_t qh = 0, qt = 0;
#ifdef GS_TIMING
    uint64_t c_work = 0, n_fl = 0;
    const uint64_t c_beg = clock64();
#endif
    // Chunks of kCh float4s, one wave's round: wave w takes chunks w and
    // kWaves + w, then the next free one from *ctr (2 kWaves before the
    // pass), so waves that the SIMDs issue more often take more chunks and
    // the pass ends when the work does, not when the least favoured wave
    // finishes an equal share.  Each wave's chunk numbers only grow.  The
    // next chunk's loads are in flight while this one's words are looked up
    // and its active elements processed.
    constexpr int kCh = 64 * kUnroll;
    const int nch = (n4 + kCh - 1) / kCh;
    auto grab = [&]() {
        uint32_t c = 0u;
        if (lane == 0) c = atomicAdd(ctr, 1u);
        return __builtin_amdgcn_readfirstlane((int)c);
    };
    float4 nv[kUnroll];
    auto load = [&](int c) {
#pragma unroll
        for (int u = 0; u < kUnroll; u++) {
            const float4 *pa = r4 + min(c * kCh + u * 64 + lane, n4 - 1);
            nv[u] = NT ? ldg_nt(pa) : ldg(pa);
        }
    };
    int cur = wave_id(), nxt = kWaves + wave_id();
    if (cur < nch) load(cur);
    while (cur < nch) {
        float4 v[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; u++) v[u] = nv[u];
        if (nxt < nch) load(nxt);
        const int nn = grab();
        const int base = cur * kCh + lane;
        float y[kE];
#pragma unroll
        for (int u = 0; u < kUnroll; u++) {
            const bool in = base + u * 64 < n4;
            y[4 * u + 0] = in ? yf(v[u].x) : -INFINITY;
            y[4 * u + 1] = in ? yf(v[u].y) : -INFINITY;
            y[4 * u + 2] = in ? yf(v[u].z) : -INFINITY;
            y[4 * u + 3] = in ? yf(v[u].w) : -INFINITY;
        }
        decltype(word(0.0f)) w[kE];
#pragma unroll
        for (int e = 0; e < kE; e++) w[e] = word(y[e]);
#pragma unroll
        for (int e = 0; e < kE; e++) {
            const bool a = act(w[e]);
            const uint64_t bm = __ballot(a);
            if (bm) {
                const uint32_t off =
                    __builtin_amdgcn_mbcnt_hi((uint32_t)(bm >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bm, 0u));
                if (a)
                    q[(qt + off) & (QN - 1)] =
                        make_uint2(__float_as_uint(y[e]), (uint32_t)(h0 + 4 * (base + (e >> 2) * 64) + (e & 3)));
                qt += (uint32_t)__popcll(bm);
                if (qt - qh >= 64u) {
                    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                    __builtin_amdgcn_wave_barrier();
                    const uint2 it = q[(qh + (uint32_t)lane) & (QN - 1)];
#ifdef GS_TIMING
                    const uint64_t c0 = clock64();
#endif
                    work((int)it.y, __uint_as_float(it.x));
#ifdef GS_TIMING
                    c_work += clock64() - c0;
                    n_fl++;
#endif
                    qh += 64u;
                    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                    __builtin_amdgcn_wave_barrier();
                }
            }
        }
        cur = nxt;
        nxt = nn;
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    if ((uint32_t)lane < qt - qh) {
        const uint2 it = q[(qh + (uint32_t)lane) & (QN - 1)];
        work((int)it.y, __uint_as_float(it.x));
    }
    if (t < h0) work(t, yf(ldg(row + t)));
    for (int i = h0 + (n4 << 2) + t; i < V; i += kThreads) work(i, yf(ldg(row + i)));
#ifdef GS_TIMING
    const int sb = QN == 256 ? 20 : 23;
    F3_STAT(sb, (clock64() - c_beg) / 100);
    F3_STAT(sb + 1, c_work / 100);
    F3_STAT(sb + 2, n_fl);
    if (lane == 0 && blockIdx.x < 1024) {
        atomicMax(&g_v3diag[blockIdx.x * 32 + (QN == 256 ? 16 : 17)], (int)((clock64() - c_beg) / 100));
        atomicMax(&g_v3diag[blockIdx.x * 32 + (QN == 256 ? 18 : 19)], (int)n_fl);
    }
#endif
}

// The exact full-vocabulary path, increment-histogram form.  Returns true
// with *tok / *status set, or false to hand the row to the next path.
// `gl` is the row's scratch (lcap u64 words).
__device__ bool full_v3_row(RowSmem &sm, const float *row, int V, float T, float top_p, bool has_pen, float r,
                            uint64_t *gl, size_t lcap, int *tok, int *status)
{
    Full3Smem &f = sm.x.f3;
    const int t = threadIdx.x;
    constexpr int kPer = kFBins / kThreads;
    static_assert(kPer * kThreads == kFBins, "bins per thread");
    const bool t_one = (T == 1.0f);
    const bool nuc = top_p < 1.0f;
    // scratch: list | sorted list of pass 2 | of pass 3 | their summands |
    // ambiguous | deferred | segment starts | roles of seqs 2, 3
    const size_t cap = f3_list_cap((size_t)V);
    if (lcap < f3_scratch_u64((size_t)V)) F3_FAIL();
    uint64_t *lst = gl;
    uint64_t *se1 = lst + cap;
    uint64_t *se3 = se1 + cap;
    float *sa1 = reinterpret_cast<float *>(se3 + cap);
    float *sa3 = sa1 + cap;
    uint64_t *amb = reinterpret_cast<uint64_t *>(sa3 + cap);
    uint64_t *def = amb + kF3AmbCap;
    uint32_t *segst = reinterpret_cast<uint32_t *>(def + kF3DefCap);
    uint32_t *role = segst + kFBins;
    float *stg_lds = reinterpret_cast<float *>(f.lvl);     // walks: staged summands
    const int h0 = (int)(((16u - ((uint32_t)reinterpret_cast<uintptr_t>(row) & 15u)) & 15u) >> 2);
    const float4 *r4 = reinterpret_cast<const float4 *>(row + h0);
    const int n4 = (V - h0) >> 2;
    if (V < h0 || n4 == 0) F3_FAIL();
    auto ydiv = [&](float x) { return t_one ? x : x / T; };
    auto pen_y = [&](int s) { return ydiv(__uint_as_float(sm.hval[s])); };

    for (int b = t; b < kF3Tab; b += kThreads) f.w[b] = 0u;
    for (int b = t; b < kFBins; b += kThreads) f.cnt[b] = 0u;
    for (int b = t; b < kFMassBins; b += kThreads) f.u.mass64[b] = 0ull;
    if (t < 32) f.exptab[t] = kExp2Tab[t];
    if (t == 0) {
        f.nover = 0; f.fail = 0; f.namb = 0; f.ndef = 0; f.ntie[0] = 0; f.ntie[1] = 0;
        f.qctr[0] = f.qctr[1] = 2u * kWaves;
    }

    // ---- pass 1 (HBM): counts, masses of the top bins, max, NaN -------------
    // Bins are of t = cb - y / w, cb = (m0 + 3) / w, m0 the maximum of the
    // first round of loads: bin b = floor(t) in [0, kFBins); t < 0 (elements
    // more than 3 above m0) go to the overflow list, t >= kFBins (more than
    // 18.5 below) add 0 to every sum.
    float tmax = -INFINITY;
    int nan = 0;
    float m0 = 0.0f, cb = 0.0f;
    auto visit1 = [&](int i, float y) {
        nan |= (int)isnan(y);
        if (y > tmax && !(has_pen && hash_find(sm, (uint32_t)i) >= 0)) tmax = y;
        const int ix = f3_tidx(y, cb);
        if (ix == 0) {
            const int slot = atomicAdd(&f.nover, 1);
            if (slot < kFOverCap) f.over[slot] = f_entry(y, (uint32_t)i);
        } else if (ix <= kFBins) {
            const int b = ix - 1;
            atomicAdd(&f.cnt[b], 1u);
            if (b < kFMassBins)
                atomicAdd((unsigned long long *)&f.u.mass64[b], (unsigned long long)(fast_exp(y - m0) * kFMassScale));
        }
    };
    auto pass1 = [&](auto yf) -> bool {
#ifdef GS_TIMING
        const uint64_t c_beg = clock64();
#endif
        float4 nv[kUnroll];
#pragma unroll
        for (int u = 0; u < kUnroll; u++) nv[u] = ldg(r4 + min(u * kThreads + t, n4 - 1));
        for (int base = 0; base < n4; base += kThreads * kUnroll) {
            float4 v[kUnroll];
#pragma unroll
            for (int u = 0; u < kUnroll; u++) v[u] = nv[u];
            if (base + kThreads * kUnroll < n4) {
#pragma unroll
                for (int u = 0; u < kUnroll; u++) nv[u] = ldg(r4 + min(base + kThreads * kUnroll + u * kThreads + t, n4 - 1));
            }
            if (base == 0) {
                float lm = -INFINITY;
#pragma unroll
                for (int u = 0; u < kUnroll; u++)
                    if (u * kThreads + t < n4) lm = fmaxf(lm, fmaxf(fmaxf(v[u].x, v[u].y), fmaxf(v[u].z, v[u].w)));
                m0 = ydiv(f_block_max(lm, sm));
                if (!isfinite(m0)) return false;
                cb = (float)(((double)m0 + (double)kFDUp) * (double)kFInvW);
#ifdef GS_TIMING
                F3_STAT(26, (clock64() - c_beg) / 100);
#endif
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
#ifdef GS_TIMING
        F3_STAT(27, (clock64() - c_beg) / 100);
#endif
        return true;
    };
    if (!(t_one ? pass1([](float x) { return x; }) : pass1([&](float x) { return x / T; }))) F3_FAIL();
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
    if (!isfinite(m) || m0 > m || f.nover > kFOverCap) F3_FAIL();
    if (t == 0) { f.m = m; f.m0 = m0; f.cb = cb; }
    F3_TS(0);

    // ---- penalty: the raw values of penalized ids leave the counts, their
    // penalized values join (w counts the raw values per bin: the list
    // segments must hold room for them) -------------------------------------
    if (has_pen) {
        for (int j = t; j < f.nover; j += kThreads)
            if (hash_find(sm, f_entry_id(f.over[j])) >= 0) f.over[j] = 0ull;
        __syncthreads();
        for (int s = t; s < kHashSlots; s += kThreads) {
            const uint32_t id = sm.hkey[s];
            if (id == kEmpty) continue;
            const float yr = ydiv(ldg(row + id));
            const int ir = f3_tidx(yr, cb);
            if (ir >= 1 && ir <= kFBins) {
                const int b = ir - 1;
                atomicSub(&f.cnt[b], 1u);
                atomicAdd(&f.w[b], 1u);
                if (b < kFMassBins)
                    atomicAdd((unsigned long long *)&f.u.mass64[b], 0ull - (unsigned long long)(fast_exp(yr - m0) * kFMassScale));
            }
            const float yp = pen_y(s);
            const int ip = f3_tidx(yp, cb);
            if (ip == 0) {
                const int slot = atomicAdd(&f.nover, 1);
                if (slot < kFOverCap) f.over[slot] = f_entry(yp, id);
            } else if (ip <= kFBins) {
                const int b = ip - 1;
                atomicAdd(&f.cnt[b], 1u);
                if (b < kFMassBins)
                    atomicAdd((unsigned long long *)&f.u.mass64[b], (unsigned long long)(fast_exp(yp - m0) * kFMassScale));
            }
        }
        __syncthreads();
        if (f.nover > kFOverCap) F3_FAIL();
    }
    const int nover = f.nover;
    const double iw = 1.0 / (double)kFInvW;
    // exp(y - m) at bin position bpos (the centre of bin b at b + 0.5)
    auto e_at = [&](double bpos) { return (double)f3_exp((float)(((double)cb - bpos) * iw - (double)m)); };
    const double dl = 1.0 - kFDelta, dh = 1.0 + kFDelta;

    // ---- plan A: the running seq-1 sum before each bin, predicted from the
    // masses (top bins) and, for the rest, the counts times the mean rounded
    // increment over the bin's range of summands (as if the summands were
    // spread evenly over it), refined once ---------------------------------
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
        double mb[kPer], ed[kPer + 1];      // ed[q]: the summand at bin kPer t + q's upper edge
        const double mscale = exp((double)m0 - (double)m) / (double)kFMassScale;
        double loc = 0.0;
#pragma unroll
        for (int q = 0; q <= kPer; q++) ed[q] = e_at((double)(kPer * t + q));
#pragma unroll
        for (int q = 0; q < kPer; q++) {
            const int b = kPer * t + q;
            cn[q] = f.cnt[b];
            mb[q] = b < kFMassBins ? (double)(int64_t)f.u.mass64[b] * mscale : (double)cn[q] * 0.5 * (ed[q] + ed[q + 1]);
            if (mb[q] < 0.0) mb[q] = 0.0;
            loc += mb[q];
        }
        double tot;
        double pre = f_block_excl_f64_buf(loc, &tot, sm.red_f64b) + osum;
        // one refinement: a second one (with the refined sums' grids) left
        // the largest error of the predicted sums at the region ends, and
        // the rows that take this path, unchanged on C3 and C4
        double ct[kPer];
        {
            double lo = pre;
            loc = 0.0;
#pragma unroll
            for (int q = 0; q < kPer; q++) {
                const int b = kPer * t + q;
                ct[q] = mb[q];
                if (b >= kFMassBins && cn[q] && lo > 0.0) {
                    // the mean of rint(u) over u in [ul, uh] (the bin's summands in
                    // units of the grid 2^ge): (F(uh) - F(ul)) / (uh - ul) with
                    // F(u) = (u^2 - (u - rint u)^2) / 2
                    const int ge = f_dexp(lo) - 23;
                    const double uh = ldexp(ed[q], -ge), ul = ldexp(ed[q + 1], -ge);
                    const double sh = uh - rint(uh), sl = ul - rint(ul);
                    const double mean = uh > ul ? 0.5 * (uh + ul) - 0.5 * (sh * sh - sl * sl) / (uh - ul) : rint(uh);
                    ct[q] = (double)cn[q] * ldexp(mean, ge);
                }
                lo += ct[q];
                loc += ct[q];
            }
            pre = f_block_excl_f64_buf(loc, &tot, sm.red_f64) + osum;
        }
        double lo = pre;
#pragma unroll
        for (int q = 0; q < kPer; q++) {
            f.pre[kPer * t + q] = (float)lo;
            lo += ct[q];
        }
        if (t == kThreads - 1) f.pre[kFBins] = (float)lo;
    }
    for (int j = t; j < nover; j += kThreads) stg(lst + j, f.over[j]);
    __syncthreads();
    F3_TS(1);

    // ---- seq-1 roles: windows (the sum may change binade in the bin), the
    // level range of every other bin, and the head: the smallest bH whose
    // runs' levels below fit kF3L1 ------------------------------------------
    int bmax = -1;    // the bin of the maximum (the head holds it)
    {
        const int im = f3_tidx(m, cb);
        if (im >= 1) bmax = min(im - 1, kFBins - 1);
    }
    {
        uint32_t key[kPer], klo[kPer], khi[kPer], c[kPer], ku[kPer];
#pragma unroll
        for (int q = 0; q < kPer; q++) {
            const int b = kPer * t + q;
            const double lo = (double)f.pre[b], hi = (double)f.pre[b + 1];
            const bool win = !(lo > 0.0) || f_dexp(lo * dl) != f_dexp(hi * dh);
            const int e = lo > 0.0 ? f_dexp(lo) : 0;
            key[q] = win ? kF3KeyListed : (uint32_t)(e + 256);
            klo[q] = 1u;
            khi[q] = 0u;
            ku[q] = kF3NoU;
            if (!win) {
                float ylo, yhi;
                f3_range(cb, b, &ylo, &yhi);
                const double sc = ldexp(1.0, 23 - e);
                const double xl = (double)f3_exp(ylo - m) * sc;      // (within 2^-18.5: the margins hold it)
                const double xh = (double)f3_exp(yhi - m) * sc;
                klo[q] = (uint32_t)fmin(floor(xl * kF3Lo), 1073741824.0);
                khi[q] = (uint32_t)fmin(floor(xh * kF3Hi + 0.5), 1073741824.0);
                ku[q] = f3_uniform(xl, xh);
            }
            f.lvl[b] = key[q];
            f.lvl[kFBins + b] = khi[q];
            reinterpret_cast<uint32_t *>(f.u.w23)[b] = klo[q];
        }
        __syncthreads();
        // level slots a bin adds to its run, counted from the bottom of the
        // run (telescoping: the run's total is its top bin's khi minus its
        // bottom bin's klo, plus one)
        uint32_t ssum = 0;
#pragma unroll
        for (int q = 0; q < kPer; q++) {
            const int b = kPer * t + q;
            c[q] = 0u;
            if (key[q] != kF3KeyListed) {
                const bool same = b + 1 < kFBins && f.lvl[b + 1] == key[q];
                const uint32_t below = same ? f.lvl[kFBins + b + 1] + 1u : klo[q];
                c[q] = khi[q] + 1u > below ? min(khi[q] + 1u - below, 262144u) : 0u;
            }
            ssum += c[q];
        }
        F3_TS(26);
        uint32_t call;
        const uint32_t sp = block_excl_u32(ssum, &call, sm);
        uint32_t run_pre = sp, cand = kFBins;
#pragma unroll
        for (int q = 0; q < kPer; q++) {
            const int b = kPer * t + q;
            if (cand == (uint32_t)kFBins && b > bmax && b >= 1 && call - run_pre <= (uint32_t)kF3L1) cand = (uint32_t)b;
            run_pre += c[q];
        }
        const int bH = f3_block_min(f, cand);
        if (bH >= kFBins) F3_FAIL();
        // runs of seq 1 and the role words; listed bins (the head and the
        // windows) get list segments (room for the raw values of penalized
        // ids too)
#pragma unroll
        for (int q = 0; q < kPer; q++) if (kPer * t + q < bH) key[q] = kF3KeyListed;
        int rid[kPer];
        F3_TS(27);
        if (!f3_plan_runs(sm, f, 0, bH, key, reinterpret_cast<const uint32_t *>(f.u.w23), f.lvl + kFBins, rid, 0u,
                          (uint32_t)kF3L1))
            F3_FAIL();
        F3_TS(28);
        uint32_t capv[kPer], capl = 0;
#pragma unroll
        for (int q = 0; q < kPer; q++) {
            const int b = kPer * t + q;
            capv[q] = key[q] == kF3KeyListed ? f.cnt[b] + f.w[b] : 0u;
            capl += capv[q];
        }
        uint32_t ltot;
        uint32_t o = block_excl_u32(capl, &ltot, sm) + (uint32_t)nover;   // (its barriers: w read)
        uint32_t wv[kPer];
#pragma unroll
        for (int q = 0; q < kPer; q++) {
            const int b = kPer * t + q;
            wv[q] = 0u;
            if (key[q] == kF3KeyListed) {
                wv[q] = kF3Listed | o;
                stg(segst + b, o);
            } else if (khi[q] >= 1u && ku[q] == kF3NoU) {
                const F3Run &R = f.run[0][rid[q]];
                wv[q] = kF3In2 | ((uint32_t)(23 - R.e) << 24) | (uint32_t)(R.off + (1 << 23));
            }
            // the walk's key of the bin (kF3KeyNone: below the bins the sum uses)
            stg(role + b, b < bH || key[q] == kF3KeyListed ? kF3KeyListed : (uint32_t)rid[q]);
            if (b == bH) f.headend = o;
            o += capv[q];
        }
        __syncthreads();
#pragma unroll
        for (int q = 0; q < kPer; q++) f.w[1 + kPer * t + q] = wv[q];
        if (t == 0) {
            f.w[0] = 0u;
            f.w[kFBins + 1] = 0u;
            f.list_end = (uint32_t)nover + ltot;
            f.bH = bH;
            f.lcount[0] = 0u;
        }
        for (int j = t; j <= kF3Lvl; j += kThreads) f.lvl[j] = 0u;
        __syncthreads();
        // uniform bins: every element adds ku (the count is exact)
        uint32_t nadd = 0;
#pragma unroll
        for (int q = 0; q < kPer; q++) {
            const int b = kPer * t + q;
            if (key[q] != kF3KeyListed && ku[q] != kF3NoU && ku[q] != 0u && f.cnt[b]) {
                const F3Run &R = f.run[0][rid[q]];
                if (ku[q] - R.klo < R.span && f.cnt[b] < 65536u) {
                    f3_lvl_add(f, R.off + (int)ku[q], f.cnt[b]);
                    nadd += f.cnt[b];
                } else {
                    f.fail = 1;
                }
            }
        }
        f3_lcount(f, 0, nadd);
        __syncthreads();
        if (f.list_end > cap || f.fail) F3_FAIL();
    }
    const int bH = f.bH;
    F3_STAT(1, bH);
    F3_STAT(2, f.headend);
    F3_STAT(3, f.list_end);
    F3_STAT(5, f.nrun[0]);
    F3_STAT(6, f.ltot[0]);
    F3_TS(2);

    // ---- pass 2 (cache): seq-1 levels; listed bins written ------------------
    {
        uint32_t nok = 0;      // level increments of this thread
        auto word = [&](float y) { return f.w[f3_tidx(y, cb)]; };
        auto common = [&](uint32_t w, float y) {
            const F3K k = f3_k1(w, y, m);
            if (k.ok) f3_lvl_add(f, k.slot, 1u);
            nok += k.ok ? 1u : 0u;
            return k.rare;
        };
        // the raw values of penalized ids are not set aside (their penalized
        // values are visited after the pass); listed ones take their slot,
        // marked dead
        bool pen_raw = has_pen;
        auto rare = [&](int i, float y, uint32_t w) {
            if (w & kF3Listed) {
                const uint32_t slot = atomicAdd(&f.w[f3_tidx(y, cb)], 1u) & kF3Cur;
                const uint64_t en = f_entry(y, (uint32_t)i);
                stg(lst + slot, pen_raw && hash_find(sm, (uint32_t)i) >= 0 ? f3_dead(en) : en);
            } else {
                if (pen_raw && hash_find(sm, (uint32_t)i) >= 0) return;
                const uint32_t s = atomicAdd((uint32_t *)&f.namb, 1u);
                if (s < kF3AmbCap) stg(amb + s, f_entry(y, (uint32_t)i));
            }
        };
        auto one = [&](int i, float y) {
            const uint32_t w = word(y);
            if (common(w, y)) rare(i, y, w);
        };
        auto act = [](uint32_t w) { return w != 0u; };
        uint2 *ring = reinterpret_cast<uint2 *>(f.u.w23) + 256 * wave_id();
        if (t_one) f3_qpass<256, false>(row, V, [](float x) { return x; }, word, act, one, ring, &f.qctr[0]);
        else f3_qpass<256, false>(row, V, [&](float x) { return x / T; }, word, act, one, ring, &f.qctr[0]);
        __syncthreads();
        if (has_pen) {
            // the raw values of penalized ids leave (the pass marked their
            // listed entries and set none aside; their levels are uncounted
            // here), then the penalized values are visited
            for (int s = t; s < kHashSlots; s += kThreads) {
                const uint32_t id = sm.hkey[s];
                if (id == kEmpty) continue;
                const float y = ydiv(ldg(row + id));
                const int ix = f3_tidx(y, cb);
                const uint32_t w = f.w[ix];
                if (w & kF3Listed) continue;
                const F3K k = f3_k1(w, y, m);
                if (k.ok) {
                    f3_lvl_add(f, k.slot, 0xffffffffu);
                    nok--;
                }
            }
            __threadfence_block();
            __syncthreads();
            pen_raw = false;
            for (int s = t; s < kHashSlots; s += kThreads)
                if (sm.hkey[s] != kEmpty) one((int)sm.hkey[s], pen_y(s));
            __threadfence_block();
            __syncthreads();
        }
        f3_lcount(f, 0, nok);
    }
    F3_STAT(4, f.namb);
    if (f.fail || (uint32_t)f.namb > kF3AmbCap) F3_FAIL();
    F3_TS(3);
    // ambiguous elements: exact increments
    {
        const uint32_t na = (uint32_t)f.namb;
        for (uint32_t j = t; j < na; j += kThreads) {
            const uint64_t en = ldg(amb + j);
            if (!f3_live(en)) continue;
            const float y = f_entry_y(en);
            const int run = (int)ldg(role + f3_bin(y, cb));
            f3_count_exact(f, 0, run, ldexpf(glibc_expf_tab(y - m, f.exptab), 23 - f.run[0][run].e));
        }
    }
    __threadfence_block();
    __syncthreads();
    f3_sort_list(f, lst, f.list_end, (uint32_t)nover, segst, [&](int b) { return f.w[1 + b] & kF3Cur; }, se1, sa1,
                 reinterpret_cast<uint32_t *>(f.u.w23), 2u * kF3Tab);
    __threadfence_block();
    __syncthreads();
    if (f.fail || f.ntie[0] > kF3Ties) F3_FAIL();
    F3_TS(4);

    // ---- walk S (src/sampler.rs:54) ----------------------------------------
    f3_totals(sm, f, 0);
    F3_TS(29);
    {
        const uint32_t n = f.list_end;
        if (n > (uint32_t)kF3Lvl) F3_FAIL();
        for (uint32_t j = t; j < n; j += kThreads) stg_lds[j] = ldg(sa1 + j);
    }
    if (!f3_regions(sm, f, bH, segst, [&](int b) { return ldg(role + b); })) F3_FAIL();
    F3_TS(30);
    if (wave_id() == 0) {
        float S;
        uint32_t arr, pos;
        const int res = f3_walk(f, stg_lds, 0u, 0, segst, [&](uint32_t b) { return f.w[1 + b] & kF3Cur; },
                                F3Never{}, false, 0u, 0u, &S, &arr, &pos);
        if (lane_id() == 0) { f.S = S; f.walk_res = res; }
    }
    __syncthreads();
    const float S = f.S;
    F3_STAT(30, __float_as_int(S));
    F3_STAT(31, __float_as_int(f.pre[kFBins]));
    if (f.walk_res != 0 || !(S > 0.0f) || !isfinite(S)) F3_FAIL();
    F3_TS(5);

    // ---- plan B (seqs 2, 3): predicted sums from the seq-1 prediction
    // normalised by its total; the cut and the draw windows; runs ----------
    float cS = 0.0f, cS3lo = 0.0f, band3 = 0.0f;
    {
        const double iP = 1.0 / (double)f.pre[kFBins];
        const double iS = 1.0 / (double)S;
        const double tp = (double)top_p, rd = (double)r;
        if (nuc && tp * dh >= 1.0) F3_FAIL();           // the cut may not happen
        if (!nuc && rd >= dl) F3_FAIL();                 // the draw may not happen
        // s2 lies in [top_p, top_p + the cut element's summand + a rounding
        // step]: the summand is at most the first cut-window bin's largest
        // (or 1/S if the cut may lie in the head)
        uint32_t cand = kFBins;
        if (nuc) {
#pragma unroll
            for (int q = 0; q < kPer; q++) {
                const int b = kPer * t + q;
                if (cand == (uint32_t)kFBins && b >= bH && (double)f.pre[b + 1] * iP * dh >= tp) cand = (uint32_t)b;
            }
        }
        const int bcut = f3_block_min(f, cand);     // the first bin the cut may lie in
        double s2lo = 1.0, s2hi = 1.0;
        if (nuc) {
            const int bc = bcut;
            double vmax = iS;
            if (bc > bH && bc < kFBins) {
                float ylo, yhi;
                f3_range(cb, bc, &ylo, &yhi);
                vmax = (double)glibc_expf_tab(yhi - m, f.exptab) * iS * 1.001;
            }
            s2lo = (double)top_p;
            s2hi = (double)__double2float_ru(tp + vmax + ldexp(tp, -22));
        }
        cS = (float)iS;
        cS3lo = __double2float_rd(iS / s2hi);
        band3 = (float)((double)kF3Band23 * 2.0 + (s2hi / s2lo - 1.0));
        __syncthreads();
        const double is2hi = 1.0 / s2hi, is2lo = 1.0 / s2lo;
        // the bins' level ranges go to LDS (free here: the top of lvl holds
        // the run planner's keys), the rest stays in registers
        uint32_t *KL2 = reinterpret_cast<uint32_t *>(f.u.w23), *KL3 = KL2 + kFBins;
        uint32_t *KH2 = f.lvl, *KH3 = f.lvl + kFBins;
        uint32_t key2[kPer], key3[kPer], rl[kPer], ku2[kPer], ku3[kPer], hk = 0u;
#pragma unroll
        for (int q = 0; q < kPer; q++) {
            const int b = kPer * t + q;
            const double lo2 = (double)f.pre[b] * iP, hi2 = (double)f.pre[b + 1] * iP;
            key2[q] = key3[q] = kF3KeyNone;
            ku2[q] = ku3[q] = kF3NoU;
            rl[q] = 0u;
            if (b < bH) continue;
            const bool past = nuc && lo2 * dl >= tp;
            if (past) continue;
            const bool cw = nuc && hi2 * dh >= tp;
            float ylo, yhi;
            f3_range(cb, b, &ylo, &yhi);
            const double pl = (double)f3_exp(ylo - m) * iS;
            const double ph = (double)f3_exp(yhi - m) * iS;
            const double plo = pl * kF3Lo, phi = ph * kF3Hi;
            if (nuc) {
                if (cw || !(lo2 > 0.0) || f_dexp(lo2 * dl) != f_dexp(hi2 * dh)) {
                    key2[q] = kF3KeyListed;
                    rl[q] |= kF3L2Bit;
                } else {
                    const int e2 = f_dexp(lo2);
                    key2[q] = (uint32_t)(e2 + 256);
                    const double sc = ldexp(1.0, 23 - e2);
                    KL2[b] = (uint32_t)fmin(floor(plo * sc), 1073741824.0);
                    const uint32_t kh = (uint32_t)fmin(floor(phi * sc + 0.5), 1073741824.0);
                    KH2[b] = kh;
                    hk |= kh >= 1u ? 1u << q : 0u;
                    ku2[q] = f3_uniform(pl * sc, ph * sc);
                }
            }
            // (reciprocals: the bounds below hold margins far above an ulp)
            const double c3lo = lo2 * is2hi, c3hi = hi2 * is2lo;
            if (c3lo * dl > rd) continue;
            if (cw || !(c3lo > 0.0) || c3hi * dh > rd || f_dexp(c3lo * dl) != f_dexp(c3hi * dh)) {
                key3[q] = kF3KeyListed;
                rl[q] |= kF3L3Bit;
            } else {
                const int e3 = f_dexp(c3lo);
                key3[q] = (uint32_t)(e3 + 256);
                const double sc = ldexp(1.0, 23 - e3);
                KL3[b] = (uint32_t)fmin(floor(plo * is2hi * sc), 1073741824.0);
                const uint32_t kh = (uint32_t)fmin(floor(phi * is2lo * sc + 0.5), 1073741824.0);
                KH3[b] = kh;
                hk |= kh >= 1u ? 16u << q : 0u;
                ku3[q] = f3_uniform(pl * is2hi * sc, ph * is2lo * sc);
            }
        }
        F3_TS(31);
        int rid2[kPer], rid3[kPer];
        if (!f3_plan_runs(sm, f, 0, bH, key2, KL2, KH2, rid2, 0u, (uint32_t)kF3L23)) F3_FAIL();
        F3_TS(16);
        if (!f3_plan_runs(sm, f, 1, bH, key3, KL3, KH3, rid3, (uint32_t)kF3L23, (uint32_t)kF3L23)) F3_FAIL();
        F3_TS(17);
        // list segments of pass 3: the bins listed for seq 2 or 3 (room for
        // the raw values of penalized ids: counted in lvl, free until pass 3)
        for (int b = t; b < kFBins; b += kThreads) f.lvl[b] = 0u;
        __syncthreads();
        if (has_pen) {
            for (int s = t; s < kHashSlots; s += kThreads) {
                const uint32_t id = sm.hkey[s];
                if (id == kEmpty) continue;
                const int ir = f3_tidx(ydiv(ldg(row + id)), cb);
                if (ir >= 1 && ir <= kFBins) atomicAdd(&f.lvl[ir - 1], 1u);
            }
            __syncthreads();
        }
        uint32_t capv[kPer], capl = 0;
#pragma unroll
        for (int q = 0; q < kPer; q++) {
            const int b = kPer * t + q;
            capv[q] = rl[q] ? f.cnt[b] + f.lvl[b] : 0u;
            capl += capv[q];
        }
        uint32_t ltot;
        uint32_t o = block_excl_u32(capl, &ltot, sm);
        uint2 wv[kPer];
#pragma unroll
        for (int q = 0; q < kPer; q++) {
            const int b = kPer * t + q;
            uint32_t rw = rl[q];
            if (rid2[q] >= 0) rw |= kF3In2 | ((uint32_t)rid2[q] << 8);
            if (rid3[q] >= 0) rw |= kF3In3 | (uint32_t)rid3[q];
            stg(role + b, rw);
            wv[q] = make_uint2(0u, 0u);
            if (rl[q]) {
                wv[q].x = kF3Listed | o;
                stg(segst + b, o);
            } else {
                if (rid2[q] >= 0 && ((hk >> q) & 1u) && ku2[q] == kF3NoU) {
                    const F3Run &R = f.run[0][rid2[q]];
                    wv[q].x = kF3In2 | ((uint32_t)(23 - R.e) << 24) | (uint32_t)(R.off + (1 << 23));
                }
                if (rid3[q] >= 0 && ((hk >> (4 + q)) & 1u) && ku3[q] == kF3NoU) {
                    const F3Run &R = f.run[1][rid3[q]];
                    wv[q].y = kF3W3 | ((uint32_t)(23 - R.e) << 24) | (uint32_t)(R.off + (1 << 23));
                }
            }
            o += capv[q];
        }
        __syncthreads();
#pragma unroll
        for (int q = 0; q < kPer; q++) f.u.w23[1 + kPer * t + q] = wv[q];
        if (t == 0) {
            f.u.w23[0] = make_uint2(0u, 0u);
            f.u.w23[kFBins + 1] = make_uint2(0u, 0u);
            f.list_end = ltot;
            f.s2lo = (float)s2lo;
            f.s2hi = (float)s2hi;
            f.ntie[0] = 0;
            f.ntie[1] = 0;
            f.namb = 0;
            f.ndef = 0;
            f.lcount[0] = 0u;
            f.lcount[1] = 0u;
        }
        for (int j = t; j <= kF3Lvl; j += kThreads) f.lvl[j] = 0u;
        __syncthreads();
        F3_TS(18);
        // uniform bins of the runs (not listed): every element adds ku
        uint32_t nadd2 = 0, nadd3 = 0;
#pragma unroll
        for (int q = 0; q < kPer; q++) {
            const int b = kPer * t + q;
            if (rl[q] || !f.cnt[b]) continue;
            if (rid2[q] >= 0 && ku2[q] != kF3NoU && ku2[q] != 0u) {
                const F3Run &R = f.run[0][rid2[q]];
                if (ku2[q] - R.klo < R.span && f.cnt[b] < 65536u) {
                    f3_lvl_add(f, R.off + (int)ku2[q], f.cnt[b]);
                    nadd2 += f.cnt[b];
                } else {
                    f.fail = 1;
                }
            }
            if (rid3[q] >= 0 && ku3[q] != kF3NoU && ku3[q] != 0u) {
                const F3Run &R = f.run[1][rid3[q]];
                if (ku3[q] - R.klo < R.span && f.cnt[b] < 65536u) {
                    f3_lvl_add(f, R.off + (int)ku3[q], f.cnt[b]);
                    nadd3 += f.cnt[b];
                } else {
                    f.fail = 1;
                }
            }
        }
        f3_lcount(f, 0, nadd2);
        f3_lcount(f, 1, nadd3);
        __syncthreads();
        if (ltot > (uint32_t)cap || f.fail) F3_FAIL();
    }
    F3_TS(6);

    // ---- pass 3 (cache): seq-2 and seq-3 levels above the cut; bins listed,
    // ambiguous seq-2 and undecided seq-3 elements set aside -----------------
    {
        uint32_t nok2 = 0, nok3 = 0;
        auto word = [&](float y) { return f.u.w23[f3_tidx(y, cb)]; };
        auto common = [&](uint2 w, float y) {
            const F3K23 k = f3_k23(w, y, m, cS, cS3lo, band3);
            if (k.ok2) f3_lvl_add(f, k.slot2, 1u);
            if (k.ok3) f3_lvl_add(f, k.slot3, 1u);
            nok2 += k.ok2 ? 1u : 0u;
            nok3 += k.ok3 ? 1u : 0u;
            return k.rare;
        };
        bool pen_raw = has_pen;      // (as in pass 2)
        auto rare = [&](int i, float y, uint2 w) {
            const uint64_t en = f_entry(y, (uint32_t)i);
            const bool raw = pen_raw && hash_find(sm, (uint32_t)i) >= 0;
            if (w.x & kF3Listed) {
                const uint32_t slot = atomicAdd(&f.u.w23[f3_tidx(y, cb)].x, 1u) & kF3Cur;
                stg(lst + slot, raw ? f3_dead(en) : en);
                return;
            }
            if (raw) return;
            const F3K23 k = f3_k23(w, y, m, cS, cS3lo, band3);
            if ((w.x & kF3In2) && !k.ok2) {
                const uint32_t s = atomicAdd((uint32_t *)&f.namb, 1u);
                if (s < kF3AmbCap) stg(amb + s, en);
            }
            if ((w.y & kF3W3) && !k.ok3) {
                const uint32_t s = atomicAdd((uint32_t *)&f.ndef, 1u);
                if (s < kF3DefCap) stg(def + s, en);
            }
        };
        auto one = [&](int i, float y) {
            const uint2 w = word(y);
            if (common(w, y)) rare(i, y, w);
        };
        auto act = [](uint2 w) { return (w.x | w.y) != 0u; };
        uint2 *ring = reinterpret_cast<uint2 *>(f.pre) + 128 * wave_id();
        if (t_one) f3_qpass<128, true>(row, V, [](float x) { return x; }, word, act, one, ring, &f.qctr[1]);
        else f3_qpass<128, true>(row, V, [&](float x) { return x / T; }, word, act, one, ring, &f.qctr[1]);
        __syncthreads();
        F3_TS(10);
        if (has_pen) {
            for (int s = t; s < kHashSlots; s += kThreads) {
                const uint32_t id = sm.hkey[s];
                if (id == kEmpty) continue;
                const float y = ydiv(ldg(row + id));
                const int ix = f3_tidx(y, cb);
                const uint2 w = f.u.w23[ix];
                if (w.x & kF3Listed) continue;
                const F3K23 k = f3_k23(w, y, m, cS, cS3lo, band3);
                if (k.ok2) {
                    f3_lvl_add(f, k.slot2, 0xffffffffu);
                    nok2--;
                }
                if (k.ok3) {
                    f3_lvl_add(f, k.slot3, 0xffffffffu);
                    nok3--;
                }
            }
            __threadfence_block();
            __syncthreads();
            pen_raw = false;
            for (int s = t; s < kHashSlots; s += kThreads)
                if (sm.hkey[s] != kEmpty) one((int)sm.hkey[s], pen_y(s));
            __threadfence_block();
            __syncthreads();
        }
        f3_lcount(f, 0, nok2);
        f3_lcount(f, 1, nok3);
        F3_STAT(7, f.list_end);
        F3_STAT(8, f.ndef);
        F3_STAT(9, f.namb);
        F3_STAT(10, f.nrun[0]);
        F3_STAT(11, f.nrun[1]);
        F3_STAT(12, f.ltot[0]);
        F3_STAT(13, f.ltot[1]);
        if (f.fail || (uint32_t)f.namb > kF3AmbCap || (uint32_t)f.ndef > kF3DefCap) F3_FAIL();
        f3_sort_list(f, lst, f.list_end, 0u, segst, [&](int b) { return f.u.w23[1 + b].x & kF3Cur; }, se3, sa3,
                     reinterpret_cast<uint32_t *>(f.pre), (uint32_t)kFBins + 1u);
        F3_TS(11);
        // seq 2: exact increments of the ambiguous elements and of the listed
        // elements of bins listed for seq 3 only
        const uint32_t na = (uint32_t)f.namb;
        for (uint32_t j = t; j < na; j += kThreads) {
            const uint64_t en = ldg(amb + j);
            if (!f3_live(en)) continue;
            const float y = f_entry_y(en);
            const int rr = (int)((ldg(role + f3_bin(y, cb)) >> 8) & 63u);
            const float p = glibc_expf_tab(y - m, f.exptab) / S;
            f3_count_exact(f, 0, rr, ldexpf(p, 23 - f.run[0][rr].e));
        }
        __threadfence_block();
        __syncthreads();
        if (nuc) {
            for (uint32_t j = t; j < f.list_end; j += kThreads) {
                const uint64_t en = ldg(se3 + j);
                if (!f3_live(en)) continue;
                const uint32_t rw = ldg(role + f3_bin(f_entry_y(en), cb));
                if (!(rw & kF3In2)) continue;
                const int rr = (int)((rw >> 8) & 63u);
                const float p = ldg(sa3 + j) / S;
                f3_count_exact(f, 0, rr, ldexpf(p, 23 - f.run[0][rr].e));
            }
        }
        __syncthreads();
        if (f.fail || f.ntie[0] > kF3Ties) F3_FAIL();
    }
    F3_TS(7);

    // ---- walk 2: the cut and s2 (src/sampler.rs:59-67) ---------------------
    float s2 = 1.0f;
    uint32_t cut_arr = 0u, cut_pos = 0u;
    const uint32_t headend = f.headend, nl3 = f.list_end;
    auto cend3 = [&](uint32_t b) { return f.u.w23[1 + b].x & kF3Cur; };
    if (nuc) {
        // the summands of seq 2 are staged in cnt and w (free since plan B
        // and walk S; contiguous), the seq-3 levels stay in lvl
        float *stg2 = reinterpret_cast<float *>(f.cnt);
        if (headend + nl3 > (uint32_t)(kFBins + kF3Tab)) F3_FAIL();
        f3_totals(sm, f, 0);
        F3_TS(12);
        for (uint32_t j = t; j < headend; j += kThreads) stg2[j] = ldg(sa1 + j) / S;
        for (uint32_t j = t; j < nl3; j += kThreads) stg2[headend + j] = ldg(sa3 + j) / S;
        if (!f3_regions(sm, f, bH, segst, [&](int b) {
                const uint32_t rw = ldg(role + b);
                return (rw & kF3L2Bit) ? kF3KeyListed : (rw & kF3In2) ? ((rw >> 8) & 63u) : kF3KeyNone;
            }))
            F3_FAIL();
        F3_TS(13);
        if (wave_id() == 0) {
            float c;
            uint32_t arr = 0u, pos = 0u;
            const int res = f3_walk(f, stg2, headend, 0, segst, cend3, F3AtLeast{top_p},
                                    false, 0u, 0u, &c, &arr, &pos);
            if (lane_id() == 0) { f.s2 = c; f.walk_res = res; f.cut_arr = arr; f.cut_pos = pos; }
        }
        __syncthreads();
        F3_STAT(14, f.walk_res);
        F3_STAT(15, f.nreg);
        if (f.walk_res != 1) F3_FAIL();
        s2 = f.s2;
        cut_arr = f.cut_arr;
        cut_pos = f.cut_pos;
        // the cut must not lie inside a run of seq 3 (walk 3 stops there)
        if (cut_arr == 1u ? cut_pos >= nl3 : cut_pos >= headend) F3_FAIL();
        if (cut_arr == 1u) {
            const uint64_t en = ldg(se3 + cut_pos);
            if (ldg(role + f3_bin(f_entry_y(en), cb)) & kF3In3) F3_FAIL();
        }
        if (!(s2 >= f.s2lo && s2 <= f.s2hi)) F3_FAIL();
    }
    F3_TS(8);

    // ---- walk 3: the draw (src/sampler.rs:71-78) ----------------------------
    {
        auto qv = [&](float a) { const float p = a / S; return nuc ? p / s2 : p; };
        const uint32_t nd = (uint32_t)f.ndef;
        for (uint32_t j = t; j < nd; j += kThreads) {
            const uint64_t en = ldg(def + j);
            if (!f3_live(en)) continue;
            const float y = f_entry_y(en);
            const int rr = (int)(ldg(role + f3_bin(y, cb)) & 63u);
            f3_count_exact(f, 1, rr, ldexpf(qv(glibc_expf_tab(y - m, f.exptab)), 23 - f.run[1][rr].e));
        }
        for (uint32_t j = t; j < nl3; j += kThreads) {
            const uint64_t en = ldg(se3 + j);
            if (!f3_live(en)) continue;
            const uint32_t rw = ldg(role + f3_bin(f_entry_y(en), cb));
            if (!(rw & kF3In3)) continue;
            const int rr = (int)(rw & 63u);
            f3_count_exact(f, 1, rr, ldexpf(qv(ldg(sa3 + j)), 23 - f.run[1][rr].e));
        }
        __threadfence_block();
        __syncthreads();
        if (f.fail || f.ntie[1] > kF3Ties) F3_FAIL();
        F3_TS(14);
        f3_totals(sm, f, 1);
        if (headend + nl3 > (uint32_t)kF3Lvl) F3_FAIL();
        for (uint32_t j = t; j < headend; j += kThreads) stg_lds[j] = qv(ldg(sa1 + j));
        for (uint32_t j = t; j < nl3; j += kThreads) stg_lds[headend + j] = qv(ldg(sa3 + j));
        if (!f3_regions(sm, f, bH, segst, [&](int b) {
                const uint32_t rw = ldg(role + b);
                return (rw & kF3L3Bit) ? kF3KeyListed : (rw & kF3In3) ? (rw & 63u) : kF3KeyNone;
            }))
            F3_FAIL();
        F3_TS(15);
        if (wave_id() == 0) {
            float c;
            uint32_t arr = 0u, pos = 0u;
            const int res = f3_walk(f, stg_lds, headend, 1, segst, cend3, F3Above{r}, nuc,
                                    cut_arr, cut_pos, &c, &arr, &pos);
            if (lane_id() == 0) {
                f.walk_res = res;
                f.tok_arr = res == 2 ? cut_arr : arr;
                f.tok_pos = res == 2 ? cut_pos : pos;
            }
        }
        __syncthreads();
        if (f.walk_res != 1 && f.walk_res != 2) F3_FAIL();
        if (f.tok_arr ? f.tok_pos >= nl3 : f.tok_pos >= headend) F3_FAIL();
        const uint64_t en = ldg((f.tok_arr ? se3 : se1) + f.tok_pos);
        if (!f3_live(en)) F3_FAIL();
        *tok = (int)f_entry_id(en);
    }
    F3_TS(9);
    return true;
}
