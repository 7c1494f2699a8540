// gs_gemv.hip -- gfx950 quantized matrix-vector product that produces the
// logits (the reference's output projection, src/model/llama.rs:333-334 on
// the GPU path, :405-407 on the CPU path), for Q4_0, Q4_1, Q8_0, Q3_K, Q4_K,
// Q5_K and Q6_K weights.
//
// HBM-bound: every weight byte is read once per call and nothing else of
// size moves.  Device layout (rearranged at upload from the GGUF blocks, the
// same 210 / 34 bytes per block as the file), chosen so that every load
// instruction of a wave reads one contiguous run of memory:
//   Q6_K: three planes of 16-byte chunks, one chunk per quarter block and
//         plane (ql[64h + l0 ..], ql[64h + 32 + l0 ..], qh[32h + l0 ..] for
//         quarter (h, l0), see below), indexed row * 4nb + quarter; a plane of
//         32-bit words, the quarter's four int8 scales; the f16 d per block.
//   Q8_0: 16-byte chunks of int8 quants, row * 2nb + half block; f16 d per block.
// Weight loads are non-temporal (each byte is used once).
//
// One wave per row, rows strided over all waves of the grid.  A lane takes a
// fixed slice of the columns (Q6_K: a quarter block, 64 weights = 16 values
// of l in one half of a block; Q8_0: half blocks of 16 weights), so its slice
// of x stays in registers for every row the wave visits (when a row fits in
// one pass of the wave, cols <= 4096), with the sums of x over its 16-weight
// groups.  Weights are decoded four to a 32-bit word and converted with the
// byte-to-float instructions; the offset of the stored values (Q6_K q + 32,
// Q8_0 q + 128 after flipping the sign bit) is taken out once per group:
// sum (u - o) x = sum u x - o * sum x.  The next row's loads are issued
// before the current row is computed.
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>
#include <new>

#include "../../include/gs_gemv.h"
#include "../../include/gs_sampler.h"

namespace gs {

constexpr int kGemvThreads = 256;       // 4 waves per workgroup
constexpr int kMaxCols = 16384;         // x staged in LDS (64 KB) on the general path

__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

// Streaming loads of the weights (read once per call: non-temporal).
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint4 ntl4(const void *p)
{
    const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t *>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 ntl2(const void *p)
{
    const u32x2_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t *>(p));
    return make_uint2(v.x, v.y);
}

__device__ __forceinline__ float wave_sum(float v)
{
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) v += __shfl_xor(v, d, 64);
    return v;
}

// Row sums of kRB rows at once (kRB = 4, 8 or 16): each lane's partial of
// row k is written to the wave's LDS tile t[k][lane]; lane L then adds the
// 64 kRB / 64 partials t[L % kRB][..] of its share, and log2(64 / kRB)
// shuffles combine the shares.  Lanes 0 .. kRB-1 return the sums of rows
// 0 .. kRB-1.
template <int kRB>
__device__ __forceinline__ float rows_sum(float (&part)[kRB], float *t)
{
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int k = 0; k < kRB; k++) t[k * 64 + lane] = part[k];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    constexpr int kC = 64 / kRB;           // lanes per row, 64 / kC partials each
    const float4 *q = reinterpret_cast<const float4 *>(t + (lane % kRB) * 64 + (64 / kC) * (lane / kRB));
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 16 / kC; i++) {
        const float4 v = q[i];
        s += (v.x + v.y) + (v.z + v.w);
    }
#pragma unroll
    for (int d = kRB; d < 64; d <<= 1) s += __shfl_xor(s, d, 64);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();       // the tile is free for the next batch
    return s;
}

// Bytes 0..3 of a word as floats (v_cvt_f32_ubyte0..3).
__device__ __forceinline__ float ub(uint32_t w, int t) { return (float)((w >> (8 * t)) & 0xffu); }

// ---------------------------------------------------------------- Q6_K -----
// Quarter qi of a row: block j = qi / 4, half h = (qi / 2) % 2, l0 = 16 (qi % 2).
// Its 64 weights sit at 256 j + 128 h + 32 g + l, g = 0..3, l = l0 .. l0 + 15
// (src/tensor/dequant.rs:203-214): group g takes the low nibble of
// ql[64h + l] (g 0) / ql[64h + 32 + l] (g 1), the high nibbles (g 2, 3), and
// bits 2g..2g+1 of qh[32h + l]; its scale is sc[8h + l0/16 + 2g].
struct Q6Quarter {
    uint4 a, b, c;      // ql[64h + l0 ..], ql[64h + 32 + l0 ..], qh[32h + l0 ..]
    uint32_t s;         // byte g: sc[8h + l0/16 + 2g]
    uint16_t d;
};

// Planes of a Q6_K matrix on the device (see the layout above); e indexes
// quarters (row * 4nb + quarter), blocks are e / 4.
struct Q6Planes {
    const uint8_t *a, *b, *c;
    const uint32_t *s;
    const uint16_t *d;
};

// e < 2^28 (the upload limits a plane to 4 GB): 32-bit offsets from the
// wave-uniform plane bases.
__device__ __forceinline__ Q6Quarter q6_load(const Q6Planes &P, uint32_t e)
{
    Q6Quarter q;
    q.a = ntl4(P.a + e * 16u);
    q.b = ntl4(P.b + e * 16u);
    q.c = ntl4(P.c + e * 16u);
    q.s = __builtin_nontemporal_load(P.s + e);
    q.d = __builtin_nontemporal_load(P.d + (e >> 2));
    return q;
}

// sum over the quarter's four groups of scale_g * sum (u - 32) x.
// xg[g][i] = x at the group's i-th weight, sx[g] = sum of xg[g].
__device__ __forceinline__ float q6_dot(const Q6Quarter &q, const float (&xg)[4][16], const float (&sx)[4])
{
    float dot[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    const uint32_t A[4] = {q.a.x, q.a.y, q.a.z, q.a.w};
    const uint32_t B[4] = {q.b.x, q.b.y, q.b.z, q.b.w};
    const uint32_t C[4] = {q.c.x, q.c.y, q.c.z, q.c.w};
#pragma unroll
    for (int w = 0; w < 4; w++) {
        const uint32_t a = A[w], b = B[w], c = C[w];
        const uint32_t u[4] = {(a & 0x0F0F0F0Fu) | ((c & 0x03030303u) << 4),
                               (b & 0x0F0F0F0Fu) | ((c & 0x0C0C0C0Cu) << 2),
                               ((a >> 4) & 0x0F0F0F0Fu) | (c & 0x30303030u),
                               ((b >> 4) & 0x0F0F0F0Fu) | ((c >> 2) & 0x30303030u)};
#pragma unroll
        for (int g = 0; g < 4; g++)
#pragma unroll
            for (int t = 0; t < 4; t++) dot[g] = fmaf(ub(u[g], t), xg[g][4 * w + t], dot[g]);
    }
    const float d = h2f(q.d);
    float acc = 0.0f;
#pragma unroll
    for (int g = 0; g < 4; g++) {
        const float scl = d * (float)(int8_t)(uint8_t)(q.s >> (8 * g));   // (d * scale), as the reference
        acc = fmaf(scl, fmaf(-32.0f, sx[g], dot[g]), acc);
    }
    return acc;
}

__device__ __forceinline__ void q6_xslice(const float *x, int j, int h, int l0, float (&xg)[4][16], float (&sx)[4])
{
#pragma unroll
    for (int g = 0; g < 4; g++) {
        const float4 *p = reinterpret_cast<const float4 *>(x + 256 * j + 128 * h + 32 * g + l0);
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float4 v = p[i];
            xg[g][4 * i] = v.x; xg[g][4 * i + 1] = v.y; xg[g][4 * i + 2] = v.z; xg[g][4 * i + 3] = v.w;
        }
#pragma unroll
        for (int i = 0; i < 16; i++) s += xg[g][i];
        sx[g] = s;
    }
}

// A block format whose lanes take quarters: 64 weights of block j at
// 256 j + 128 h + 32 g + l0 + (0..15), g = 0..3 (Q6_K, Q3_K).
struct Q6Fmt {
    typedef Q6Planes Planes;
    typedef Q6Quarter Unit;
    static __device__ __forceinline__ Unit load(const Planes &P, uint32_t e) { return q6_load(P, e); }
    static __device__ __forceinline__ float dot(const Unit &u, const float (&xg)[4][16], const float (&sx)[4])
    {
        return q6_dot(u, xg, sx);
    }
};

// Rows of up to 16 blocks (cols <= 4096): one quarter per lane, x in
// registers.  One NT-thread workgroup per CU stages x in LDS once; each wave
// then takes a contiguous run of rows and keeps the loads of the next PF rows
// in flight while it computes one (PF divides kRB, so the ring of row
// buffers is indexed statically).
template <class F, int kRB, int PF, int NT>
__device__ __forceinline__ void quarter_rows_xreg(const typename F::Planes &P, const float *x, float *out, int rows,
                                                  int nb, float *xs, float (*tiles)[kRB * 64])
{
    static_assert(kRB % PF == 0, "ring of PF row buffers, kRB rows per batch");
    const int cols = 256 * nb;
    for (int i = threadIdx.x; i < cols; i += NT) xs[i] = x[i];
    __syncthreads();
    const int lane = threadIdx.x & 63;
    const int nw = gridDim.x * (NT / 64);
    const int gw = blockIdx.x * (NT / 64) + (threadIdx.x >> 6);
    const int NQ = 4 * nb;
    const bool act = lane < NQ;
    const int qi = act ? lane : 0;
    const int j = qi >> 2, h = (qi >> 1) & 1, l0 = (qi & 1) * 16;
    float xg[4][16], sx[4];
    q6_xslice(xs, j, h, l0, xg, sx);
    const int rpw = (rows + nw - 1) / nw;
    const int r0 = gw * rpw, r1 = min(rows, r0 + rpw);
    if (r0 >= r1) return;
    float *tile = tiles[threadIdx.x >> 6];
    const uint32_t e1 = (uint32_t)(r1 - 1) * NQ + qi;
    auto row_e = [&](int r) { return min((uint32_t)r * NQ + qi, e1); };   // past the run: its last row
    typename F::Unit buf[PF];
#pragma unroll
    for (int i = 0; i < PF; i++) buf[i] = F::load(P, row_e(r0 + i));
    int rb = r0;
    for (; rb + kRB <= r1; rb += kRB) {        // full batches
        float part[kRB];
#pragma unroll
        for (int k = 0; k < kRB; k++) {
            const typename F::Unit nxt = F::load(P, row_e(rb + k + PF));
            part[k] = act ? F::dot(buf[k % PF], xg, sx) : 0.0f;
            buf[k % PF] = nxt;
        }
        const float v = rows_sum<kRB>(part, tile);
        if (lane < kRB) out[rb + lane] = v;
    }
    if (rb < r1) {                             // the last, partial batch
        float part[kRB];
#pragma unroll
        for (int k = 0; k < kRB; k++) {
            part[k] = 0.0f;
            if (rb + k < r1 && act) part[k] = F::dot(buf[k % PF], xg, sx);   // rows rb .. r1-1 are in the ring
            if (k + 1 < kRB && (k + 1) % PF == 0 && rb + k + 1 < r1) {
#pragma unroll
                for (int i = 0; i < PF; i++) buf[i] = F::load(P, row_e(rb + k + 1 + i));
            }
        }
        const float v = rows_sum<kRB>(part, tile);
        if (lane < kRB && rb + lane < r1) out[rb + lane] = v;
    }
}
template <int kRB, int PF, int NT>
__global__ void __launch_bounds__(NT)
q6k_gemv_xreg(Q6Planes P, const float *x, float *out, int rows, int nb)
{
    __shared__ float xs[4096];
    __shared__ float tiles[NT / 64][kRB * 64];
    quarter_rows_xreg<Q6Fmt, kRB, PF, NT>(P, x, out, rows, nb, xs, tiles);
}

// Any row length up to kMaxCols: x staged in LDS, lanes loop over quarters.
template <class F>
__device__ __forceinline__ void quarter_rows_lds(const typename F::Planes &P, const float *x, float *out, int rows,
                                                 int nb, float *xs)
{
    const int cols = 256 * nb;
    for (int i = threadIdx.x; i < cols; i += kGemvThreads) xs[i] = x[i];
    __syncthreads();
    const int lane = threadIdx.x & 63;
    const int nw = gridDim.x * (kGemvThreads / 64);
    const int gw = blockIdx.x * (kGemvThreads / 64) + (threadIdx.x >> 6);
    const int NQ = 4 * nb;
    for (int r = gw; r < rows; r += nw) {
        float v = 0.0f;
        for (int qi = lane; qi < NQ; qi += 64) {
            const int j = qi >> 2, h = (qi >> 1) & 1, l0 = (qi & 1) * 16;
            float xg[4][16], sx[4];
            q6_xslice(xs, j, h, l0, xg, sx);
            v += F::dot(F::load(P, (uint32_t)r * NQ + qi), xg, sx);
        }
        v = wave_sum(v);
        if (lane == 0) out[r] = v;
    }
}
__global__ void __launch_bounds__(kGemvThreads)
q6k_gemv_lds(Q6Planes P, const float *x, float *out, int rows, int nb)
{
    __shared__ float xs[kMaxCols];
    quarter_rows_lds<Q6Fmt>(P, x, out, rows, nb, xs);
}

// ---------------------------------------------------------------- Q3_K -----
// The GGUF layout (110 bytes: hmask[32], qs[64], scales[12], f16 d): weight
// 128 n + 32 j + l has low bits (qs[32 n + l] >> 2 j) & 3, third bit
// (hmask[l] >> (4 n + j)) & 1, value q = bits - 4, and scale (16 sub-blocks
// of 16, 6 bits each, minus 32).  A quarter (n, l0) is the Q6_K quarter
// (h = n, g = j).  The upload merges the three bits of a weight into a
// nibble, u = q + 4 (the decode is then Q4_K's: 146 bytes per block on the
// device for the file's 110, and about half the instructions per weight).
// Planes, element e = 4 block + 2 n + l0 / 16:
//   q: 32 bytes per quarter: byte k of the first 16 holds u of weight
//   l0 + k of group 0 (low nibble) and group 1 (high), of the second 16
//   groups 2 and 3; s: one word per quarter, byte j = the signed scale of
//   group j; d: the f16 d per block.
struct Q3Planes {
    const uint8_t *q;
    const uint32_t *s;
    const uint16_t *d;
};
struct Q3Quarter {
    uint4 a, b;
    uint32_t s;
    uint16_t d;
};
struct Q3Fmt {
    typedef Q3Planes Planes;
    typedef Q3Quarter Unit;
    static __device__ __forceinline__ Unit load(const Planes &P, uint32_t e)
    {
        Unit u;
        u.a = ntl4(P.q + e * 32u);
        u.b = ntl4(P.q + e * 32u + 16u);
        u.s = __builtin_nontemporal_load(P.s + e);
        u.d = __builtin_nontemporal_load(P.d + (e >> 2));
        return u;
    }
    // sum over the groups of (d * scale_j) * (sum u x - 4 sum x), u = q + 4
    static __device__ __forceinline__ float dot(const Unit &u, const float (&xg)[4][16], const float (&sx)[4])
    {
        const uint32_t A[4] = {u.a.x, u.a.y, u.a.z, u.a.w}, B[4] = {u.b.x, u.b.y, u.b.z, u.b.w};
        float dt[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int w = 0; w < 4; w++) {
            const uint32_t v[4] = {A[w] & 0x0F0F0F0Fu, (A[w] >> 4) & 0x0F0F0F0Fu, B[w] & 0x0F0F0F0Fu,
                                   (B[w] >> 4) & 0x0F0F0F0Fu};
#pragma unroll
            for (int j = 0; j < 4; j++)
#pragma unroll
                for (int t = 0; t < 4; t++) dt[j] = fmaf(ub(v[j], t), xg[j][4 * w + t], dt[j]);
        }
        const float d = h2f(u.d);
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const float scl = d * (float)(int8_t)(uint8_t)(u.s >> (8 * j));   // (d * sc), as the reference
            acc = fmaf(scl, fmaf(-4.0f, sx[j], dt[j]), acc);
        }
        return acc;
    }
};
constexpr int kRB3 = 8, kPF3 = 2, kNT3 = 768;   // Q3_K: the Q6_K structure
template <int kRB, int PF, int NT>
__global__ void __launch_bounds__(NT)
q3k_gemv_xreg(Q3Planes P, const float *x, float *out, int rows, int nb)
{
    __shared__ float xs[4096];
    __shared__ float tiles[NT / 64][kRB * 64];
    quarter_rows_xreg<Q3Fmt, kRB, PF, NT>(P, x, out, rows, nb, xs, tiles);
}
__global__ void __launch_bounds__(kGemvThreads)
q3k_gemv_lds(Q3Planes P, const float *x, float *out, int rows, int nb)
{
    __shared__ float xs[kMaxCols];
    quarter_rows_lds<Q3Fmt>(P, x, out, rows, nb, xs);
}

// ---------------------------------------------------------------- Q8_0 -----
// Half block hb of a row: block hb / 2, weights 32 (hb / 2) + 16 (hb % 2) .. + 15.
__device__ __forceinline__ float q8_dot(uint4 q, uint16_t d16, const float *xs16, float sx)
{
    const uint32_t W[4] = {q.x ^ 0x80808080u, q.y ^ 0x80808080u, q.z ^ 0x80808080u, q.w ^ 0x80808080u};
    float dot = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; w++)
#pragma unroll
        for (int t = 0; t < 4; t++) dot = fmaf(ub(W[w], t), xs16[4 * w + t], dot);
    return h2f(d16) * fmaf(-128.0f, sx, dot);
}

// Measured on MI355X at the Qwen2.5-7B shape (same box, interleaved runs):
// Q6_K 768 threads (12 waves per CU, 157 VGPRs), 2 rows in flight, 8 rows
// per reduction batch: 77-78 us; one row in flight at 1024 threads: 88-89 us;
// 4 rows in flight (211 VGPRs, 8 waves): 84 us.  Q8_0: 4 rows per batch
// (8 spill at 1024 threads with one row in flight).
constexpr int kRB6 = 8, kPF6 = 2, kNT6 = 768;   // Q6_K: rows per batch, rows in flight, threads
constexpr int kRB8 = 8, kPF8 = 2, kNT8 = 768;   // Q8_0: the same structure
constexpr int kQ8Halves = 4;            // half blocks per lane on the register path (cols <= 4096)

// One row's quants and scales for a lane (kQ8Halves half blocks).
struct Q8Row {
    uint4 q[kQ8Halves];
    uint16_t d[kQ8Halves];
};

// As q6k_gemv_xreg: x (64 values per lane) in registers, PF rows in flight.
template <int kRB, int PF, int NT>
__global__ void __launch_bounds__(NT)
q80_gemv_xreg(const uint8_t *bits, const uint16_t *dq, const float *x, float *out, int rows, int nb)
{
    static_assert(kRB % PF == 0, "ring of PF row buffers, kRB rows per batch");
    __shared__ float xs[4096];
    __shared__ float tiles[NT / 64][kRB * 64];
    const int cols = 32 * nb;
    for (int i = threadIdx.x; i < cols; i += NT) xs[i] = x[i];
    __syncthreads();
    const int lane = threadIdx.x & 63;
    const int nw = gridDim.x * (NT / 64);
    const int gw = blockIdx.x * (NT / 64) + (threadIdx.x >> 6);
    const int nh = 2 * nb;
    float xv[kQ8Halves][16], sx[kQ8Halves];
    bool act[kQ8Halves];
    int hb[kQ8Halves];
#pragma unroll
    for (int k = 0; k < kQ8Halves; k++) {
        act[k] = lane + 64 * k < nh;
        hb[k] = act[k] ? lane + 64 * k : 0;
        const float4 *p = reinterpret_cast<const float4 *>(xs + 16 * hb[k]);
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const float4 v = p[i];
            xv[k][4 * i] = v.x; xv[k][4 * i + 1] = v.y; xv[k][4 * i + 2] = v.z; xv[k][4 * i + 3] = v.w;
        }
#pragma unroll
        for (int i = 0; i < 16; i++) s += xv[k][i];
        sx[k] = s;
    }
    const int rpw = (rows + nw - 1) / nw;
    const int r0 = gw * rpw, r1 = min(rows, r0 + rpw);
    if (r0 >= r1) return;
    float *tile = tiles[threadIdx.x >> 6];
    auto load = [&](int r) {                   // rows past the run read its last row
        const uint32_t rr = (uint32_t)min(r, r1 - 1);
        Q8Row w;
#pragma unroll
        for (int k = 0; k < kQ8Halves; k++) {
            const uint32_t e = rr * (uint32_t)nh + (uint32_t)hb[k];
            w.q[k] = ntl4(bits + e * 16u);
            w.d[k] = __builtin_nontemporal_load(dq + (e >> 1));
        }
        return w;
    };
    auto dot = [&](const Q8Row &w) {
        float v = 0.0f;
#pragma unroll
        for (int k = 0; k < kQ8Halves; k++)
            if (act[k]) v += q8_dot(w.q[k], w.d[k], xv[k], sx[k]);
        return v;
    };
    Q8Row buf[PF];
#pragma unroll
    for (int i = 0; i < PF; i++) buf[i] = load(r0 + i);
    int rb = r0;
    for (; rb + kRB <= r1; rb += kRB) {        // full batches
        float part[kRB];
#pragma unroll
        for (int k = 0; k < kRB; k++) {
            const Q8Row nxt = load(rb + k + PF);
            part[k] = dot(buf[k % PF]);
            buf[k % PF] = nxt;
        }
        const float v = rows_sum<kRB>(part, tile);
        if (lane < kRB) out[rb + lane] = v;
    }
    if (rb < r1) {                             // the last, partial batch
        float part[kRB];
#pragma unroll
        for (int k = 0; k < kRB; k++) {
            part[k] = rb + k < r1 ? dot(buf[k % PF]) : 0.0f;
            if (k + 1 < kRB && (k + 1) % PF == 0 && rb + k + 1 < r1) {
#pragma unroll
                for (int i = 0; i < PF; i++) buf[i] = load(rb + k + 1 + i);
            }
        }
        const float v = rows_sum<kRB>(part, tile);
        if (lane < kRB && rb + lane < r1) out[rb + lane] = v;
    }
}

__global__ void __launch_bounds__(kGemvThreads)
q80_gemv_lds(const uint8_t *bits, const uint16_t *dq, const float *x, float *out, int rows, int nb)
{
    __shared__ float xs[kMaxCols];
    const int cols = 32 * nb;
    for (int i = threadIdx.x; i < cols; i += kGemvThreads) xs[i] = x[i];
    __syncthreads();
    const int lane = threadIdx.x & 63;
    const int nw = gridDim.x * (kGemvThreads / 64);
    const int gw = blockIdx.x * (kGemvThreads / 64) + (threadIdx.x >> 6);
    for (int r = gw; r < rows; r += nw) {
        float v = 0.0f;
        for (int hbk = lane; hbk < 2 * nb; hbk += 64) {
            const size_t blk = (size_t)r * nb + (hbk >> 1);
            const uint4 q = ntl4(bits + blk * 32 + 16 * (hbk & 1));
            const float *xp = xs + 16 * hbk;
            float s = 0.0f;
            for (int i = 0; i < 16; i++) s += xp[i];
            v += q8_dot(q, __builtin_nontemporal_load(dq + blk), xp, s);
        }
        v = wave_sum(v);
        if (lane == 0) out[r] = v;
    }
}

// ---------------------------------------------------------- Q4_0 / Q4_1 -----
// Block j of a row (src/tensor/dequant.rs:26-54): byte l of its 16 bytes of
// nibbles holds weight 32 j + l (low nibble) and 32 j + 16 + l (high).
// Q4_0: w = (q - 8) d; Q4_1: w = q d + m.  Planes: qs, 16 bytes per block;
// Q4_0 the f16 d per block, Q4_1 one word per block, d | m << 16.
struct Q4Planes {
    const uint8_t *qs;
    const uint16_t *d;      // Q4_0
    const uint32_t *dm;     // Q4_1
};
constexpr int kQ4Blocks = 2;            // blocks per lane on the register path (cols <= 4096)
constexpr int kRB4 = 8, kPF4 = 4, kNT4 = 768;   // rows per batch, rows in flight, threads

template <bool Q41>
__device__ __forceinline__ uint32_t q4_dm(const Q4Planes &P, uint32_t blk)
{
    return Q41 ? __builtin_nontemporal_load(P.dm + blk) : (uint32_t)__builtin_nontemporal_load(P.d + blk);
}
// Q4_0: d (sum q x - 8 sum x); Q4_1: d sum q x + m sum x.  xv: the block's
// 32 values of x, sx their sum.
template <bool Q41>
__device__ __forceinline__ float q4_dot(uint4 q, uint32_t dm, const float *xv, float sx)
{
    const uint32_t W[4] = {q.x, q.y, q.z, q.w};
    float lo = 0.0f, hi = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; w++) {
        const uint32_t a = W[w] & 0x0F0F0F0Fu, b = (W[w] >> 4) & 0x0F0F0F0Fu;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            lo = fmaf(ub(a, t), xv[4 * w + t], lo);
            hi = fmaf(ub(b, t), xv[16 + 4 * w + t], hi);
        }
    }
    const float d = h2f((uint16_t)(dm & 0xffffu));
    if (Q41) return fmaf(d, lo + hi, h2f((uint16_t)(dm >> 16)) * sx);
    return d * fmaf(-8.0f, sx, lo + hi);
}

// As q80_gemv_xreg: kQ4Blocks blocks per lane, x (64 values) in registers,
// PF rows in flight.
template <bool Q41, int kRB, int PF, int NT>
__global__ void __launch_bounds__(NT)
q4_gemv_xreg(Q4Planes P, const float *x, float *out, int rows, int nb)
{
    static_assert(kRB % PF == 0, "ring of PF row buffers, kRB rows per batch");
    __shared__ float xs[4096];
    __shared__ float tiles[NT / 64][kRB * 64];
    const int cols = 32 * nb;
    for (int i = threadIdx.x; i < cols; i += NT) xs[i] = x[i];
    __syncthreads();
    const int lane = threadIdx.x & 63;
    const int nw = gridDim.x * (NT / 64);
    const int gw = blockIdx.x * (NT / 64) + (threadIdx.x >> 6);
    float xv[kQ4Blocks][32], sx[kQ4Blocks];
    bool act[kQ4Blocks];
    int bk[kQ4Blocks];
#pragma unroll
    for (int k = 0; k < kQ4Blocks; k++) {
        act[k] = lane + 64 * k < nb;
        bk[k] = act[k] ? lane + 64 * k : 0;
        const float4 *p = reinterpret_cast<const float4 *>(xs + 32 * bk[k]);
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float4 v = p[i];
            xv[k][4 * i] = v.x; xv[k][4 * i + 1] = v.y; xv[k][4 * i + 2] = v.z; xv[k][4 * i + 3] = v.w;
        }
#pragma unroll
        for (int i = 0; i < 32; i++) s += xv[k][i];
        sx[k] = s;
    }
    const int rpw = (rows + nw - 1) / nw;
    const int r0 = gw * rpw, r1 = min(rows, r0 + rpw);
    if (r0 >= r1) return;
    float *tile = tiles[threadIdx.x >> 6];
    struct Row { uint4 q[kQ4Blocks]; uint32_t dm[kQ4Blocks]; };
    auto load = [&](int r) {                   // rows past the run read its last row
        const uint32_t rr = (uint32_t)min(r, r1 - 1);
        Row w;
#pragma unroll
        for (int k = 0; k < kQ4Blocks; k++) {
            const uint32_t e = rr * (uint32_t)nb + (uint32_t)bk[k];
            w.q[k] = ntl4(P.qs + e * 16u);
            w.dm[k] = q4_dm<Q41>(P, e);
        }
        return w;
    };
    auto dot = [&](const Row &w) {
        float v = 0.0f;
#pragma unroll
        for (int k = 0; k < kQ4Blocks; k++)
            if (act[k]) v += q4_dot<Q41>(w.q[k], w.dm[k], xv[k], sx[k]);
        return v;
    };
    Row buf[PF];
#pragma unroll
    for (int i = 0; i < PF; i++) buf[i] = load(r0 + i);
    int rb = r0;
    for (; rb + kRB <= r1; rb += kRB) {        // full batches
        float part[kRB];
#pragma unroll
        for (int k = 0; k < kRB; k++) {
            const Row nxt = load(rb + k + PF);
            part[k] = dot(buf[k % PF]);
            buf[k % PF] = nxt;
        }
        const float v = rows_sum<kRB>(part, tile);
        if (lane < kRB) out[rb + lane] = v;
    }
    if (rb < r1) {                             // the last, partial batch
        float part[kRB];
#pragma unroll
        for (int k = 0; k < kRB; k++) {
            part[k] = rb + k < r1 ? dot(buf[k % PF]) : 0.0f;
            if (k + 1 < kRB && (k + 1) % PF == 0 && rb + k + 1 < r1) {
#pragma unroll
                for (int i = 0; i < PF; i++) buf[i] = load(rb + k + 1 + i);
            }
        }
        const float v = rows_sum<kRB>(part, tile);
        if (lane < kRB && rb + lane < r1) out[rb + lane] = v;
    }
}

template <bool Q41>
__global__ void __launch_bounds__(kGemvThreads)
q4_gemv_lds(Q4Planes P, const float *x, float *out, int rows, int nb)
{
    __shared__ float xs[kMaxCols];
    const int cols = 32 * nb;
    for (int i = threadIdx.x; i < cols; i += kGemvThreads) xs[i] = x[i];
    __syncthreads();
    const int lane = threadIdx.x & 63;
    const int nw = gridDim.x * (kGemvThreads / 64);
    const int gw = blockIdx.x * (kGemvThreads / 64) + (threadIdx.x >> 6);
    for (int r = gw; r < rows; r += nw) {
        float v = 0.0f;
        for (int b = lane; b < nb; b += 64) {
            const uint32_t e = (uint32_t)r * (uint32_t)nb + (uint32_t)b;
            const float *xp = xs + 32 * b;
            float s = 0.0f;
            for (int i = 0; i < 32; i++) s += xp[i];
            v += q4_dot<Q41>(ntl4(P.qs + e * 16u), q4_dm<Q41>(P, e), xp, s);
        }
        v = wave_sum(v);
        if (lane == 0) out[r] = v;
    }
}

// ------------------------------------------------------- Q4_K / Q5_K -----
// Step s of block j (src/tensor/dequant.rs:149-196, a "pair" here) holds the
// 64 weights 256 j + 64 s + l (sub-block 2s: low nibbles of qs[32 s + l])
// and 256 j + 64 s + 32 + l (sub-block 2s + 1: high nibbles), l = 0..31;
// Q5_K adds bit 2s / 2s + 1 of qh[l] as 16.  w = (d * sc) * q - dmin * m.
// Planes (element e = 4 j + s of a row; rows of 4 nb pairs):
//   qs: 32 bytes per pair; h (Q5_K): two words per pair, bit l = the fifth
//   bit of weight l of sub-block 2s / 2s + 1; sm: one word per pair, bytes
//   sc(2s), m(2s), sc(2s + 1), m(2s + 1); dd: one word per block, d | dmin << 16.
struct KPlanes {
    const uint8_t *qs;
    const uint2 *h;
    const uint32_t *sm;
    const uint32_t *dd;
};
struct KPair {
    uint4 a, b;         // qs[32 s .. 32 s + 15], qs[32 s + 16 .. 32 s + 31]
    uint2 h;
    uint32_t sm, dd;
};
template <bool Q5>
__device__ __forceinline__ KPair kq_load(const KPlanes &P, uint32_t e)
{
    KPair q;
    q.a = ntl4(P.qs + e * 32u);
    q.b = ntl4(P.qs + e * 32u + 16u);
    q.h = Q5 ? ntl2(P.h + e) : make_uint2(0u, 0u);
    q.sm = __builtin_nontemporal_load(P.sm + e);
    q.dd = __builtin_nontemporal_load(P.dd + (e >> 2));
    return q;
}
// Bits 0..3 of n to bit 4 of bytes 0..3.
__device__ __forceinline__ uint32_t kq_hi4(uint32_t n) { return ((n * 0x00204081u) & 0x01010101u) << 4; }

// (d sc_A) sum qA x - (dmin m_A) sum x + the same for sub-block B; xa / xb
// the pair's x, sa / sb their sums.
template <bool Q5>
__device__ __forceinline__ float kq_dot(const KPair &q, const float (&xa)[32], const float (&xb)[32], float sa, float sb)
{
    const uint32_t W[8] = {q.a.x, q.a.y, q.a.z, q.a.w, q.b.x, q.b.y, q.b.z, q.b.w};
    float da = 0.0f, db = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        uint32_t lo = W[k] & 0x0F0F0F0Fu, hi = (W[k] >> 4) & 0x0F0F0F0Fu;
        if (Q5) {
            lo |= kq_hi4((q.h.x >> (4 * k)) & 0xFu);
            hi |= kq_hi4((q.h.y >> (4 * k)) & 0xFu);
        }
#pragma unroll
        for (int t = 0; t < 4; t++) {
            da = fmaf(ub(lo, t), xa[4 * k + t], da);
            db = fmaf(ub(hi, t), xb[4 * k + t], db);
        }
    }
    const float d = h2f((uint16_t)(q.dd & 0xffffu)), dmin = h2f((uint16_t)(q.dd >> 16));
    const float d1 = d * (float)(q.sm & 0xffu), mb1 = dmin * (float)((q.sm >> 8) & 0xffu);     // as the reference
    const float d2 = d * (float)((q.sm >> 16) & 0xffu), mb2 = dmin * (float)(q.sm >> 24);
    return fmaf(d1, da, fmaf(-mb1, sa, fmaf(d2, db, -mb2 * sb)));
}
__device__ __forceinline__ void kq_xslice(const float *x, int j, int st, float (&xa)[32], float (&xb)[32],
                                          float *sa, float *sb)
{
    const float4 *pa = reinterpret_cast<const float4 *>(x + 256 * j + 64 * st);
    const float4 *pb = reinterpret_cast<const float4 *>(x + 256 * j + 64 * st + 32);
    float s1 = 0.0f, s2 = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const float4 u = pa[i], v = pb[i];
        xa[4 * i] = u.x; xa[4 * i + 1] = u.y; xa[4 * i + 2] = u.z; xa[4 * i + 3] = u.w;
        xb[4 * i] = v.x; xb[4 * i + 1] = v.y; xb[4 * i + 2] = v.z; xb[4 * i + 3] = v.w;
    }
#pragma unroll
    for (int i = 0; i < 32; i++) { s1 += xa[i]; s2 += xb[i]; }
    *sa = s1;
    *sb = s2;
}

// As q6k_gemv_xreg, a pair per lane (rows of up to 16 blocks).
template <bool Q5, int kRB, int PF, int NT>
__global__ void __launch_bounds__(NT)
kq_gemv_xreg(KPlanes P, const float *x, float *out, int rows, int nb)
{
    static_assert(kRB % PF == 0, "ring of PF row buffers, kRB rows per batch");
    __shared__ float xs[4096];
    __shared__ float tiles[NT / 64][kRB * 64];
    const int cols = 256 * nb;
    for (int i = threadIdx.x; i < cols; i += NT) xs[i] = x[i];
    __syncthreads();
    const int lane = threadIdx.x & 63;
    const int nw = gridDim.x * (NT / 64);
    const int gw = blockIdx.x * (NT / 64) + (threadIdx.x >> 6);
    const int NQ = 4 * nb;
    const bool act = lane < NQ;
    const int qi = act ? lane : 0;
    float xa[32], xb[32], sa, sb;
    kq_xslice(xs, qi >> 2, qi & 3, xa, xb, &sa, &sb);
    const int rpw = (rows + nw - 1) / nw;
    const int r0 = gw * rpw, r1 = min(rows, r0 + rpw);
    if (r0 >= r1) return;
    float *tile = tiles[threadIdx.x >> 6];
    const uint32_t e1 = (uint32_t)(r1 - 1) * NQ + qi;
    auto row_e = [&](int r) { return min((uint32_t)r * NQ + qi, e1); };   // past the run: its last row
    KPair buf[PF];
#pragma unroll
    for (int i = 0; i < PF; i++) buf[i] = kq_load<Q5>(P, row_e(r0 + i));
    int rb = r0;
    for (; rb + kRB <= r1; rb += kRB) {
        float part[kRB];
#pragma unroll
        for (int k = 0; k < kRB; k++) {
            const KPair nxt = kq_load<Q5>(P, row_e(rb + k + PF));
            part[k] = act ? kq_dot<Q5>(buf[k % PF], xa, xb, sa, sb) : 0.0f;
            buf[k % PF] = nxt;
        }
        const float v = rows_sum<kRB>(part, tile);
        if (lane < kRB) out[rb + lane] = v;
    }
    if (rb < r1) {
        float part[kRB];
#pragma unroll
        for (int k = 0; k < kRB; k++) {
            part[k] = 0.0f;
            if (rb + k < r1 && act) part[k] = kq_dot<Q5>(buf[k % PF], xa, xb, sa, sb);
            if (k + 1 < kRB && (k + 1) % PF == 0 && rb + k + 1 < r1) {
#pragma unroll
                for (int i = 0; i < PF; i++) buf[i] = kq_load<Q5>(P, row_e(rb + k + 1 + i));
            }
        }
        const float v = rows_sum<kRB>(part, tile);
        if (lane < kRB && rb + lane < r1) out[rb + lane] = v;
    }
}

template <bool Q5>
__global__ void __launch_bounds__(kGemvThreads)
kq_gemv_lds(KPlanes P, const float *x, float *out, int rows, int nb)
{
    __shared__ float xs[kMaxCols];
    const int cols = 256 * nb;
    for (int i = threadIdx.x; i < cols; i += kGemvThreads) xs[i] = x[i];
    __syncthreads();
    const int lane = threadIdx.x & 63;
    const int nw = gridDim.x * (kGemvThreads / 64);
    const int gw = blockIdx.x * (kGemvThreads / 64) + (threadIdx.x >> 6);
    const int NQ = 4 * nb;
    for (int r = gw; r < rows; r += nw) {
        float v = 0.0f;
        for (int qi = lane; qi < NQ; qi += 64) {
            float xa[32], xb[32], sa, sb;
            kq_xslice(xs, qi >> 2, qi & 3, xa, xb, &sa, &sb);
            v += kq_dot<Q5>(kq_load<Q5>(P, (uint32_t)r * NQ + qi), xa, xb, sa, sb);
        }
        v = wave_sum(v);
        if (lane == 0) out[r] = v;
    }
}
constexpr int kRBK = 8, kPFK = 2, kNTK = 768;   // K-quants: the Q6_K structure

} // namespace gs

// ------------------------------------------------------------- host side ---
struct gs_qmatrix {
    uint32_t qtype;
    size_t rows, cols, nb;     // nb: blocks per row
    int device;
    int cus;                   // compute units: one 1024-thread workgroup each on the register paths
    uint8_t *base;             // one device allocation holding the planes
    gs::Q6Planes q6;           // Q6_K
    gs::KPlanes kq;            // Q4_K / Q5_K
    gs::Q3Planes q3;           // Q3_K
    gs::Q4Planes q4;           // Q4_0 / Q4_1
    const uint8_t *q8;         // Q8_0: int8 quants
    const uint16_t *d;         // f16 d per block (Q8_0, Q6_K)
};

namespace {
// get_scale_min_k4 (src/tensor/dequant.rs:141-148): the 6-bit scale and min
// of sub-block j from the block's 12 packed bytes.
void scale_min_k4(int j, const uint8_t *q, uint8_t *d, uint8_t *m)
{
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (uint8_t)((q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4));
        *m = (uint8_t)((q[j + 4] >> 4) | ((q[j] >> 6) << 4));
    }
}

// Q4_K (144-byte blocks) / Q5_K (176) to the K planes (see KPlanes).
int upload_kquant(bool q5, const uint8_t *src, size_t rows, size_t nb, gs_qmatrix *m)
{
    const size_t n = rows * nb, np = 4 * n;
    auto al = [](size_t v) { return (v + 255) & ~(size_t)255; };
    const size_t off_h = al(np * 32), off_sm = off_h + (q5 ? al(np * 8) : 0), off_dd = off_sm + al(np * 4);
    const size_t total = off_dd + n * 4;
    uint8_t *h = new (std::nothrow) uint8_t[total];
    if (!h) return GS_ERR_NOMEM;
    const size_t bb = q5 ? 176 : 144;
    for (size_t i = 0; i < n; i++) {
        const uint8_t *b = src + i * bb;
        const uint8_t *scales = b + 4, *qh = b + 16, *qs = b + (q5 ? 48 : 16);
        for (int st = 0; st < 4; st++) {
            const size_t e = 4 * i + st;
            memcpy(h + e * 32, qs + 32 * st, 32);
            uint8_t sc1, m1, sc2, m2;
            scale_min_k4(2 * st, scales, &sc1, &m1);
            scale_min_k4(2 * st + 1, scales, &sc2, &m2);
            const uint32_t w = (uint32_t)sc1 | ((uint32_t)m1 << 8) | ((uint32_t)sc2 << 16) | ((uint32_t)m2 << 24);
            memcpy(h + off_sm + e * 4, &w, 4);
            if (q5) {
                uint32_t ha = 0, hb = 0;
                for (int l = 0; l < 32; l++) {
                    ha |= (uint32_t)((qh[l] >> (2 * st)) & 1u) << l;
                    hb |= (uint32_t)((qh[l] >> (2 * st + 1)) & 1u) << l;
                }
                memcpy(h + off_h + e * 8, &ha, 4);
                memcpy(h + off_h + e * 8 + 4, &hb, 4);
            }
        }
        memcpy(h + off_dd + i * 4, b, 4);   // d, dmin (f16 each)
    }
    if (hipMalloc((void **)&m->base, total) != hipSuccess) {
        (void)hipGetLastError();
        delete[] h;
        return GS_ERR_NOMEM;
    }
    const hipError_t ce = hipMemcpy(m->base, h, total, hipMemcpyHostToDevice);
    delete[] h;
    if (ce != hipSuccess) { (void)hipFree(m->base); m->base = nullptr; return GS_ERR_HIP; }
    m->kq = gs::KPlanes{m->base, q5 ? (const uint2 *)(m->base + off_h) : nullptr,
                        (const uint32_t *)(m->base + off_sm), (const uint32_t *)(m->base + off_dd)};
    return GS_OK;
}
// Q4_0 (18-byte blocks) / Q4_1 (20) to the Q4 planes (see Q4Planes).
int upload_q4(bool q41, const uint8_t *src, size_t rows, size_t nb, gs_qmatrix *m)
{
    const size_t n = rows * nb;
    const size_t off_d = (n * 16 + 255) & ~(size_t)255;
    const size_t total = off_d + n * (q41 ? 4 : 2);
    uint8_t *h = new (std::nothrow) uint8_t[total];
    if (!h) return GS_ERR_NOMEM;
    const size_t bb = q41 ? 20 : 18;
    for (size_t i = 0; i < n; i++) {
        const uint8_t *b = src + i * bb;
        memcpy(h + i * 16, b + (q41 ? 4 : 2), 16);
        memcpy(h + off_d + i * (q41 ? 4 : 2), b, q41 ? 4 : 2);   // d (, m): f16 each
    }
    if (hipMalloc((void **)&m->base, total) != hipSuccess) {
        (void)hipGetLastError();
        delete[] h;
        return GS_ERR_NOMEM;
    }
    const hipError_t ce = hipMemcpy(m->base, h, total, hipMemcpyHostToDevice);
    delete[] h;
    if (ce != hipSuccess) { (void)hipFree(m->base); m->base = nullptr; return GS_ERR_HIP; }
    m->q4 = gs::Q4Planes{m->base, q41 ? nullptr : (const uint16_t *)(m->base + off_d),
                         q41 ? (const uint32_t *)(m->base + off_d) : nullptr};
    return GS_OK;
}

// The signed 6-bit scale of sub-block is of a Q3_K block in the GGUF
// packing: low nibble from byte is % 8 (bits 0-3 for is < 8, 4-7 above),
// top two bits from bits 2 (is / 4) of byte 8 + is % 4; minus 32.
int q3k_scale(const uint8_t *sc, int is)
{
    const int k = is >> 2, j = is & 3;
    const uint8_t nb = sc[(k & 1) * 4 + j];
    const int low = k < 2 ? (nb & 0xF) : (nb >> 4);
    return (low | (((sc[8 + j] >> (2 * k)) & 3) << 4)) - 32;
}

// Q3_K (110-byte blocks) to the Q3 planes (see Q3Planes).
int upload_q3k(const uint8_t *src, size_t rows, size_t nb, gs_qmatrix *m)
{
    const size_t n = rows * nb, np = 4 * n;
    auto al = [](size_t v) { return (v + 255) & ~(size_t)255; };
    const size_t off_s = al(np * 32), off_d = off_s + al(np * 4);
    const size_t total = off_d + n * 2;
    uint8_t *h = new (std::nothrow) uint8_t[total];
    if (!h) return GS_ERR_NOMEM;
    for (size_t i = 0; i < n; i++) {
        const uint8_t *b = src + i * 110;
        const uint8_t *hm = b, *qs = b + 32, *sc = b + 96;
        for (int qq = 0; qq < 4; qq++) {
            const int nn = qq >> 1, l0 = (qq & 1) * 16;
            const size_t e = 4 * i + qq;
            for (int j = 0; j < 4; j++)
                for (int k = 0; k < 16; k++) {
                    const int l = l0 + k;
                    const uint8_t u = (uint8_t)(((qs[32 * nn + l] >> (2 * j)) & 3u) | (((hm[l] >> (4 * nn + j)) & 1u) << 2));
                    uint8_t &dst = h[e * 32 + 16 * (j >> 1) + k];
                    dst = (j & 1) ? (uint8_t)(dst | (u << 4)) : u;
                }
            for (int j = 0; j < 4; j++)
                h[off_s + e * 4 + j] = (uint8_t)(int8_t)q3k_scale(sc, 8 * nn + 2 * j + l0 / 16);
        }
        memcpy(h + off_d + i * 2, b + 108, 2);
    }
    if (hipMalloc((void **)&m->base, total) != hipSuccess) {
        (void)hipGetLastError();
        delete[] h;
        return GS_ERR_NOMEM;
    }
    const hipError_t ce = hipMemcpy(m->base, h, total, hipMemcpyHostToDevice);
    delete[] h;
    if (ce != hipSuccess) { (void)hipFree(m->base); m->base = nullptr; return GS_ERR_HIP; }
    m->q3 = gs::Q3Planes{m->base, (const uint32_t *)(m->base + off_s), (const uint16_t *)(m->base + off_d)};
    return GS_OK;
}
} // namespace

extern "C" {

int gs_qmatrix_upload(uint32_t qtype, const void *blocks, size_t rows, size_t cols, gs_qmatrix **out)
{
    if (!out) return GS_ERR_INVALID;
    *out = nullptr;
    if (!blocks || rows == 0 || cols == 0) return GS_ERR_INVALID;
    if (qtype != GS_QTYPE_Q8_0 && qtype != GS_QTYPE_Q6_K && qtype != GS_QTYPE_Q4_K && qtype != GS_QTYPE_Q5_K &&
        qtype != GS_QTYPE_Q4_0 && qtype != GS_QTYPE_Q4_1 && qtype != GS_QTYPE_Q3_K)
        return GS_ERR_UNSUPPORTED;
    if (qtype == GS_QTYPE_Q4_K || qtype == GS_QTYPE_Q5_K || qtype == GS_QTYPE_Q4_0 || qtype == GS_QTYPE_Q4_1 ||
        qtype == GS_QTYPE_Q3_K) {
        const bool q4 = qtype == GS_QTYPE_Q4_0 || qtype == GS_QTYPE_Q4_1;
        const size_t bw = q4 ? 32 : 256;
        if (cols % bw != 0 || cols > (size_t)gs::kMaxCols || rows > 0x7fffffffu) return GS_ERR_UNSUPPORTED;
        // 32-bit byte offsets of the widest plane
        if (rows * (cols / 64) >= (q4 ? (1ull << 29) : (1ull << 27))) return GS_ERR_UNSUPPORTED;
        gs_qmatrix *m = new (std::nothrow) gs_qmatrix();
        if (!m) return GS_ERR_NOMEM;
        m->qtype = qtype; m->rows = rows; m->cols = cols; m->nb = cols / bw;
        if (hipGetDevice(&m->device) != hipSuccess ||
            hipDeviceGetAttribute(&m->cus, hipDeviceAttributeMultiprocessorCount, m->device) != hipSuccess) {
            delete m; return GS_ERR_HIP;
        }
        if (m->cus <= 0) m->cus = 256;
        const int rc = q4 ? upload_q4(qtype == GS_QTYPE_Q4_1, (const uint8_t *)blocks, rows, cols / 32, m)
                       : qtype == GS_QTYPE_Q3_K ? upload_q3k((const uint8_t *)blocks, rows, cols / 256, m)
                       : upload_kquant(qtype == GS_QTYPE_Q5_K, (const uint8_t *)blocks, rows, cols / 256, m);
        if (rc != GS_OK) { delete m; return rc; }
        *out = m;
        return GS_OK;
    }
    const bool q6 = qtype == GS_QTYPE_Q6_K;
    const size_t bw = q6 ? 256 : 32;        // weights per block
    const size_t bb = q6 ? 210 : 34;        // bytes per GGUF block
    if (cols % bw != 0 || cols > (size_t)gs::kMaxCols || rows > 0x7fffffffu) return GS_ERR_UNSUPPORTED;
    if (rows * (cols / 64) >= (1ull << 28)) return GS_ERR_UNSUPPORTED;   // 32-bit chunk offsets
    const size_t nb = cols / bw, n = rows * nb;
    auto al = [](size_t v) { return (v + 255) & ~(size_t)255; };
    // planes: Q6_K a | b | c (64 bytes per block each) | scale words (16) | d (2);
    //         Q8_0 quants (32 bytes per block) | d (2)
    const size_t pa = q6 ? al(n * 64) : al(n * 32);
    const size_t off_b = pa, off_c = q6 ? 2 * pa : pa, off_s = q6 ? 3 * pa : pa;
    const size_t off_d = q6 ? off_s + al(n * 16) : pa;
    const size_t total = off_d + n * 2;
    uint8_t *h = new (std::nothrow) uint8_t[total];
    if (!h) return GS_ERR_NOMEM;
    const uint8_t *src = (const uint8_t *)blocks;
    for (size_t i = 0; i < n; i++) {
        const uint8_t *b = src + i * bb;
        if (q6) {
            // quarter qq = 2h + l0/16 of block i: element e = 4i + qq of each plane
            for (int qq = 0; qq < 4; qq++) {
                const int hh = qq >> 1, l0 = (qq & 1) * 16, is = l0 / 16;
                const size_t e = 4 * i + qq;
                memcpy(h + e * 16, b + 64 * hh + l0, 16);                  // ql[64h + l0 ..]
                memcpy(h + off_b + e * 16, b + 64 * hh + 32 + l0, 16);     // ql[64h + 32 + l0 ..]
                memcpy(h + off_c + e * 16, b + 128 + 32 * hh + l0, 16);    // qh[32h + l0 ..]
                for (int g = 0; g < 4; g++) h[off_s + e * 4 + g] = b[192 + 8 * hh + is + 2 * g];
            }
            memcpy(h + off_d + i * 2, b + 208, 2);
        } else {
            memcpy(h + i * 32, b + 2, 32);
            memcpy(h + off_d + i * 2, b, 2);
        }
    }
    gs_qmatrix *m = new (std::nothrow) gs_qmatrix();
    if (!m) { delete[] h; return GS_ERR_NOMEM; }
    m->qtype = qtype; m->rows = rows; m->cols = cols; m->nb = nb;
    if (hipGetDevice(&m->device) != hipSuccess ||
        hipDeviceGetAttribute(&m->cus, hipDeviceAttributeMultiprocessorCount, m->device) != hipSuccess) {
        delete[] h; delete m; return GS_ERR_HIP;
    }
    if (m->cus <= 0) m->cus = 256;
    if (hipMalloc((void **)&m->base, total) != hipSuccess) {
        (void)hipGetLastError(); delete[] h; delete m; return GS_ERR_NOMEM;
    }
    const hipError_t ce = hipMemcpy(m->base, h, total, hipMemcpyHostToDevice);
    delete[] h;
    if (ce != hipSuccess) { (void)hipFree(m->base); delete m; return GS_ERR_HIP; }
    m->d = (const uint16_t *)(m->base + off_d);
    if (q6) m->q6 = gs::Q6Planes{m->base, m->base + off_b, m->base + off_c, (const uint32_t *)(m->base + off_s), m->d};
    else m->q8 = m->base;
    *out = m;
    return GS_OK;
}

int gs_qmatrix_destroy(gs_qmatrix *m)
{
    if (!m) return GS_ERR_INVALID;
    int dev;
    (void)hipGetDevice(&dev);
    (void)hipSetDevice(m->device);
    (void)hipDeviceSynchronize();
    (void)hipFree(m->base);
    (void)hipSetDevice(dev);
    delete m;
    return GS_OK;
}

int gs_qmatrix_shape(const gs_qmatrix *m, uint32_t *qtype, size_t *rows, size_t *cols)
{
    if (!m) return GS_ERR_INVALID;
    if (qtype) *qtype = m->qtype;
    if (rows) *rows = m->rows;
    if (cols) *cols = m->cols;
    return GS_OK;
}

int gs_gemv(const gs_qmatrix *m, const float *d_x, size_t B, float *d_out, void *stream)
{
    if (!m || (B > 0 && (!d_x || !d_out))) return GS_ERR_INVALID;
    if (((uintptr_t)d_x & 15u) != 0 || (B > 1 && (m->cols & 3) != 0)) return GS_ERR_INVALID;   // x is read as float4
    const hipStream_t st = (hipStream_t)stream;
    const int rows = (int)m->rows, nb = (int)m->nb;
    for (size_t b = 0; b < B; b++) {
        const float *x = d_x + b * m->cols;
        float *o = d_out + b * m->rows;
        if (m->qtype == GS_QTYPE_Q4_K || m->qtype == GS_QTYPE_Q5_K) {
            const bool q5 = m->qtype == GS_QTYPE_Q5_K;
            if (4 * nb <= 64) {
                if (q5) hipLaunchKernelGGL((gs::kq_gemv_xreg<true, gs::kRBK, gs::kPFK, gs::kNTK>), dim3(m->cus), dim3(gs::kNTK), 0, st, m->kq, x, o, rows, nb);
                else hipLaunchKernelGGL((gs::kq_gemv_xreg<false, gs::kRBK, gs::kPFK, gs::kNTK>), dim3(m->cus), dim3(gs::kNTK), 0, st, m->kq, x, o, rows, nb);
            } else {
                if (q5) hipLaunchKernelGGL(gs::kq_gemv_lds<true>, dim3(2 * m->cus), dim3(gs::kGemvThreads), 0, st, m->kq, x, o, rows, nb);
                else hipLaunchKernelGGL(gs::kq_gemv_lds<false>, dim3(2 * m->cus), dim3(gs::kGemvThreads), 0, st, m->kq, x, o, rows, nb);
            }
        } else if (m->qtype == GS_QTYPE_Q4_0 || m->qtype == GS_QTYPE_Q4_1) {
            const bool q41 = m->qtype == GS_QTYPE_Q4_1;
            if (nb <= 64 * gs::kQ4Blocks) {
                if (q41) hipLaunchKernelGGL((gs::q4_gemv_xreg<true, gs::kRB4, gs::kPF4, gs::kNT4>), dim3(m->cus), dim3(gs::kNT4), 0, st, m->q4, x, o, rows, nb);
                else hipLaunchKernelGGL((gs::q4_gemv_xreg<false, gs::kRB4, gs::kPF4, gs::kNT4>), dim3(m->cus), dim3(gs::kNT4), 0, st, m->q4, x, o, rows, nb);
            } else {
                if (q41) hipLaunchKernelGGL(gs::q4_gemv_lds<true>, dim3(2 * m->cus), dim3(gs::kGemvThreads), 0, st, m->q4, x, o, rows, nb);
                else hipLaunchKernelGGL(gs::q4_gemv_lds<false>, dim3(2 * m->cus), dim3(gs::kGemvThreads), 0, st, m->q4, x, o, rows, nb);
            }
        } else if (m->qtype == GS_QTYPE_Q3_K) {
            if (4 * nb <= 64)
                hipLaunchKernelGGL((gs::q3k_gemv_xreg<gs::kRB3, gs::kPF3, gs::kNT3>), dim3(m->cus), dim3(gs::kNT3), 0, st, m->q3, x, o, rows, nb);
            else
                hipLaunchKernelGGL(gs::q3k_gemv_lds, dim3(2 * m->cus), dim3(gs::kGemvThreads), 0, st, m->q3, x, o, rows, nb);
        } else if (m->qtype == GS_QTYPE_Q6_K) {
            if (4 * nb <= 64)
                hipLaunchKernelGGL((gs::q6k_gemv_xreg<gs::kRB6, gs::kPF6, gs::kNT6>), dim3(m->cus), dim3(gs::kNT6), 0, st, m->q6, x, o, rows, nb);
            else
                hipLaunchKernelGGL(gs::q6k_gemv_lds, dim3(2 * m->cus), dim3(gs::kGemvThreads), 0, st, m->q6, x, o, rows, nb);
        } else {
            if (2 * nb <= 64 * gs::kQ8Halves)
                hipLaunchKernelGGL((gs::q80_gemv_xreg<gs::kRB8, gs::kPF8, gs::kNT8>), dim3(m->cus), dim3(gs::kNT8), 0, st, m->q8, m->d, x, o, rows, nb);
            else
                hipLaunchKernelGGL(gs::q80_gemv_lds, dim3(2 * m->cus), dim3(gs::kGemvThreads), 0, st, m->q8, m->d, x, o, rows, nb);
        }
        if (hipGetLastError() != hipSuccess) return GS_ERR_HIP;
    }
    return GS_OK;
}

} // extern "C"
