// gs_device.hpp -- device helpers for the gfx950 token sampler.
//
// Everything here is bit-exact with the host semantics of gguf-rs-cli's
// src/sampler.rs (Rust f32 ops are single IEEE ops; f32::exp is glibc expf).
// Compiled with -ffp-contract=off; every fused multiply-add below is written
// explicitly where the host code it mirrors uses one.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "gs_lcg.hpp"

namespace gs {

// ---------------------------------------------------------------------------
// expf, bit-exact with glibc 2.35 expf on x86_64 (FMA ifunc variant).
//
// Published method: ARM optimized-routines expf (Szabolcs Nagy, 2017), the
// algorithm glibc ships as sysdeps/ieee754/flt-32/e_expf.c:
//   exp(x) = 2^(k/32) * 2^(r/32),  k = round(x*32/ln2), |r| <= 1/2,
// evaluated in double: a 32-entry table of 2^(i/32) and a cubic for 2^(r/32).
// The table entries are RN(2^(i/32)) with i<<47 subtracted (recomputed from the
// definition, not copied).  The cubic coefficients are the published minimax
// coefficients of that method.  The FMA on the reduction steps reproduces the
// x86_64 FMA build of glibc; the pairing was verified exhaustively on every
// f32 in [-103.97, 0] against the host libm (0 mismatches of 1.12e9).
// The sampler only evaluates exp at x = y - max <= 0.
// ---------------------------------------------------------------------------
__device__ __constant__ uint64_t kExp2Tab[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull};

// The same function with the table read from `tab` (e.g. a copy in LDS).
__device__ __forceinline__ float glibc_expf_tab(float x, const uint64_t *tab);
__device__ __forceinline__ float glibc_expf(float x)
{
    return glibc_expf_tab(x, kExp2Tab);
}
__device__ __forceinline__ float glibc_expf_tab(float x, const uint64_t *tab)
{
    const uint32_t ux = __float_as_uint(x);
    const uint32_t abstop = (ux >> 20) & 0x7ff;
    if (abstop >= 0x42b) {                       // |x| >= 88 or x is nan/inf
        if (ux == 0xff800000u) return 0.0f;      // -inf
        if (abstop >= 0x7f8) return x + x;       // nan, +inf
        if (x > 0x1.62e42ep6f) return __uint_as_float(0x7f800000u);
        if (x < -0x1.9fe368p6f) return 0.0f;     // underflow
    }
    const double N = 32.0;
    const double InvLn2N = 0x1.71547652b82fep+0 * N;
    const double Shift = 0x1.8p+52;
    const double C0 = 0x1.c6af84b912394p-5 / N / N / N;
    const double C1 = 0x1.ebfce50fac4f3p-3 / N / N;
    const double C2 = 0x1.62e42ff0c52d6p-1 / N;
    const double xd = (double)x;
    double kd = __builtin_fma(InvLn2N, xd, Shift);
    const uint64_t ki = (uint64_t)__double_as_longlong(kd);
    kd = kd - Shift;
    const double r = __builtin_fma(InvLn2N, xd, -kd);
    uint64_t t = tab[ki & 31];
    t += ki << 47;
    const double s = __longlong_as_double((long long)t);
    const double z = __builtin_fma(C0, r, C1);
    const double r2 = r * r;
    double y = __builtin_fma(C2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    y = y * s;
    return (float)y;
}

// Order-preserving map f32 -> u32 (larger float -> larger key).  -0.0 is
// folded onto +0.0 because the reference compares with partial_cmp, under
// which the two are equal (and therefore tie-broken by index).
__device__ __forceinline__ uint32_t f2key(float f)
{
    uint32_t u = __float_as_uint(f);
    if ((u << 1) == 0) u = 0;
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float key2f(uint32_t k)
{
    uint32_t u = (k & 0x80000000u) ? (k & 0x7fffffffu) : ~k;
    return __uint_as_float(u);
}

// Repetition penalty of one logit seen `count` times (src/sampler.rs:23-30):
// the reference applies the op once per occurrence, re-testing the sign.
__device__ __forceinline__ float penalize(float l, uint32_t count, float p)
{
    for (uint32_t c = 0; c < count; c++) l = (l > 0.0f) ? (l / p) : (l * p);
    return l;
}

// Counter-based synthetic logits (Irwin-Hall(4) over splitmix64 words).
// Equal, bit for bit, to the host restatement used by the tests.
__host__ __device__ __forceinline__ uint64_t splitmix64(uint64_t x)
{
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}
__host__ __device__ __forceinline__ float synth_logit(uint64_t seed, uint64_t counter, float sigma)
{
    uint64_t h = splitmix64(seed ^ splitmix64(counter));
    int32_t s = (int32_t)(h & 0xFFFF) + (int32_t)((h >> 16) & 0xFFFF) +
                (int32_t)((h >> 32) & 0xFFFF) + (int32_t)((h >> 48) & 0xFFFF);
    float z = (float)(2 * s - 262140) * 0x1.bb67bp-17f;
    return z * sigma;
}

// Global-memory accessors.  The address space is stated so that the backend
// emits global_* instructions: a flat access also counts against the LDS
// wait counter, so in loops that mix row loads with LDS atomics every LDS
// wait would also wait for the outstanding row loads.
template <class T>
__device__ __forceinline__ T ldg(const T *p)
{
    return *(const __attribute__((address_space(1))) T *)p;
}
typedef float gs_f4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 ldg(const float4 *p)
{
    const gs_f4 v = *(const __attribute__((address_space(1))) gs_f4 *)p;
    return make_float4(v.x, v.y, v.z, v.w);
}
// The same load with the non-temporal hint, for logits read for the last time
// (a row's single pass, or its last): they then stream past L2 instead of
// evicting lines still in use (candidate lists, written list entries).
__device__ __forceinline__ float4 ldg_nt(const float4 *p)
{
    const gs_f4 v = __builtin_nontemporal_load((const __attribute__((address_space(1))) gs_f4 *)p);
    return make_float4(v.x, v.y, v.z, v.w);
}
typedef uint32_t gs_u4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 ldg(const uint4 *p)
{
    const gs_u4 v = *(const __attribute__((address_space(1))) gs_u4 *)p;
    return make_uint4(v.x, v.y, v.z, v.w);
}
template <class T>
__device__ __forceinline__ void stg(T *p, T v)
{
    *(__attribute__((address_space(1))) T *)p = v;
}

} // namespace gs
