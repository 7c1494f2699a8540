// gs_lcg.hpp -- the reference LCG, shared by host and device code.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gs {

// The reference's LCG (src/sampler.rs:7-12) with O(log n) jump-ahead.
__host__ __device__ __forceinline__ uint64_t lcg_jump(uint64_t s, uint64_t n)
{
    uint64_t a = 6364136223846793005ull, c = 1442695040888963407ull;
    uint64_t A = 1, C = 0;
    while (n) {
        if (n & 1) { A = A * a; C = C * a + c; }
        c = c * (a + 1);
        a = a * a;
        n >>= 1;
    }
    return A * s + C;
}
__host__ __device__ __forceinline__ float lcg_value(uint64_t s)
{
    return (float)(s >> 33) / 4294967296.0f;   // u32::MAX as f32 == 2^32
}

} // namespace gs
