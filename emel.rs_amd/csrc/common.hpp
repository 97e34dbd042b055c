// common.hpp -- device helpers shared by the gfx950 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace emel {

constexpr int kWave = 64;      // CDNA wavefront width
constexpr int kBlock = 256;    // threads per workgroup (4 waves)

// Unsigned 32-bit division by a run-time invariant divisor through a
// multiply-high (Granlund & Montgomery, "Division by Invariant Integers
// using Multiplication", PLDI 1994, Fig. 4.1): with l = ceil(log2 d) and
// m = floor(2^32 (2^l - d) / d) + 1, n / d = (mulhi(n, m) + n) >> l for all
// n < 2^32 (the sum is formed in 64 bits).
struct FastDiv {
    uint32_t d;
    uint32_t m;
    uint32_t l;

    FastDiv() = default;
    __host__ explicit FastDiv(uint32_t divisor) : d(divisor)
    {
        l = 0;
        while ((uint64_t{1} << l) < divisor) ++l;
        m = static_cast<uint32_t>(((uint64_t{1} << 32) * ((uint64_t{1} << l) - divisor)) / divisor + 1);
    }
    __host__ __device__ __forceinline__ uint32_t div(uint32_t n) const
    {
        const uint32_t hi = static_cast<uint32_t>((static_cast<uint64_t>(n) * m) >> 32);
        return static_cast<uint32_t>((static_cast<uint64_t>(hi) + n) >> l);
    }
    __host__ __device__ __forceinline__ uint32_t mod(uint32_t n) const { return n - div(n) * d; }
};

// ---- wave reductions (wave64, butterfly over ds_swizzle/DPP) ------------

__device__ __forceinline__ double wave_sum(double v)
{
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

__device__ __forceinline__ float wave_sum(float v)
{
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

// Maximum that ignores NaN operands (IEEE maxNum).  The reductions that use
// it only need the maximum of the non-NaN values: a NaN anywhere in a
// soft_max row turns the whole row into NaN through its sum.
__device__ __forceinline__ float wave_max(float v)
{
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) v = __builtin_fmaxf(v, __shfl_xor(v, off, kWave));
    return v;
}

// (value, index) candidates for argmax: b beats a when it is strictly
// greater, or equal with a lower index.  NaN never enters a candidate.
__device__ __forceinline__ void argmax_merge(float &bv, uint32_t &bi, float v, uint32_t i)
{
    if (v > bv || (v == bv && i < bi)) {
        bv = v;
        bi = i;
    }
}

__device__ __forceinline__ void wave_argmax(float &bv, uint32_t &bi)
{
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off, kWave);
        const uint32_t oi = __shfl_xor(bi, off, kWave);
        argmax_merge(bv, bi, ov, oi);
    }
}

// Non-temporal (streaming) 128-bit global accesses, for data that is read
// once or written once: they keep row streams from displacing cached
// operands (weight rows, masks, tables) in L2 and the Infinity Cache.
typedef float v4f __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float4 ld_nt(const float4 *p)
{
    const v4f v = __builtin_nontemporal_load(reinterpret_cast<const v4f *>(p));
    return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void st_nt(float4 *p, float4 a)
{
    const v4f v = {a.x, a.y, a.z, a.w};
    __builtin_nontemporal_store(v, reinterpret_cast<v4f *>(p));
}

// Block index remapped so that consecutive logical blocks run on the same
// XCD (the dispatcher places block b on XCD b % 8): logical ids
// [x*per, (x+1)*per) execute on XCD x.  Requires gridDim.x % 8 == 0.
__device__ __forceinline__ uint32_t xcd_major_block(uint32_t nxcd)
{
    const uint32_t b = blockIdx.x;
    const uint32_t per = gridDim.x / nxcd;
    return (b % nxcd) * per + b / nxcd;
}

} // namespace emel
