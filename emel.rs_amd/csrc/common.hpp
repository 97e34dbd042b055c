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

// ---- wave reductions over DPP (no LDS traffic) ------------------------------
//
// Within each 16-lane row, four DPP steps combine lanes pairwise: quad_perm
// [1,0,3,2] and [2,3,0,1] (lane ^ 1, lane ^ 2), row_half_mirror (lane i of
// an 8-lane half with lane 7 - i, i.e. the other quad) and row_mirror (lane
// i with lane 15 - i, the other half).  After them every lane holds its
// row's result; v_readlane of lanes 0, 16, 32 and 48 then combines the four
// rows.  The combination order is fixed, so results do not depend on which
// wave computes them.
enum : int { kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140 };

template <int CTRL>
__device__ __forceinline__ uint32_t dpp32(uint32_t v)
{
    return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, 0xF, 0xF, false));
}

template <int CTRL>
__device__ __forceinline__ double dpp64(double v)
{
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint64_t lo = dpp32<CTRL>(static_cast<uint32_t>(b));
    const uint64_t hi = dpp32<CTRL>(static_cast<uint32_t>(b >> 32));
    return __builtin_bit_cast(double, lo | (hi << 32));
}

__device__ __forceinline__ uint32_t lane_u32(uint32_t v, int lane)
{
    return static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(v), lane));
}

__device__ __forceinline__ float lane_f32(float v, int lane)
{
    return __builtin_bit_cast(float, lane_u32(__builtin_bit_cast(uint32_t, v), lane));
}

__device__ __forceinline__ double lane_f64(double v, int lane)
{
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint64_t lo = lane_u32(static_cast<uint32_t>(b), lane);
    const uint64_t hi = lane_u32(static_cast<uint32_t>(b >> 32), lane);
    return __builtin_bit_cast(double, lo | (hi << 32));
}

// Sum over the wave, returned uniformly (every lane must be active).
__device__ __forceinline__ double wave_sum_dpp(double v)
{
    v += dpp64<kDppXor1>(v);
    v += dpp64<kDppXor2>(v);
    v += dpp64<kDppHalfMirror>(v);
    v += dpp64<kDppMirror>(v);
    return (lane_f64(v, 0) + lane_f64(v, 16)) + (lane_f64(v, 32) + lane_f64(v, 48));
}

// f32 sum over the wave, uniform, as a fixed tree of six levels (relative
// error at most 6 2^-24 for non-negative terms).
__device__ __forceinline__ float wave_sum_dpp(float v)
{
    v += __builtin_bit_cast(float, dpp32<kDppXor1>(__builtin_bit_cast(uint32_t, v)));
    v += __builtin_bit_cast(float, dpp32<kDppXor2>(__builtin_bit_cast(uint32_t, v)));
    v += __builtin_bit_cast(float, dpp32<kDppHalfMirror>(__builtin_bit_cast(uint32_t, v)));
    v += __builtin_bit_cast(float, dpp32<kDppMirror>(__builtin_bit_cast(uint32_t, v)));
    return (lane_f32(v, 0) + lane_f32(v, 16)) + (lane_f32(v, 32) + lane_f32(v, 48));
}

// Maximum of the non-NaN values over the wave, uniform.
__device__ __forceinline__ float wave_max_dpp(float v)
{
    v = __builtin_fmaxf(v, __builtin_bit_cast(float, dpp32<kDppXor1>(__builtin_bit_cast(uint32_t, v))));
    v = __builtin_fmaxf(v, __builtin_bit_cast(float, dpp32<kDppXor2>(__builtin_bit_cast(uint32_t, v))));
    v = __builtin_fmaxf(v, __builtin_bit_cast(float, dpp32<kDppHalfMirror>(__builtin_bit_cast(uint32_t, v))));
    v = __builtin_fmaxf(v, __builtin_bit_cast(float, dpp32<kDppMirror>(__builtin_bit_cast(uint32_t, v))));
    return __builtin_fmaxf(__builtin_fmaxf(lane_f32(v, 0), lane_f32(v, 16)),
                           __builtin_fmaxf(lane_f32(v, 32), lane_f32(v, 48)));
}

__device__ __forceinline__ uint32_t wave_min_dpp(uint32_t v)
{
    v = min(v, dpp32<kDppXor1>(v));
    v = min(v, dpp32<kDppXor2>(v));
    v = min(v, dpp32<kDppHalfMirror>(v));
    v = min(v, dpp32<kDppMirror>(v));
    return min(min(lane_u32(v, 0), lane_u32(v, 16)), min(lane_u32(v, 32), lane_u32(v, 48)));
}

// (value, index) argmax over the wave, uniform: the largest value, and the
// lowest index among the lanes holding it.  Candidates are never NaN; a lane
// without one holds (-inf, 0xffffffff).
__device__ __forceinline__ void wave_argmax_dpp(float &bv, uint32_t &bi)
{
    const float m = wave_max_dpp(bv);
    bi = wave_min_dpp(bv == m ? bi : 0xffffffffu);
    bv = m;
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

// Raw buffer access: a descriptor over [base, base + bytes) in scalar
// registers.  A load whose offset is at or past `bytes` returns zeros and
// makes no memory access, so a lane-dependent tail needs no branch.  Word 3
// is the gfx9-family raw-buffer format (32-bit data, no swizzle).
typedef __amdgpu_buffer_rsrc_t BufRsrc;
typedef unsigned v4u __attribute__((ext_vector_type(4)));
__device__ __forceinline__ BufRsrc buffer_rsrc(const void *base, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), 0, static_cast<int>(bytes), 0x00020000);
}
// Cache-policy bits of a gfx950 buffer load: nt (bit 1) marks it streaming.
constexpr int kBufNt = 2;
__device__ __forceinline__ float4 ld_buf_nt(BufRsrc r, uint32_t offset)
{
    return __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(r, offset, 0, kBufNt));
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
