// getrows.hip -- gfx950 row gather (crates/emel-kernels/src/any/get_rows.rs):
// destination row r of a dense F32 [cols, rows] output receives source row
// indices[r] of batch (i1, i2), where (i0, i1, i2) is r decoded by the index
// extents (the reference's i2 / i1 / i0 loop order, :1453-1480).
//
// A pure gather: each output value is a copy or the decode of one packed
// block, so the bound is HBM (read the selected rows, write the output).
//   k_gr_row_*  one workgroup per destination row (and per 4096-float4 chunk
//               of very wide rows): the row's index is a uniform load, and
//               each lane produces one float4 of output per step: 128-bit
//               loads for F32 / F16 / BF16 rows, 16-bit (Q4_0, Q8_0) or
//               32-bit (Q4_K) loads for packed blocks.  Indices come from
//               device memory or from the launch arguments (host-checked).
//   k_rows_*    the fallback for misaligned or odd-width rows: one work item
//               per value (per block for packed rows), grid-stride.
#include "common.hpp"
#include "launch.hpp"
#include "libm_replica.hpp"

namespace emel {
namespace {

constexpr uint64_t kQBlock = 32;       // Q4_0 / Q8_0 values per block (quant.rs:13)
constexpr uint64_t kQ40Bytes = 18;     // quant.rs:15
constexpr uint64_t kQ80Bytes = 34;     // quant.rs:17
constexpr uint64_t kQ4KValues = 256;   // quant_more.rs:48
constexpr uint64_t kQ4KBytes = 144;    // quant_more.rs:38

// The index value and source batch of destination row r.
struct RowRef {
    uint64_t index, i1, i2;
};

__device__ __forceinline__ RowRef row_ref(const GetRowsArgs &a, uint64_t r)
{
    const uint64_t i0 = r % a.idx_ne[0];
    const uint64_t rem = r / a.idx_ne[0];
    const uint64_t i1 = rem % a.idx_ne[1];
    const uint64_t i2 = rem / a.idx_ne[1];
    const int32_t v = a.idx[static_cast<int64_t>(i0) * a.idx_st[0] + static_cast<int64_t>(i1) * a.idx_st[1] +
                            static_cast<int64_t>(i2) * a.idx_st[2]];
    return RowRef{static_cast<uint64_t>(static_cast<uint32_t>(v)), i1, i2};
}

// Index sources of the one-workgroup-per-row kernels: device memory read
// through the index strides, or the host-checked values in the arguments.
struct IdxDevice {
    __device__ __forceinline__ int32_t get(const GetRowsArgs &a, uint64_t, uint64_t i0, uint64_t i1,
                                           uint64_t i2) const
    {
        return a.idx[static_cast<int64_t>(i0) * a.idx_st[0] + static_cast<int64_t>(i1) * a.idx_st[1] +
                     static_cast<int64_t>(i2) * a.idx_st[2]];
    }
};

struct IdxArgs {
    IdxInline ix;
    __device__ __forceinline__ int32_t get(const GetRowsArgs &, uint64_t r, uint64_t, uint64_t, uint64_t) const
    {
        return ix.v[r];
    }
};

template <class IX>
__device__ __forceinline__ RowRef row_ref_ix(const GetRowsArgs &a, const IX &src, uint64_t r)
{
    const uint64_t i0 = r % a.idx_ne[0];
    const uint64_t rem = r / a.idx_ne[0];
    const uint64_t i1 = rem % a.idx_ne[1];
    const uint64_t i2 = rem / a.idx_ne[1];
    const int32_t v = src.get(a, r, i0, i1, i2);
    return RowRef{static_cast<uint64_t>(static_cast<uint32_t>(v)), i1, i2};
}

// Byte offset of a source row's start from nb[1..3] (F32, F32-bytes, F16, BF16).
__device__ __forceinline__ int64_t row_base(const GetRowsArgs &a, const RowRef &rr)
{
    return static_cast<int64_t>(rr.index) * a.src_st[1] + static_cast<int64_t>(rr.i1) * a.src_st[2] +
           static_cast<int64_t>(rr.i2) * a.src_st[3];
}

// f16_to_f32 of f16_matmul.rs:508-531: exact widening that keeps NaN payloads.
__device__ __forceinline__ uint32_t f16_bits_to_f32_bits(uint16_t h)
{
    const uint32_t sign = static_cast<uint32_t>(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu;
    const uint32_t f = h & 0x3ffu;
    if (e == 0) {
        if (f == 0) return sign;
        const uint32_t shift = static_cast<uint32_t>(__builtin_clz(f)) - 21u; // normalises bit 10
        return sign | ((127u - 14u - shift) << 23) | (((f << shift) & 0x3ffu) << 13);
    }
    if (e == 0x1fu) return sign | 0x7f800000u | (f << 13);
    return sign | ((e + 112u) << 23) | (f << 13);
}

// F32, every row base and the destination 16-byte aligned, cols % 4 == 0.
__global__ __launch_bounds__(kBlock) void k_rows_f32_vec(GetRowsArgs a, uint64_t items)
{
    const uint64_t per_row = a.cols / 4;
    const char *src = static_cast<const char *>(a.src);
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kBlock;
    for (uint64_t it = static_cast<uint64_t>(blockIdx.x) * kBlock + threadIdx.x; it < items; it += stride) {
        const uint64_t r = it / per_row;
        const uint64_t v = it - r * per_row;
        const RowRef rr = row_ref(a, r);
        const float4 x = *reinterpret_cast<const float4 *>(src + row_base(a, rr) + 16 * static_cast<int64_t>(v));
        reinterpret_cast<float4 *>(a.dst)[it] = x;
    }
}

// F32 one value per item; BYTES reads each value byte-wise (OpGetRowsF32Bytes,
// or an F32 row base that is not 4-byte aligned).
template <bool BYTES>
__global__ __launch_bounds__(kBlock) void k_rows_f32(GetRowsArgs a, uint64_t items)
{
    const unsigned char *src = static_cast<const unsigned char *>(a.src);
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kBlock;
    for (uint64_t it = static_cast<uint64_t>(blockIdx.x) * kBlock + threadIdx.x; it < items; it += stride) {
        const uint64_t r = it / a.cols;
        const uint64_t c = it - r * a.cols;
        const RowRef rr = row_ref(a, r);
        const unsigned char *p = src + row_base(a, rr) + 4 * static_cast<int64_t>(c);
        uint32_t bits;
        if constexpr (BYTES) {
            bits = static_cast<uint32_t>(p[0]) | (static_cast<uint32_t>(p[1]) << 8) |
                   (static_cast<uint32_t>(p[2]) << 16) | (static_cast<uint32_t>(p[3]) << 24);
        } else {
            bits = *reinterpret_cast<const uint32_t *>(p);
        }
        reinterpret_cast<uint32_t *>(a.dst)[it] = bits;
    }
}

// F16 / BF16: the value at source coordinates (c, index, i1, i2) through the
// source's effective strides, widened exactly.
template <bool BF16>
__global__ __launch_bounds__(kBlock) void k_rows_half(GetRowsArgs a, uint64_t items)
{
    const unsigned char *src = static_cast<const unsigned char *>(a.src);
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kBlock;
    for (uint64_t it = static_cast<uint64_t>(blockIdx.x) * kBlock + threadIdx.x; it < items; it += stride) {
        const uint64_t r = it / a.cols;
        const uint64_t c = it - r * a.cols;
        const RowRef rr = row_ref(a, r);
        const uint16_t h =
            *reinterpret_cast<const uint16_t *>(src + row_base(a, rr) + static_cast<int64_t>(c) * a.src_st[0]);
        const uint32_t bits = BF16 ? static_cast<uint32_t>(h) << 16 : f16_bits_to_f32_bits(h);
        reinterpret_cast<uint32_t *>(a.dst)[it] = bits;
    }
}

__device__ __forceinline__ float ld_f16(const unsigned char *p)
{
    return emel_fp16_to_f32(static_cast<uint16_t>(p[0] | (p[1] << 8)));
}

__device__ __forceinline__ void st8(float *o, const float *v)
{
    // 8 consecutive outputs as two float4 when aligned (always: blocks start
    // at multiples of 32 values of a 16-byte aligned dense row).
    reinterpret_cast<float4 *>(o)[0] = make_float4(v[0], v[1], v[2], v[3]);
    reinterpret_cast<float4 *>(o)[1] = make_float4(v[4], v[5], v[6], v[7]);
}

// Q4_0 / Q8_0: one 32-value block per item (quant.rs:106-134, :178-205).
template <bool Q8>
__global__ __launch_bounds__(kBlock) void k_rows_q8(GetRowsArgs a, uint64_t items, bool vec_out)
{
    constexpr uint64_t kBytes = Q8 ? kQ80Bytes : kQ40Bytes;
    const unsigned char *src = static_cast<const unsigned char *>(a.src);
    const uint64_t blocks = a.cols / kQBlock;
    const uint64_t row_bytes = blocks * kBytes;
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kBlock;
    for (uint64_t it = static_cast<uint64_t>(blockIdx.x) * kBlock + threadIdx.x; it < items; it += stride) {
        const uint64_t r = it / blocks;
        const uint64_t b = it - r * blocks;
        const RowRef rr = row_ref(a, r);
        const uint64_t row = (rr.i2 * a.src_ne[2] + rr.i1) * a.src_ne[1] + rr.index;
        const unsigned char *blk = src + row * row_bytes + b * kBytes;
        const float scale = ld_f16(blk);
        float out[kQBlock];
        if constexpr (Q8) {
#pragma unroll
            for (int j = 0; j < 32; ++j) out[j] = static_cast<float>(static_cast<int8_t>(blk[2 + j])) * scale;
        } else {
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const uint32_t q = blk[2 + j];
                out[j] = (static_cast<float>(q & 0x0fu) - 8.0f) * scale;
                out[j + 16] = (static_cast<float>(q >> 4) - 8.0f) * scale;
            }
        }
        float *o = a.dst + r * a.cols + b * kQBlock;
        if (vec_out) {
#pragma unroll
            for (int j = 0; j < 32; j += 8) st8(o + j, out + j);
        } else {
#pragma unroll
            for (int j = 0; j < 32; ++j) o[j] = out[j];
        }
    }
}

// Q4_K scale/min of sub-block j (quant_more.rs:952-961).
__device__ __forceinline__ void q4k_scale_min(int j, const unsigned char *s, uint32_t &sc, uint32_t &mn)
{
    if (j < 4) {
        sc = s[j] & 0x3fu;
        mn = s[j + 4] & 0x3fu;
    } else {
        sc = (s[j + 4] & 0x0fu) | ((s[j - 4] >> 6) << 4);
        mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

// Q4_K: one 64-value quarter of a 256-value block per item
// (quant_more.rs:438-468): low nibbles scaled by sub-block 2q, high nibbles
// by 2q+1, each value d*sc*q - dmin*m with three separate roundings.
__global__ __launch_bounds__(kBlock) void k_rows_q4k(GetRowsArgs a, uint64_t items, bool vec_out)
{
    const unsigned char *src = static_cast<const unsigned char *>(a.src);
    const uint64_t quarters = a.cols / 64;
    const uint64_t row_bytes = (a.cols / kQ4KValues) * kQ4KBytes;
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kBlock;
    for (uint64_t it = static_cast<uint64_t>(blockIdx.x) * kBlock + threadIdx.x; it < items; it += stride) {
        const uint64_t r = it / quarters;
        const uint64_t qi = it - r * quarters;
        const uint64_t b = qi / 4;
        const int q = static_cast<int>(qi % 4);
        const RowRef rr = row_ref(a, r);
        const uint64_t row = (rr.i2 * a.src_ne[2] + rr.i1) * a.src_ne[1] + rr.index;
        const unsigned char *blk = src + row * row_bytes + b * kQ4KBytes;
        const float d = ld_f16(blk);
        const float dmin = ld_f16(blk + 2);
        uint32_t sa, ma, sb, mb;
        q4k_scale_min(2 * q, blk + 4, sa, ma);
        q4k_scale_min(2 * q + 1, blk + 4, sb, mb);
        const float d0 = d * static_cast<float>(sa);
        const float d1 = d * static_cast<float>(sb);
        const float m0 = dmin * static_cast<float>(ma);
        const float m1 = dmin * static_cast<float>(mb);
        const unsigned char *qs = blk + 16 + 32 * q;
        float *o = a.dst + r * a.cols + b * kQ4KValues + 64 * static_cast<uint64_t>(q);
        for (int h = 0; h < 32; h += 8) {
            float lo[8], hi[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint32_t p = qs[h + j];
                lo[j] = d0 * static_cast<float>(p & 0x0fu) - m0;
                hi[j] = d1 * static_cast<float>(p >> 4) - m1;
            }
            if (vec_out) {
                st8(o + h, lo);
                st8(o + 32 + h, hi);
            } else {
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    o[h + j] = lo[j];
                    o[32 + h + j] = hi[j];
                }
            }
        }
    }
}

// ---- one workgroup per destination row ----------------------------------------------
// The row's index is then a uniform (scalar) load, and the row streams with
// one 128-bit store per lane per step.  blockIdx.y splits very wide rows
// into chunks of kGrChunk float4.

constexpr uint32_t kGrBlock = 256;
constexpr uint64_t kGrChunk = 4096; // float4 per (row, chunk) workgroup

typedef unsigned int v4u __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint4 ld_nt_u4(const void *p)
{
    const v4u v = __builtin_nontemporal_load(reinterpret_cast<const v4u *>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

// hardware widening (exact for every non-NaN half), NaN payloads kept as the
// reference's bit-level conversion does
__device__ __forceinline__ float f16_exact(uint32_t h)
{
    const float w = hw_fp16_to_f32(static_cast<uint16_t>(h));
    const bool nan = (h & 0x7c00u) == 0x7c00u && (h & 0x3ffu) != 0;
    return nan ? bits_to_f32(((h & 0x8000u) << 16) | 0x7f800000u | ((h & 0x3ffu) << 13)) : w;
}

struct RowSpan {
    uint64_t r, v0, v1; // destination row, float4 range [v0, v1)
};

__device__ __forceinline__ RowSpan row_span(uint64_t n4)
{
    const uint64_t v0 = static_cast<uint64_t>(blockIdx.y) * kGrChunk;
    const uint64_t v1 = v0 + kGrChunk < n4 ? v0 + kGrChunk : n4;
    return RowSpan{blockIdx.x, v0, v1};
}

// F32, 16-byte aligned row bases, cols % 4 == 0.
template <class IX>
__global__ __launch_bounds__(kGrBlock) void k_gr_row_f32(GetRowsArgs a, IX ix)
{
    const uint64_t n4 = a.cols / 4;
    const RowSpan sp = row_span(n4);
    const RowRef rr = row_ref_ix(a, ix, sp.r);
    const float4 *src = reinterpret_cast<const float4 *>(static_cast<const char *>(a.src) + row_base(a, rr));
    float4 *dst = reinterpret_cast<float4 *>(a.dst) + sp.r * n4;
    uint64_t v = sp.v0 + threadIdx.x;
    for (; v + 3 * kGrBlock < sp.v1; v += 4 * kGrBlock) {
        const float4 x0 = ld_nt(src + v), x1 = ld_nt(src + v + kGrBlock);
        const float4 x2 = ld_nt(src + v + 2 * kGrBlock), x3 = ld_nt(src + v + 3 * kGrBlock);
        dst[v] = x0;
        dst[v + kGrBlock] = x1;
        dst[v + 2 * kGrBlock] = x2;
        dst[v + 3 * kGrBlock] = x3;
    }
    for (; v < sp.v1; v += kGrBlock) dst[v] = ld_nt(src + v);
}

// F16 / BF16 with unit element stride, 16-byte aligned row bases, cols % 8 == 0:
// eight halves per lane per step, widened, two 128-bit stores.
template <bool BF16, class IX>
__global__ __launch_bounds__(kGrBlock) void k_gr_row_half(GetRowsArgs a, IX ix)
{
    const uint64_t n4 = a.cols / 4;
    const RowSpan sp = row_span(n4);
    const RowRef rr = row_ref_ix(a, ix, sp.r);
    const char *src = static_cast<const char *>(a.src) + row_base(a, rr);
    float4 *dst = reinterpret_cast<float4 *>(a.dst) + sp.r * n4;
    // the chunk bounds are even numbers of float4, so pairs never straddle one
    for (uint64_t p = sp.v0 / 2 + threadIdx.x; 2 * p < sp.v1; p += kGrBlock) {
        const uint4 h = ld_nt_u4(src + 16 * p);
        const uint32_t w[4] = {h.x, h.y, h.z, h.w};
        float f[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if constexpr (BF16) {
                f[2 * i] = bits_to_f32(w[i] << 16);
                f[2 * i + 1] = bits_to_f32(w[i] & 0xffff0000u);
            } else {
                f[2 * i] = f16_exact(w[i] & 0xffffu);
                f[2 * i + 1] = f16_exact(w[i] >> 16);
            }
        }
        dst[2 * p] = make_float4(f[0], f[1], f[2], f[3]);
        dst[2 * p + 1] = make_float4(f[4], f[5], f[6], f[7]);
    }
}

__device__ __forceinline__ uint32_t ld_u32_via_u16(const unsigned char *p)
{
    const uint16_t *q = reinterpret_cast<const uint16_t *>(p);
    return static_cast<uint32_t>(q[0]) | (static_cast<uint32_t>(q[1]) << 16);
}

// Packed rows, one float4 of output per lane: Q8_0 / Q4_0 blocks give 8
// float4 (lane j of a block reads quant bytes 4(j&3).. with two 16-bit loads,
// the table base being 2-byte aligned); Q4_K blocks give 64 float4 (32-bit
// loads, the table base being 4-byte aligned).
template <RowSrc K, class IX>
__global__ __launch_bounds__(kGrBlock) void k_gr_row_q(GetRowsArgs a, IX ix)
{
    const uint64_t n4 = a.cols / 4;
    const RowSpan sp = row_span(n4);
    const RowRef rr = row_ref_ix(a, ix, sp.r);
    const uint64_t row = (rr.i2 * a.src_ne[2] + rr.i1) * a.src_ne[1] + rr.index;
    float4 *dst = reinterpret_cast<float4 *>(a.dst) + sp.r * n4;
    if constexpr (K == RowSrc::Q8_0 || K == RowSrc::Q4_0) {
        constexpr uint64_t kBytes = K == RowSrc::Q8_0 ? kQ80Bytes : kQ40Bytes;
        const unsigned char *base = static_cast<const unsigned char *>(a.src) + row * (a.cols / kQBlock) * kBytes;
        for (uint64_t v = sp.v0 + threadIdx.x; v < sp.v1; v += kGrBlock) {
            const uint64_t b = v / 8;
            const uint32_t j = static_cast<uint32_t>(v % 8);
            const unsigned char *blk = base + b * kBytes;
            const float d = hw_fp16_to_f32(*reinterpret_cast<const uint16_t *>(blk));
            float4 o;
            if constexpr (K == RowSrc::Q8_0) {
                const uint32_t q = ld_u32_via_u16(blk + 2 + 4 * j);
                o.x = static_cast<float>(static_cast<int8_t>(q & 0xffu)) * d;
                o.y = static_cast<float>(static_cast<int8_t>((q >> 8) & 0xffu)) * d;
                o.z = static_cast<float>(static_cast<int8_t>((q >> 16) & 0xffu)) * d;
                o.w = static_cast<float>(static_cast<int8_t>(q >> 24)) * d;
            } else {
                const uint32_t q = ld_u32_via_u16(blk + 2 + 4 * (j & 3u));
                const uint32_t s = j < 4 ? 0u : 4u; // low nibbles for outputs 0..15, high for 16..31
                o.x = (static_cast<float>((q >> s) & 0xfu) - 8.0f) * d;
                o.y = (static_cast<float>((q >> (8 + s)) & 0xfu) - 8.0f) * d;
                o.z = (static_cast<float>((q >> (16 + s)) & 0xfu) - 8.0f) * d;
                o.w = (static_cast<float>((q >> (24 + s)) & 0xfu) - 8.0f) * d;
            }
            dst[v] = o;
        }
    } else {
        const unsigned char *base = static_cast<const unsigned char *>(a.src) + row * (a.cols / kQ4KValues) * kQ4KBytes;
        for (uint64_t v = sp.v0 + threadIdx.x; v < sp.v1; v += kGrBlock) {
            const uint64_t b = v / 64;
            const uint32_t k = static_cast<uint32_t>(v % 64);
            const uint32_t q = k / 16, t = k % 16;
            const unsigned char *blk = base + b * kQ4KBytes;
            const uint32_t *w = reinterpret_cast<const uint32_t *>(blk);
            const uint32_t hdr = w[0];
            const uint32_t sw[3] = {w[1], w[2], w[3]}; // the 12 scale bytes
            auto sbyte = [&](uint32_t i) { return (sw[i >> 2] >> (8 * (i & 3u))) & 0xffu; };
            const uint32_t sj = 2 * q + (t < 8 ? 0u : 1u);
            uint32_t sc, mn;
            if (sj < 4) {
                sc = sbyte(sj) & 0x3fu;
                mn = sbyte(sj + 4) & 0x3fu;
            } else {
                sc = (sbyte(sj + 4) & 0x0fu) | ((sbyte(sj - 4) >> 6) << 4);
                mn = (sbyte(sj + 4) >> 4) | ((sbyte(sj) >> 6) << 4);
            }
            const float dx = hw_fp16_to_f32(static_cast<uint16_t>(hdr & 0xffffu)) * static_cast<float>(sc);
            const float mx = hw_fp16_to_f32(static_cast<uint16_t>(hdr >> 16)) * static_cast<float>(mn);
            const uint32_t qw = w[(16 + 32 * q + 4 * (t & 7u)) / 4];
            const uint32_t s = t < 8 ? 0u : 4u;
            float4 o;
            o.x = dx * static_cast<float>((qw >> s) & 0xfu) - mx;
            o.y = dx * static_cast<float>((qw >> (8 + s)) & 0xfu) - mx;
            o.z = dx * static_cast<float>((qw >> (16 + s)) & 0xfu) - mx;
            o.w = dx * static_cast<float>((qw >> (24 + s)) & 0xfu) - mx;
            dst[v] = o;
        }
    }
}

uint32_t grid_for(uint64_t items)
{
    uint64_t blocks = (items + kBlock - 1) / kBlock;
    if (blocks > 65536) blocks = 65536;
    if (blocks == 0) blocks = 1;
    return static_cast<uint32_t>(blocks);
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

enum class RowKernel { None, F32, F16, Bf16, Q4_0, Q8_0, Q4K };

// The one-workgroup-per-row kernel for these arguments, if its alignment
// and size conditions hold.
RowKernel row_kernel(const GetRowsArgs &a)
{
    const uint64_t n4 = a.cols / 4;
    const uint64_t chunks = (n4 + kGrChunk - 1) / kGrChunk;
    if (!(a.rows >= 1 && a.rows <= 0x7fffffffull && chunks >= 1 && chunks <= 65535 && a.cols % 4 == 0 &&
          aligned16(a.dst)))
        return RowKernel::None;
    auto rows16 = [&]() {
        if (!aligned16(a.src)) return false;
        for (int d = 1; d < 4; ++d)
            if (a.src_st[d] % 16 != 0) return false;
        return true;
    };
    const uintptr_t sp = reinterpret_cast<uintptr_t>(a.src);
    switch (a.kind) {
    case RowSrc::F32: return rows16() ? RowKernel::F32 : RowKernel::None;
    case RowSrc::F16:
    case RowSrc::Bf16:
        if (a.cols % 8 == 0 && a.src_st[0] == 2 && rows16())
            return a.kind == RowSrc::F16 ? RowKernel::F16 : RowKernel::Bf16;
        return RowKernel::None;
    case RowSrc::Q4_0: return (sp & 1u) == 0 ? RowKernel::Q4_0 : RowKernel::None;
    case RowSrc::Q8_0: return (sp & 1u) == 0 ? RowKernel::Q8_0 : RowKernel::None;
    case RowSrc::Q4K: return (sp & 3u) == 0 ? RowKernel::Q4K : RowKernel::None;
    default: return RowKernel::None;
    }
}

template <class IX>
hipError_t launch_row_kernel(RowKernel k, const GetRowsArgs &a, const IX &ix, hipStream_t s)
{
    const uint64_t chunks = (a.cols / 4 + kGrChunk - 1) / kGrChunk;
    const dim3 grid(static_cast<uint32_t>(a.rows), static_cast<uint32_t>(chunks));
    switch (k) {
    case RowKernel::F32: k_gr_row_f32<IX><<<grid, kGrBlock, 0, s>>>(a, ix); break;
    case RowKernel::F16: k_gr_row_half<false, IX><<<grid, kGrBlock, 0, s>>>(a, ix); break;
    case RowKernel::Bf16: k_gr_row_half<true, IX><<<grid, kGrBlock, 0, s>>>(a, ix); break;
    case RowKernel::Q4_0: k_gr_row_q<RowSrc::Q4_0, IX><<<grid, kGrBlock, 0, s>>>(a, ix); break;
    case RowKernel::Q8_0: k_gr_row_q<RowSrc::Q8_0, IX><<<grid, kGrBlock, 0, s>>>(a, ix); break;
    case RowKernel::Q4K: k_gr_row_q<RowSrc::Q4K, IX><<<grid, kGrBlock, 0, s>>>(a, ix); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

} // namespace

bool get_rows_row_kernels(const GetRowsArgs &a) { return row_kernel(a) != RowKernel::None; }

hipError_t launch_get_rows(const GetRowsArgs &a, const IdxInline *inline_idx, hipStream_t s)
{
    if (a.rows == 0 || a.cols == 0) return hipSuccess;
    const RowKernel rk = row_kernel(a);
    if (inline_idx) {
        if (rk == RowKernel::None || a.rows > kInlineIndices) return hipErrorInvalidValue;
        return launch_row_kernel(rk, a, IdxArgs{*inline_idx}, s);
    }
    if (rk != RowKernel::None) return launch_row_kernel(rk, a, IdxDevice{}, s);
    const bool dst16 = aligned16(a.dst);

    switch (a.kind) {
    case RowSrc::F32: {
        // Every row base 16-byte aligned: the base pointer and the strides of
        // every dim that selects rows.
        bool vec = a.cols % 4 == 0 && dst16 && aligned16(a.src);
        for (int d = 1; d < 4; ++d)
            if (a.src_st[d] % 16 != 0) vec = false;
        if (vec) {
            const uint64_t items = a.rows * (a.cols / 4);
            k_rows_f32_vec<<<grid_for(items), kBlock, 0, s>>>(a, items);
        } else {
            bool word = (reinterpret_cast<uintptr_t>(a.src) & 3u) == 0;
            for (int d = 1; d < 4; ++d)
                if (a.src_st[d] % 4 != 0) word = false;
            const uint64_t items = a.rows * a.cols;
            if (word) k_rows_f32<false><<<grid_for(items), kBlock, 0, s>>>(a, items);
            else k_rows_f32<true><<<grid_for(items), kBlock, 0, s>>>(a, items);
        }
        break;
    }
    case RowSrc::F32Bytes: {
        const uint64_t items = a.rows * a.cols;
        k_rows_f32<true><<<grid_for(items), kBlock, 0, s>>>(a, items);
        break;
    }
    case RowSrc::F16:
    case RowSrc::Bf16: {
        const uint64_t items = a.rows * a.cols;
        if (a.kind == RowSrc::F16) k_rows_half<false><<<grid_for(items), kBlock, 0, s>>>(a, items);
        else k_rows_half<true><<<grid_for(items), kBlock, 0, s>>>(a, items);
        break;
    }
    case RowSrc::Q4_0:
    case RowSrc::Q8_0: {
        const uint64_t items = a.rows * (a.cols / kQBlock);
        if (a.kind == RowSrc::Q8_0) k_rows_q8<true><<<grid_for(items), kBlock, 0, s>>>(a, items, dst16);
        else k_rows_q8<false><<<grid_for(items), kBlock, 0, s>>>(a, items, dst16);
        break;
    }
    case RowSrc::Q4K: {
        const uint64_t items = a.rows * (a.cols / 64);
        k_rows_q4k<<<grid_for(items), kBlock, 0, s>>>(a, items, dst16);
        break;
    }
    default:
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

} // namespace emel
