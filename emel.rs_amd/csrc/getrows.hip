// getrows.hip -- gfx950 row gather (crates/emel-kernels/src/any/get_rows.rs):
// destination row r of a dense F32 [cols, rows] output receives source row
// indices[r] of batch (i1, i2), where (i0, i1, i2) is r decoded by the index
// extents (the reference's i2 / i1 / i0 loop order, :1453-1480).
//
// A pure gather: each output value is a copy or the decode of one packed
// block, so the bound is HBM (read the selected rows, write the output).
// One work item per output float4 (F32), per output value (F32 with a
// misaligned row, F16, BF16), per 32-value block (Q4_0, Q8_0) or per
// 64-value quarter block (Q4_K); items are walked grid-stride.
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

uint32_t grid_for(uint64_t items)
{
    uint64_t blocks = (items + kBlock - 1) / kBlock;
    if (blocks > 65536) blocks = 65536;
    if (blocks == 0) blocks = 1;
    return static_cast<uint32_t>(blocks);
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

} // namespace

hipError_t launch_get_rows(const GetRowsArgs &a, hipStream_t s)
{
    if (a.rows == 0 || a.cols == 0) return hipSuccess;
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
