// generic.hip -- gfx950 kernels for the generic wire envelope's maintained
// F32 routes that the typed kernels do not already cover
// (crates/emel-kernels/src/any/generic.rs:1264-2055).
//
// Every route here is a sequential loop in the reference whose rounding
// depends on the order of its additions, so each kernel but k_gen_norm
// gives one lane the reference's whole loop for its unit of independent
// work, in the reference's order:
//   k_gen_rows      one lane per row: cumsum, soft_max_back, rms_norm_back,
//                   and norm / rms_norm rows narrower than a wave (soft_max
//                   uses the typed strided path's exact sequential-sum
//                   kernel);
//   k_gen_norm      a workgroup per row for norm and rms_norm rows of 64 or
//                   more columns that the typed row kernels cannot take
//                   (those run vectorisable rows with the generic arithmetic);
//                   both sum in f64 as a fixed-order tree: within rms_norm's
//                   1e-5 tolerance, the one route here not in the
//                   reference's order;
//   k_gen_ord       one lane per destination element: fill, arange, diag,
//                   diag_mask_inf/zero, concat, repeat_back (the source
//                   elements of one target summed in source-ordinal order);
//   k_l2_sum        one lane for the whole tensor (l2_norm's f32 sum), then
//                   k_l2_apply over every element;
//   k_count_*       an exact integer count (count_equal's f32 counter
//                   saturates at 2^24, which min() reproduces);
//   k_mm_*          one lane per output element (mul_mat F32 / F16) or per
//                   row (mul_mat_argmax), the inner products in order.
// Operands are addressed through their own extents and element strides, the
// reference's coordinates_for_index/byte_offset (generic.rs:896-933), walked
// incrementally along a row instead of re-decoded per element.
#include "common.hpp"
#include "launch.hpp"
#include "libm_replica.hpp"

namespace emel {
namespace {

constexpr int kRowBlock = 64; // one wave per workgroup spreads few rows over more CUs

// Ordinal -> element offset, advanced one ordinal at a time.
struct Walk {
    uint64_t c[4];
    int64_t off;

    __device__ __forceinline__ void init(const GView &v, uint64_t k)
    {
        off = 0;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            c[d] = k % v.ne[d];
            k /= v.ne[d];
            off += static_cast<int64_t>(c[d]) * v.st[d];
        }
    }

    __device__ __forceinline__ void next(const GView &v)
    {
        off += v.st[0];
        if (++c[0] < v.ne[0]) return;
        c[0] = 0;
        off += v.st[1] - static_cast<int64_t>(v.ne[0]) * v.st[0];
        if (++c[1] < v.ne[1]) return;
        c[1] = 0;
        off += v.st[2] - static_cast<int64_t>(v.ne[1]) * v.st[1];
        if (++c[2] < v.ne[2]) return;
        c[2] = 0;
        off += v.st[3] - static_cast<int64_t>(v.ne[2]) * v.st[2];
        ++c[3];
    }
};

__device__ __forceinline__ int64_t coords_offset(const GView &v, const uint64_t *c)
{
    int64_t off = 0;
#pragma unroll
    for (int d = 0; d < 4; ++d) off += static_cast<int64_t>(c[d]) * v.st[d];
    return off;
}

// ---- one lane per row -------------------------------------------------------------

template <GenRow OP>
__global__ __launch_bounds__(kRowBlock) void k_gen_rows(GenRowArgs a)
{
    const uint64_t r = static_cast<uint64_t>(blockIdx.x) * kRowBlock + threadIdx.x;
    if (r >= a.rows) return;
    const float *x = static_cast<const float *>(a.x.data);
    const float *g = static_cast<const float *>(a.g.data);
    float *y = static_cast<float *>(a.y.data);
    const uint64_t w = a.width;
    Walk x0, y0;
    x0.init(a.x, r * w);
    y0.init(a.y, r * w);

    if constexpr (OP == GenRow::Cumsum) { // generic.rs:1585-1609
        float sum = 0.0f;
        for (uint64_t c = 0; c < w; ++c) {
            sum += x[x0.off];
            y[y0.off] = sum;
            x0.next(a.x);
            y0.next(a.y);
        }
    } else if constexpr (OP == GenRow::Norm || OP == GenRow::RmsNorm) { // generic.rs:1988-2055
        Walk xi = x0;
        double sum = 0.0;
        for (uint64_t c = 0; c < w; ++c) {
            const float v = x[xi.off];
            sum += OP == GenRow::RmsNorm ? static_cast<double>(v * v) : static_cast<double>(v);
            xi.next(a.x);
        }
        const float mean = static_cast<float>(sum / static_cast<double>(w));
        double var = 0.0;
        if constexpr (OP == GenRow::Norm) {
            xi = x0;
            for (uint64_t c = 0; c < w; ++c) {
                const float centered = x[xi.off] - mean;
                var += static_cast<double>(centered * centered);
                xi.next(a.x);
            }
            var /= static_cast<double>(w);
        }
        const double base = OP == GenRow::RmsNorm ? static_cast<double>(mean) : var;
        const float scale = static_cast<float>(1.0 / __builtin_sqrt(base + static_cast<double>(a.eps)));
        xi = x0;
        Walk yi = y0;
        for (uint64_t c = 0; c < w; ++c) {
            const float v = x[xi.off];
            y[yi.off] = OP == GenRow::RmsNorm ? v * scale : (v - mean) * scale;
            xi.next(a.x);
            yi.next(a.y);
        }
    } else if constexpr (OP == GenRow::SoftMaxBack) { // generic.rs:1849-1881
        Walk g0;
        g0.init(a.g, r * w);
        Walk xi = x0, gi = g0;
        float dot = 0.0f;
        for (uint64_t c = 0; c < w; ++c) {
            dot = __builtin_fmaf(x[xi.off], g[gi.off], dot);
            xi.next(a.x);
            gi.next(a.g);
        }
        xi = x0;
        gi = g0;
        Walk yi = y0;
        for (uint64_t c = 0; c < w; ++c) {
            y[yi.off] = x[xi.off] * (g[gi.off] - dot);
            xi.next(a.x);
            gi.next(a.g);
            yi.next(a.y);
        }
    } else { // RmsNormBack, generic.rs:1883-1926
        Walk g0;
        g0.init(a.g, r * w);
        const double wd = static_cast<double>(w);
        Walk xi = x0;
        double sum = 0.0;
        for (uint64_t c = 0; c < w; ++c) {
            const float v = x[xi.off];
            sum += static_cast<double>(v * v);
            xi.next(a.x);
        }
        const double inv = 1.0 / __builtin_sqrt(sum / wd + static_cast<double>(a.eps));
        xi = x0;
        Walk gi = g0;
        double dot = 0.0;
        for (uint64_t c = 0; c < w; ++c) {
            dot += static_cast<double>(g[gi.off] * x[xi.off]);
            xi.next(a.x);
            gi.next(a.g);
        }
        xi = x0;
        gi = g0;
        Walk yi = y0;
        for (uint64_t c = 0; c < w; ++c) {
            const double xv = static_cast<double>(x[xi.off]);
            const double dy = static_cast<double>(g[gi.off]);
            y[yi.off] = static_cast<float>(dy * inv - xv * inv * inv * inv * dot / wd);
            xi.next(a.x);
            gi.next(a.g);
            yi.next(a.y);
        }
    }
}

// ---- one lane per destination element ------------------------------------------

template <GenOrd OP>
__global__ __launch_bounds__(kBlock) void k_gen_ord(GenOrdArgs a, uint64_t count)
{
    const float *x = static_cast<const float *>(a.a.data);
    const float *xb = static_cast<const float *>(a.b.data);
    float *y = static_cast<float *>(a.y.data);
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kBlock;
    for (uint64_t k = static_cast<uint64_t>(blockIdx.x) * kBlock + threadIdx.x; k < count; k += stride) {
        uint64_t c[4];
        uint64_t rem = k;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            c[d] = rem % a.y.ne[d];
            rem /= a.y.ne[d];
        }
        const int64_t oo = coords_offset(a.y, c);
        float v;
        if constexpr (OP == GenOrd::Fill) { // generic.rs:1736-1750
            v = a.p0;
        } else if constexpr (OP == GenOrd::Arange) { // generic.rs:1752-1770
            v = __builtin_fmaf(static_cast<float>(k), a.p1, a.p0);
        } else if constexpr (OP == GenOrd::Diag) { // generic.rs:1772-1793: dst (column, row)
            v = c[0] == c[1] ? x[static_cast<int64_t>(c[1]) * a.a.st[0]] : 0.0f;
        } else if constexpr (OP == GenOrd::DiagMaskInf || OP == GenOrd::DiagMaskZero) { // :1795-1820
            if (c[0] > c[1] + a.n_past)
                v = OP == GenOrd::DiagMaskInf ? -__builtin_inff() : 0.0f;
            else
                v = x[coords_offset(a.a, c)];
        } else if constexpr (OP == GenOrd::Concat) { // generic.rs:1703-1734
            const uint32_t ax = a.axis;
            if (c[ax] < a.a.ne[ax]) {
                v = x[coords_offset(a.a, c)];
            } else {
                c[ax] -= a.a.ne[ax];
                v = xb[coords_offset(a.b, c)];
            }
        } else { // RepeatBack, generic.rs:1667-1701
            // The source elements that map onto target t are t + m * T for
            // every multiple m; increasing source ordinal is lexicographic
            // (m3, m2, m1, m0).
            uint64_t q[4];
#pragma unroll
            for (int d = 0; d < 4; ++d) q[d] = a.a.ne[d] / a.y.ne[d];
            float acc = 0.0f;
            for (uint64_t m3 = 0; m3 < q[3]; ++m3)
                for (uint64_t m2 = 0; m2 < q[2]; ++m2)
                    for (uint64_t m1 = 0; m1 < q[1]; ++m1) {
                        const int64_t base = static_cast<int64_t>(c[1] + m1 * a.y.ne[1]) * a.a.st[1] +
                                             static_cast<int64_t>(c[2] + m2 * a.y.ne[2]) * a.a.st[2] +
                                             static_cast<int64_t>(c[3] + m3 * a.y.ne[3]) * a.a.st[3];
                        for (uint64_t m0 = 0; m0 < q[0]; ++m0)
                            acc = acc + x[base + static_cast<int64_t>(c[0] + m0 * a.y.ne[0]) * a.a.st[0]];
                    }
            v = acc;
        }
        y[oo] = v;
    }
}

// ---- l2_norm: one sequential f32 sum, then a scale pass (generic.rs:1822-1847) ----

__global__ __launch_bounds__(64) void k_l2_sum(GView xv, uint64_t count, float *scale_out)
{
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    const float *x = static_cast<const float *>(xv.data);
    float sum = 0.0f;
    Walk w;
    w.init(xv, 0);
    for (uint64_t k = 0; k < count; ++k) {
        const float v = x[w.off];
        sum += v * v;
        w.next(xv);
    }
    scale_out[0] = 1.0f / __builtin_sqrtf(sum);
    scale_out[1] = sum;
}

__global__ __launch_bounds__(kBlock) void k_l2_apply(GView xv, GView yv, uint64_t count, const float *scale)
{
    const float *x = static_cast<const float *>(xv.data);
    float *y = static_cast<float *>(yv.data);
    const float s = scale[0];
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kBlock;
    for (uint64_t k = static_cast<uint64_t>(blockIdx.x) * kBlock + threadIdx.x; k < count; k += stride) {
        Walk wx, wy;
        wx.init(xv, k);
        wy.init(yv, k);
        y[wy.off] = x[wx.off] * s;
    }
}

// ---- count_equal (generic.rs:1928-1946) -------------------------------------------

constexpr uint32_t kCountBlocks = 1024;

__global__ __launch_bounds__(kBlock) void k_count_partial(GView av, GView bv, uint64_t count,
                                                          unsigned long long *partial)
{
    __shared__ unsigned long long part[kBlock / kWave];
    const uint32_t *pa = static_cast<const uint32_t *>(av.data);
    const uint32_t *pb = static_cast<const uint32_t *>(bv.data);
    unsigned long long n = 0;
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kBlock;
    for (uint64_t k = static_cast<uint64_t>(blockIdx.x) * kBlock + threadIdx.x; k < count; k += stride) {
        Walk wa, wb;
        wa.init(av, k);
        wb.init(bv, k);
        n += pa[wa.off] == pb[wb.off] ? 1ull : 0ull;
    }
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) n += __shfl_xor(n, off, kWave);
    if (threadIdx.x % kWave == 0) part[threadIdx.x / kWave] = n;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long t = 0;
        for (int i = 0; i < kBlock / kWave; ++i) t += part[i];
        partial[blockIdx.x] = t;
    }
}

__global__ __launch_bounds__(kBlock) void k_count_final(const unsigned long long *partial, uint32_t n, float *dst)
{
    __shared__ unsigned long long part[kBlock / kWave];
    unsigned long long t = 0;
    for (uint32_t i = threadIdx.x; i < n; i += kBlock) t += partial[i];
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) t += __shfl_xor(t, off, kWave);
    if (threadIdx.x % kWave == 0) part[threadIdx.x / kWave] = t;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long total = 0;
        for (int i = 0; i < kBlock / kWave; ++i) total += part[i];
        // The reference counts in f32: 2^24 + 1 rounds back to 2^24.
        dst[0] = static_cast<float>(total < (1ull << 24) ? total : (1ull << 24));
    }
}

// ---- mul_mat (generic.rs:1422-1450, :1482-1515) ------------------------------------

// F32: lhs [k, m], rhs [n, k], dst [n, m]; dst(col, row) = sum over inner of
// lhs(inner, row) * rhs(col, inner), one fused multiply-add per step.
__global__ __launch_bounds__(kBlock) void k_mm_f32(GenMatArgs a)
{
    const float *l = static_cast<const float *>(a.lhs.data);
    const float *r = static_cast<const float *>(a.rhs.data);
    float *y = static_cast<float *>(a.y.data);
    const uint64_t total = a.m * a.n;
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kBlock;
    for (uint64_t t = static_cast<uint64_t>(blockIdx.x) * kBlock + threadIdx.x; t < total; t += stride) {
        const uint64_t row = t / a.n;
        const uint64_t col = t - row * a.n;
        const float *lp = l + static_cast<int64_t>(row) * a.lhs.st[1];
        const float *rp = r + static_cast<int64_t>(col) * a.rhs.st[0];
        float v = 0.0f;
        for (uint64_t i = 0; i < a.k; ++i)
            v = __builtin_fmaf(lp[static_cast<int64_t>(i) * a.lhs.st[0]], rp[static_cast<int64_t>(i) * a.rhs.st[1]], v);
        y[static_cast<int64_t>(col) * a.y.st[0] + static_cast<int64_t>(row) * a.y.st[1]] = v;
    }
}

// F16: dense lhs [k, m] and rhs [k, n]; dst [m, n] f32 gets the f64 sum of
// the f32 products of the widened halves.
__global__ __launch_bounds__(kBlock) void k_mm_f16(GenMatArgs a)
{
    const uint16_t *l = static_cast<const uint16_t *>(a.lhs.data);
    const uint16_t *r = static_cast<const uint16_t *>(a.rhs.data);
    float *y = static_cast<float *>(a.y.data);
    const uint64_t total = a.m * a.n;
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kBlock;
    for (uint64_t t = static_cast<uint64_t>(blockIdx.x) * kBlock + threadIdx.x; t < total; t += stride) {
        const uint64_t col = t / a.m;
        const uint64_t row = t - col * a.m;
        const uint16_t *lp = l + row * a.k;
        const uint16_t *rp = r + col * a.k;
        double s = 0.0;
        for (uint64_t i = 0; i < a.k; ++i)
            s += static_cast<double>(emel_fp16_to_f32(lp[i]) * emel_fp16_to_f32(rp[i]));
        y[static_cast<int64_t>(row) * a.y.st[0] + static_cast<int64_t>(col) * a.y.st[1]] = static_cast<float>(s);
    }
}

// mul_mat_argmax: per row of lhs [k, rows] the fused dot with rhs [k], then
// the first row with the greatest dot.  A sequential scan from row 0 with a
// strict > keeps row 0 when its dot is NaN; otherwise the result is the
// lowest row holding the maximum of the non-NaN dots.
struct MmBest {
    float v;
    uint32_t has;
    uint64_t i;
};

__device__ __forceinline__ void mm_merge(MmBest &a, const MmBest &b)
{
    if (!b.has) return;
    if (!a.has || b.v > a.v || (b.v == a.v && b.i < a.i)) a = b;
}

__global__ __launch_bounds__(kBlock) void k_mm_argmax_partial(GenMatArgs a, MmBest *partial, float *row0)
{
    __shared__ MmBest part[kBlock / kWave];
    const float *l = static_cast<const float *>(a.lhs.data);
    const float *r = static_cast<const float *>(a.rhs.data);
    MmBest best{0.0f, 0u, 0ull};
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kBlock;
    for (uint64_t row = static_cast<uint64_t>(blockIdx.x) * kBlock + threadIdx.x; row < a.m; row += stride) {
        const float *lp = l + static_cast<int64_t>(row) * a.lhs.st[1];
        float v = 0.0f;
        for (uint64_t i = 0; i < a.k; ++i)
            v = __builtin_fmaf(lp[static_cast<int64_t>(i) * a.lhs.st[0]], r[static_cast<int64_t>(i) * a.rhs.st[0]], v);
        if (row == 0) row0[0] = v;
        if (v == v) mm_merge(best, MmBest{v, 1u, row});
    }
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) {
        MmBest o;
        o.v = __shfl_xor(best.v, off, kWave);
        o.has = __shfl_xor(best.has, off, kWave);
        o.i = __shfl_xor(best.i, off, kWave);
        mm_merge(best, o);
    }
    if (threadIdx.x % kWave == 0) part[threadIdx.x / kWave] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int i = 1; i < kBlock / kWave; ++i) mm_merge(best, part[i]);
        partial[blockIdx.x] = best;
    }
}

__global__ __launch_bounds__(kBlock) void k_mm_argmax_final(const MmBest *partial, uint32_t n, const float *row0,
                                                            float *dst, int32_t *index_out)
{
    __shared__ MmBest part[kBlock / kWave];
    MmBest best{0.0f, 0u, 0ull};
    for (uint32_t i = threadIdx.x; i < n; i += kBlock) mm_merge(best, partial[i]);
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) {
        MmBest o;
        o.v = __shfl_xor(best.v, off, kWave);
        o.has = __shfl_xor(best.has, off, kWave);
        o.i = __shfl_xor(best.i, off, kWave);
        mm_merge(best, o);
    }
    if (threadIdx.x % kWave == 0) part[threadIdx.x / kWave] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int i = 1; i < kBlock / kWave; ++i) mm_merge(best, part[i]);
        const float v0 = row0[0];
        if (v0 != v0 || !best.has) {
            dst[0] = v0;
            index_out[0] = 0;
        } else {
            dst[0] = best.v;
            index_out[0] = static_cast<int32_t>(best.i);
        }
    }
}

uint32_t grid_for(uint64_t count, uint32_t block, uint64_t cap)
{
    uint64_t blocks = (count + block - 1) / block;
    if (blocks > cap) blocks = cap;
    if (blocks == 0) blocks = 1;
    return static_cast<uint32_t>(blocks);
}

constexpr uint32_t kMmArgmaxBlocks = 2048;

} // namespace

// ---- norm and rms_norm: a workgroup per row ------------------------------------------
// generic.rs:1988-2055: per row of width = src0.ne[0] ordinals, s = sum of
// f64(v*v) (rms) or f64(v) (norm), mean = f32(s / width); norm adds the f64
// sum of f32(centered^2) divided by width; scale = f32(1 / sqrt(base + eps))
// in f64; y = v * scale or (v - mean) * scale in f32.  The f64 sums run as a
// fixed-order tree over the row's threads (parity within the 1e-5 relative
// tolerance of rms_norm, not bit for bit against the reference's sequential
// order); every f32 step is the reference's.  A generic row is one dim-0
// row of src0, so its elements sit at a row base plus column * st[0]; dst
// rows are addressed the same way when dst.ne[0] == width, else each
// element's ordinal is decoded through dst's own extents.
template <int BS>
__device__ __forceinline__ double block_sum_f64(double v, double *lds)
{
    v = wave_sum_dpp(v);
    if constexpr (BS == kWave) {
        return v;
    } else {
        const uint32_t w = threadIdx.x / kWave;
        __syncthreads(); // lds is reused by the next reduction
        if (threadIdx.x % kWave == 0) lds[w] = v;
        __syncthreads();
        double t = lds[0];
#pragma unroll
        for (int i = 1; i < BS / kWave; ++i) t += lds[i];
        return t;
    }
}

template <bool RMS, int BS>
__global__ __launch_bounds__(BS) void k_gen_norm(GenRowArgs a, bool dst_rows)
{
    __shared__ double lds[BS / kWave];
    const uint64_t r = blockIdx.x;
    const uint64_t w = a.width;
    const float *x = static_cast<const float *>(a.x.data);
    float *y = static_cast<float *>(a.y.data);
    Walk xr, yr;
    xr.init(a.x, r * w); // column 0 of the row
    const int64_t sx = a.x.st[0];
    if (dst_rows) yr.init(a.y, r * w);
    double sum = 0.0;
    for (uint64_t c = threadIdx.x; c < w; c += BS) {
        const float v = x[xr.off + static_cast<int64_t>(c) * sx];
        sum += RMS ? static_cast<double>(v * v) : static_cast<double>(v);
    }
    sum = block_sum_f64<BS>(sum, lds);
    const float mean = static_cast<float>(sum / static_cast<double>(w));
    double base = static_cast<double>(mean);
    if constexpr (!RMS) {
        double var = 0.0;
        for (uint64_t c = threadIdx.x; c < w; c += BS) {
            const float centered = x[xr.off + static_cast<int64_t>(c) * sx] - mean;
            var += static_cast<double>(centered * centered);
        }
        var = block_sum_f64<BS>(var, lds);
        base = var / static_cast<double>(w);
    }
    const float scale = static_cast<float>(1.0 / __builtin_sqrt(base + static_cast<double>(a.eps)));
    for (uint64_t c = threadIdx.x; c < w; c += BS) {
        const float v = x[xr.off + static_cast<int64_t>(c) * sx];
        const float o = RMS ? v * scale : (v - mean) * scale;
        int64_t yo;
        if (dst_rows) {
            yo = yr.off + static_cast<int64_t>(c) * a.y.st[0];
        } else {
            Walk e;
            e.init(a.y, r * w + c);
            yo = e.off;
        }
        y[yo] = o;
    }
}

Operand as_operand(const GView &v)
{
    return Operand{v.data, {v.ne[0], v.ne[1], v.ne[2], v.ne[3]}, {v.st[0], v.st[1], v.st[2], v.st[3]}};
}

// Vectorisable rows (dim 0 contiguous, 16-byte aligned, same shapes) run on
// the typed row kernels with the generic arithmetic (RowOp::GenRmsNorm /
// GenNorm: rows in registers, 128-bit accesses); other layouts on
// k_gen_norm.
template <bool RMS>
hipError_t launch_gen_norm(const GenRowArgs &a, hipStream_t s)
{
    RowArgs ra{};
    ra.op = RMS ? RowOp::GenRmsNorm : RowOp::GenNorm;
    ra.x = as_operand(a.x);
    ra.y = as_operand(a.y);
    ra.eps = a.eps;
    const hipError_t e = launch_rows(ra, s);
    if (e != hipErrorNotSupported) return e;
    if (a.rows > 0x7fffffffull) return hipErrorInvalidConfiguration;
    const bool dst_rows = a.y.ne[0] == a.width;
    const dim3 grid(static_cast<uint32_t>(a.rows));
    if (a.width <= 1024) k_gen_norm<RMS, kWave><<<grid, kWave, 0, s>>>(a, dst_rows);
    else k_gen_norm<RMS, kBlock><<<grid, kBlock, 0, s>>>(a, dst_rows);
    return hipGetLastError();
}

// Rows narrower than a wave keep one lane per row (and the reference's
// sequential order).
constexpr uint64_t kNormRowMin = kWave;

hipError_t launch_generic_rows(const GenRowArgs &a, hipStream_t s)
{
    if (a.rows == 0) return hipSuccess;
    const uint64_t blocks = (a.rows + kRowBlock - 1) / kRowBlock;
    if (blocks > 0x7fffffffull) return hipErrorInvalidConfiguration;
    const dim3 grid(static_cast<uint32_t>(blocks));
    switch (a.op) {
    case GenRow::Cumsum: k_gen_rows<GenRow::Cumsum><<<grid, kRowBlock, 0, s>>>(a); break;
    case GenRow::SoftMax: { // generic.rs:1948-1986: the exact sequential-sum kernel of the typed strided path
        return launch_softmax_seq(as_operand(a.x), as_operand(a.y), s);
    }
    case GenRow::Norm:
        if (a.width >= kNormRowMin) return launch_gen_norm<false>(a, s);
        k_gen_rows<GenRow::Norm><<<grid, kRowBlock, 0, s>>>(a);
        break;
    case GenRow::RmsNorm:
        if (a.width >= kNormRowMin) return launch_gen_norm<true>(a, s);
        k_gen_rows<GenRow::RmsNorm><<<grid, kRowBlock, 0, s>>>(a);
        break;
    case GenRow::SoftMaxBack: k_gen_rows<GenRow::SoftMaxBack><<<grid, kRowBlock, 0, s>>>(a); break;
    case GenRow::RmsNormBack: k_gen_rows<GenRow::RmsNormBack><<<grid, kRowBlock, 0, s>>>(a); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_generic_ordinal(const GenOrdArgs &a, hipStream_t s)
{
    uint64_t count = 1;
    for (int d = 0; d < 4; ++d) count *= a.y.ne[d];
    const dim3 grid(grid_for(count, kBlock, 65536));
    switch (a.op) {
    case GenOrd::Fill: k_gen_ord<GenOrd::Fill><<<grid, kBlock, 0, s>>>(a, count); break;
    case GenOrd::Arange: k_gen_ord<GenOrd::Arange><<<grid, kBlock, 0, s>>>(a, count); break;
    case GenOrd::Diag: k_gen_ord<GenOrd::Diag><<<grid, kBlock, 0, s>>>(a, count); break;
    case GenOrd::DiagMaskInf: k_gen_ord<GenOrd::DiagMaskInf><<<grid, kBlock, 0, s>>>(a, count); break;
    case GenOrd::DiagMaskZero: k_gen_ord<GenOrd::DiagMaskZero><<<grid, kBlock, 0, s>>>(a, count); break;
    case GenOrd::Concat: k_gen_ord<GenOrd::Concat><<<grid, kBlock, 0, s>>>(a, count); break;
    case GenOrd::RepeatBack: k_gen_ord<GenOrd::RepeatBack><<<grid, kBlock, 0, s>>>(a, count); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

uint64_t generic_workspace_bytes(GenWork w)
{
    switch (w) {
    case GenWork::L2Norm: return 256;
    case GenWork::CountEqual: return kCountBlocks * sizeof(unsigned long long);
    case GenWork::MulMatArgmax: return 256 + kMmArgmaxBlocks * sizeof(MmBest);
    }
    return 0;
}

hipError_t launch_generic_l2_norm(const GView &x, const GView &y, void *workspace, hipStream_t s)
{
    uint64_t count = 1;
    for (int d = 0; d < 4; ++d) count *= x.ne[d];
    float *scale = static_cast<float *>(workspace);
    k_l2_sum<<<1, 64, 0, s>>>(x, count, scale);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    k_l2_apply<<<grid_for(count, kBlock, 65536), kBlock, 0, s>>>(x, y, count, scale);
    return hipGetLastError();
}

hipError_t launch_generic_l2_sum(const GView &x, void *workspace, hipStream_t s)
{
    uint64_t count = 1;
    for (int d = 0; d < 4; ++d) count *= x.ne[d];
    k_l2_sum<<<1, 64, 0, s>>>(x, count, static_cast<float *>(workspace));
    return hipGetLastError();
}

hipError_t launch_generic_l2_apply(const GView &x, const GView &y, const void *workspace, hipStream_t s)
{
    uint64_t count = 1;
    for (int d = 0; d < 4; ++d) count *= x.ne[d];
    k_l2_apply<<<grid_for(count, kBlock, 65536), kBlock, 0, s>>>(x, y, count, static_cast<const float *>(workspace));
    return hipGetLastError();
}

hipError_t launch_generic_count_equal(const GView &a, const GView &b, float *dst, void *workspace, hipStream_t s)
{
    uint64_t count = 1;
    for (int d = 0; d < 4; ++d) count *= a.ne[d];
    auto *partial = static_cast<unsigned long long *>(workspace);
    const uint32_t blocks = grid_for(count, kBlock, kCountBlocks);
    k_count_partial<<<blocks, kBlock, 0, s>>>(a, b, count, partial);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    k_count_final<<<1, kBlock, 0, s>>>(partial, blocks, dst);
    return hipGetLastError();
}

hipError_t launch_generic_mul_mat(const GenMatArgs &a, hipStream_t s)
{
    if (a.argmax) {
        char *ws = static_cast<char *>(a.workspace);
        float *row0 = reinterpret_cast<float *>(ws);
        MmBest *partial = reinterpret_cast<MmBest *>(ws + 256);
        const uint32_t blocks = grid_for(a.m, kBlock, kMmArgmaxBlocks);
        k_mm_argmax_partial<<<blocks, kBlock, 0, s>>>(a, partial, row0);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        k_mm_argmax_final<<<1, kBlock, 0, s>>>(partial, blocks, row0, static_cast<float *>(a.y.data), a.index_out);
        return hipGetLastError();
    }
    const dim3 grid(grid_for(a.m * a.n, kBlock, 65536));
    if (a.f16)
        k_mm_f16<<<grid, kBlock, 0, s>>>(a);
    else
        k_mm_f32<<<grid, kBlock, 0, s>>>(a);
    return hipGetLastError();
}

} // namespace emel
