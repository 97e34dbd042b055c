// rows.hip -- gfx950 kernels for the per-row ops: rms_norm (+weight),
// norm, soft_max (dense and strided) and the scaled + masked soft_max.
//
// A row is dim 0 of the view; rows enumerate (i1, i2, i3).  A wave (short
// rows) or a 4-wave workgroup (long rows) owns one row: it loads the row
// once into registers (128-bit non-temporal loads), reduces with butterfly
// shuffles and, across waves, through LDS, and writes the result once, so
// each row costs one HBM read and one HBM write.  Rows wider than the
// register budget stream through global memory in several passes (the later
// passes hit L2).  Row reductions keep the reference's
// arithmetic: f32-rounded squares summed in f64 (normalization.rs:343-362),
// exp(x - max) summed in f64 (reductions.rs:565-601), divisions and square
// roots correctly rounded.  The strided soft_max keeps the reference's
// sequential f32 sum (reductions.rs:603-638), evaluated exactly by a
// workgroup per row (one lane per row for rows of at most 64 columns).
#include <cstdlib>

#include "common.hpp"
#include "launch.hpp"
#include "libm_replica.hpp"
#include "seqsum.hpp"

namespace emel {
namespace {

struct RowGeo {
    uint32_t rows;
    uint32_t ncols;
    FastDiv ne1, ne2; // row index -> (i1, i2, i3)
    int64_t x_st[4];
    int64_t y_st[4];
};

struct MaskGeo {
    const uint16_t *p; // dense f16 [ncols, ne1, m2, m3] or null
    uint32_t ne1;
    FastDiv m2, m3;    // the mask's extents along dims 2 and 3 (divide the source's)
};

__device__ __forceinline__ void row_coords(const RowGeo &g, uint32_t r, uint32_t &i1, uint32_t &i2, uint32_t &i3)
{
    const uint32_t t = g.ne1.div(r);
    i1 = r - t * g.ne1.d;
    i3 = g.ne2.div(t);
    i2 = t - i3 * g.ne2.d;
}

__device__ __forceinline__ int64_t row_base(const int64_t *st, uint32_t i1, uint32_t i2, uint32_t i3)
{
    return static_cast<int64_t>(i1) * st[1] + static_cast<int64_t>(i2) * st[2] + static_cast<int64_t>(i3) * st[3];
}

// Four f16 mask values widened to f32 (fp16_to_f32, quant.rs:287-300; the
// hardware widening is exact and gives the same values).
__device__ __forceinline__ float4 mask4(const uint16_t *m)
{
    const uint2 raw = *reinterpret_cast<const uint2 *>(m);
    return make_float4(hw_fp16_to_f32(static_cast<uint16_t>(raw.x & 0xffffu)),
                       hw_fp16_to_f32(static_cast<uint16_t>(raw.x >> 16)),
                       hw_fp16_to_f32(static_cast<uint16_t>(raw.y & 0xffffu)),
                       hw_fp16_to_f32(static_cast<uint16_t>(raw.y >> 16)));
}

// f32 products rounded, then accumulated in f64 (run_rms_norm).
__device__ __forceinline__ double sumsq4(float4 v)
{
    const float a = v.x * v.x, b = v.y * v.y, c = v.z * v.z, d = v.w * v.w;
    return (static_cast<double>(a) + static_cast<double>(b)) + (static_cast<double>(c) + static_cast<double>(d));
}

__device__ __forceinline__ double sum4(float4 v)
{
    return (static_cast<double>(v.x) + static_cast<double>(v.y)) +
           (static_cast<double>(v.z) + static_cast<double>(v.w));
}

__device__ __forceinline__ float max4(float4 v)
{
    return __builtin_fmaxf(__builtin_fmaxf(v.x, v.y), __builtin_fmaxf(v.z, v.w));
}

__device__ __forceinline__ float4 mul4(float4 v, float k) { return make_float4(v.x * k, v.y * k, v.z * k, v.w * k); }
__device__ __forceinline__ float4 mul4(float4 v, float4 w)
{
    return make_float4(v.x * w.x, v.y * w.y, v.z * w.z, v.w * w.w);
}
__device__ __forceinline__ float4 add4(float4 v, float4 w)
{
    return make_float4(v.x + w.x, v.y + w.y, v.z + w.z, v.w + w.w);
}
__device__ __forceinline__ float4 sub4(float4 v, float k) { return make_float4(v.x - k, v.y - k, v.z - k, v.w - k); }
// v / den for a row sum den >= 1, via the row's double reciprocal.
__device__ __forceinline__ float4 div4(float4 v, double recip)
{
    return make_float4(div_by_recip(v.x, recip), div_by_recip(v.y, recip), div_by_recip(v.z, recip),
                       div_by_recip(v.w, recip));
}
// exp(v - max): arguments are <= 0 or NaN.
__device__ __forceinline__ float4 exp4(float4 v, const uint64_t *t, const ExpfConsts &c)
{
    return make_float4(emel_expf_nonpos(v.x, t, c), emel_expf_nonpos(v.y, t, c), emel_expf_nonpos(v.z, t, c),
                       emel_expf_nonpos(v.w, t, c));
}

// The scale factors of the two normalisations.  Typed events
// (normalization.rs:316-362): k = 1 / sqrtf(mean + eps) in f32, norm's
// variance the f64 sum of f64 products of the centered values, rounded to
// f32 before its square root.  The generic envelope (generic.rs:2030-2040):
// k = f32(1 / sqrt(base + eps)) in f64, norm's variance the f64 sum of f32
// squares, kept in f64.
template <RowOp OP>
constexpr bool kRmsOp = OP == RowOp::RmsNorm || OP == RowOp::RmsNormMul || OP == RowOp::GenRmsNorm;
template <RowOp OP>
constexpr bool kNormOp = OP == RowOp::Norm || OP == RowOp::GenNorm;

template <RowOp OP>
__device__ __forceinline__ float rms_scale(float mean, float eps)
{
    if constexpr (OP == RowOp::GenRmsNorm)
        return static_cast<float>(1.0 / __builtin_sqrt(static_cast<double>(mean) + static_cast<double>(eps)));
    else
        return 1.0f / __builtin_sqrtf(mean + eps);
}

template <RowOp OP>
__device__ __forceinline__ double centered_sq4(float4 c)
{
    if constexpr (OP == RowOp::GenNorm)
        return sumsq4(c);
    else
        return (static_cast<double>(c.x) * c.x + static_cast<double>(c.y) * c.y) +
               (static_cast<double>(c.z) * c.z + static_cast<double>(c.w) * c.w);
}

template <RowOp OP>
__device__ __forceinline__ float norm_scale(double var, uint32_t ncols, float eps)
{
    if constexpr (OP == RowOp::GenNorm) {
        return static_cast<float>(1.0 / __builtin_sqrt(var / static_cast<double>(ncols) + static_cast<double>(eps)));
    } else {
        const float variance = static_cast<float>(var / static_cast<double>(ncols));
        return 1.0f / __builtin_sqrtf(variance + eps);
    }
}

// ---- vectorized rows: contiguous dim 0, ncols % 4 == 0 ------------------
// NW waves own a row: NW = 1 puts four rows in a 256-thread workgroup (rows
// of at most 1024 columns), NW = 4 gives each row its own workgroup.  Thread
// t of a row holds float4 t, t + 64*NW, ... in registers, NV of them; FULL
// means the row fills them exactly, so no per-element bounds checks run.
// NV == 0 streams rows too wide for registers in passes.  Row data is read
// and written with non-temporal accesses (each byte moves once); weights
// and masks stay on the cached path.  Rows run in memory order.

// Row reductions over the NW waves of a row: wave partials go to LDS slots
// [first wave of the row, + NW); the slots are fixed, so the sum's order is.
template <int NW>
__device__ __forceinline__ double row_sum(double v, double *lds)
{
    v = wave_sum(v);
    if constexpr (NW == 1) {
        return v;
    } else {
        const uint32_t w = threadIdx.x / kWave;
        if (threadIdx.x % kWave == 0) lds[w] = v;
        __syncthreads();
        const double *p = lds + (w / NW) * NW;
        double t = p[0];
#pragma unroll
        for (int i = 1; i < NW; ++i) t += p[i];
        return t;
    }
}

template <int NW>
__device__ __forceinline__ float row_max(float v, double *lds)
{
    v = wave_max(v);
    if constexpr (NW == 1) {
        return v;
    } else {
        const uint32_t w = threadIdx.x / kWave;
        if (threadIdx.x % kWave == 0) lds[w] = v;
        __syncthreads();
        const double *p = lds + (w / NW) * NW;
        float t = static_cast<float>(p[0]);
#pragma unroll
        for (int i = 1; i < NW; ++i) t = __builtin_fmaxf(t, static_cast<float>(p[i]));
        return t;
    }
}

template <RowOp OP, int NW, int NV, bool FULL, bool MASK, int BS = kBlock>
__global__ __launch_bounds__(BS) void k_row_vec(RowGeo g, const float *x, float *y, const float *w, MaskGeo mg,
                                                 float eps, float scale)
{
    constexpr bool kSoft = OP == RowOp::SoftMax || OP == RowOp::SoftMaxExt;
    constexpr uint32_t kTPR = NW * kWave;      // threads per row
    constexpr uint32_t kRPB = BS / kTPR;       // rows per workgroup
    static_assert(kRPB >= 1 && BS % kTPR == 0, "a workgroup holds whole rows");
    __shared__ uint64_t lds_tab[32];
    __shared__ double lds_a[BS / kWave];       // first row reduction
    __shared__ double lds_b[BS / kWave];       // second row reduction
    const uint64_t *tab = nullptr;
    ExpfConsts ec;
    // The expf table goes to LDS.  With NW > 1, wave 0 loads it into a
    // register ahead of the row and writes it once the row's loads are
    // issued (waiting for the table load only), and the max reduction's
    // barrier orders it before use: no wave waits for the table before
    // issuing its row loads.  With NW == 1 it is staged up front, before
    // any wave may leave.
    uint64_t tab_word = 0;
    if constexpr (kSoft) {
        if constexpr (NW == 1) {
            if (threadIdx.x < 32) lds_tab[threadIdx.x] = kExp2Table[threadIdx.x];
            __syncthreads();
        } else {
            if (threadIdx.x < kWave) tab_word = kExp2Table[threadIdx.x % 32];
        }
        tab = lds_tab;
        ec = expf_consts_in_vgprs();
    }
    auto stage_table = [&]() {
        if (threadIdx.x < 32) lds_tab[threadIdx.x] = tab_word;
    };
    const uint32_t t = threadIdx.x % kTPR;
    uint32_t r; // uniform across the row's waves
    if constexpr (kRPB == 1) {
        r = blockIdx.x;
    } else {
        r = blockIdx.x * kRPB + __builtin_amdgcn_readfirstlane(threadIdx.x / kTPR);
        // NW == 1: no workgroup barrier follows, so a wave past the end may
        // leave.  NW > 1: the host launches these only when kRPB divides
        // the row count, so every row of every workgroup exists.
        if constexpr (NW == 1) {
            if (r >= g.rows) return;
        }
    }

    uint32_t i1, i2, i3;
    row_coords(g, r, i1, i2, i3);
    const float4 *xr = reinterpret_cast<const float4 *>(x + row_base(g.x_st, i1, i2, i3));
    float4 *yr = reinterpret_cast<float4 *>(y + row_base(g.y_st, i1, i2, i3));
    const uint32_t nv = g.ncols / 4;
    const uint16_t *mr = nullptr;
    if constexpr (MASK) {
        const uint64_t mrow = (static_cast<uint64_t>(mg.m3.mod(i3)) * mg.m2.d + mg.m2.mod(i2)) * mg.ne1 + i1;
        mr = mg.p + mrow * g.ncols;
    }
    auto load = [&](uint32_t idx) {
        float4 v = ld_nt(xr + idx);
        if constexpr (OP == RowOp::SoftMaxExt) {
            v = mul4(v, scale);                              // OpScale
            if constexpr (MASK) v = add4(v, mask4(mr + 4 * idx)); // OpAdd(f16 mask -> f32)
        }
        return v;
    };
    auto in_row = [&](int j) { return FULL || t + kTPR * j < nv; };

    if constexpr (NV > 0) {
        float4 v[NV];
#pragma unroll
        for (int j = 0; j < NV; ++j) v[j] = in_row(j) ? load(t + kTPR * j) : make_float4(0.f, 0.f, 0.f, 0.f);
        if constexpr (kSoft && NW > 1) stage_table();
        if constexpr (kRmsOp<OP>) {
            double acc = 0.0;
#pragma unroll
            for (int j = 0; j < NV; ++j)
                if (in_row(j)) acc += sumsq4(v[j]);
            acc = row_sum<NW>(acc, lds_a);
            const float mean = static_cast<float>(acc / static_cast<double>(g.ncols));
            const float k = rms_scale<OP>(mean, eps);
#pragma unroll
            for (int j = 0; j < NV; ++j) {
                if (in_row(j)) {
                    const uint32_t idx = t + kTPR * j;
                    float4 o = mul4(v[j], k);
                    if constexpr (OP == RowOp::RmsNormMul) o = mul4(o, reinterpret_cast<const float4 *>(w)[idx]);
                    st_nt(yr + idx, o);
                }
            }
        } else if constexpr (kNormOp<OP>) {
            double acc = 0.0;
#pragma unroll
            for (int j = 0; j < NV; ++j)
                if (in_row(j)) acc += sum4(v[j]);
            acc = row_sum<NW>(acc, lds_a);
            const float mean = static_cast<float>(acc / static_cast<double>(g.ncols));
            double var = 0.0;
#pragma unroll
            for (int j = 0; j < NV; ++j)
                if (in_row(j)) var += centered_sq4<OP>(sub4(v[j], mean));
            var = row_sum<NW>(var, lds_b);
            const float k = norm_scale<OP>(var, g.ncols, eps);
#pragma unroll
            for (int j = 0; j < NV; ++j)
                if (in_row(j)) st_nt(yr + t + kTPR * j, mul4(sub4(v[j], mean), k));
        } else { // soft_max, f64 row sum
            float mx = -__builtin_inff();
#pragma unroll
            for (int j = 0; j < NV; ++j)
                if (in_row(j)) mx = __builtin_fmaxf(mx, max4(v[j]));
            mx = row_max<NW>(mx, lds_a);
            double acc = 0.0;
#pragma unroll
            for (int j = 0; j < NV; ++j) {
                if (in_row(j)) {
                    v[j] = exp4(sub4(v[j], mx), tab, ec);
                    acc += sum4(v[j]);
                }
            }
            acc = row_sum<NW>(acc, lds_b);
            const double recip = 1.0 / static_cast<double>(static_cast<float>(acc));
#pragma unroll
            for (int j = 0; j < NV; ++j)
                if (in_row(j)) st_nt(yr + t + kTPR * j, div4(v[j], recip));
        }
    } else {
        // streamed passes for rows wider than the register budget; the
        // intermediate passes use cached accesses so re-reads hit L2
        if constexpr (kSoft && NW > 1) stage_table();
        if constexpr (kRmsOp<OP>) {
            double acc = 0.0;
            for (uint32_t idx = t; idx < nv; idx += kTPR) acc += sumsq4(xr[idx]);
            acc = row_sum<NW>(acc, lds_a);
            const float mean = static_cast<float>(acc / static_cast<double>(g.ncols));
            const float k = rms_scale<OP>(mean, eps);
            for (uint32_t idx = t; idx < nv; idx += kTPR) {
                float4 o = mul4(xr[idx], k);
                if constexpr (OP == RowOp::RmsNormMul) o = mul4(o, reinterpret_cast<const float4 *>(w)[idx]);
                st_nt(yr + idx, o);
            }
        } else if constexpr (kNormOp<OP>) {
            double acc = 0.0;
            for (uint32_t idx = t; idx < nv; idx += kTPR) acc += sum4(xr[idx]);
            acc = row_sum<NW>(acc, lds_a);
            const float mean = static_cast<float>(acc / static_cast<double>(g.ncols));
            double var = 0.0;
            for (uint32_t idx = t; idx < nv; idx += kTPR) var += centered_sq4<OP>(sub4(xr[idx], mean));
            var = row_sum<NW>(var, lds_b);
            const float k = norm_scale<OP>(var, g.ncols, eps);
            for (uint32_t idx = t; idx < nv; idx += kTPR) st_nt(yr + idx, mul4(sub4(xr[idx], mean), k));
        } else {
            auto load_cached = [&](uint32_t idx) {
                float4 v = xr[idx];
                if constexpr (OP == RowOp::SoftMaxExt) {
                    v = mul4(v, scale);
                    if constexpr (MASK) v = add4(v, mask4(mr + 4 * idx));
                }
                return v;
            };
            float mx = -__builtin_inff();
            for (uint32_t idx = t; idx < nv; idx += kTPR) mx = __builtin_fmaxf(mx, max4(load_cached(idx)));
            mx = row_max<NW>(mx, lds_a);
            double acc = 0.0;
            for (uint32_t idx = t; idx < nv; idx += kTPR) {
                const float4 e = exp4(sub4(load_cached(idx), mx), tab, ec);
                yr[idx] = e;
                acc += sum4(e);
            }
            acc = row_sum<NW>(acc, lds_b);
            const double recip = 1.0 / static_cast<double>(static_cast<float>(acc));
            for (uint32_t idx = t; idx < nv; idx += kTPR) st_nt(yr + idx, div4(yr[idx], recip));
        }
    }
}

// ---- general rows: any strides, per-element ordinal addressing ----------

struct OrdView {
    uint64_t ne[4];
    int64_t st[4];
};

__device__ __forceinline__ int64_t ord_index(const OrdView &v, uint64_t k)
{
    int64_t off = 0;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        off += static_cast<int64_t>(k % v.ne[d]) * v.st[d];
        k /= v.ne[d];
    }
    return off;
}

// One wave per row; element k of row r is ordinal r*ncols + k of each view.
template <RowOp OP>
__global__ __launch_bounds__(kBlock) void k_row_generic(OrdView xv, OrdView yv, uint64_t rows, uint64_t ncols,
                                                         const float *x, float *y, const float *w, int64_t w_st0,
                                                         float eps)
{
    const uint32_t wave = threadIdx.x / kWave;
    const uint32_t lane = threadIdx.x % kWave;
    const uint64_t r = static_cast<uint64_t>(blockIdx.x) * (kBlock / kWave) + wave;
    if (r >= rows) return;
    const uint64_t base = r * ncols;
    if constexpr (OP == RowOp::RmsNorm || OP == RowOp::RmsNormMul) {
        double acc = 0.0;
        for (uint64_t c = lane; c < ncols; c += kWave) {
            const float v = x[ord_index(xv, base + c)];
            const float sq = v * v;
            acc += static_cast<double>(sq);
        }
        acc = wave_sum(acc);
        const float mean = static_cast<float>(acc / static_cast<double>(ncols));
        const float k = 1.0f / __builtin_sqrtf(mean + eps);
        for (uint64_t c = lane; c < ncols; c += kWave) {
            float out = x[ord_index(xv, base + c)] * k;
            if constexpr (OP == RowOp::RmsNormMul) out = out * w[static_cast<int64_t>(c) * w_st0];
            y[ord_index(yv, base + c)] = out;
        }
    } else if constexpr (OP == RowOp::Norm) {
        double acc = 0.0;
        for (uint64_t c = lane; c < ncols; c += kWave) acc += static_cast<double>(x[ord_index(xv, base + c)]);
        acc = wave_sum(acc);
        const float mean = static_cast<float>(acc / static_cast<double>(ncols));
        double var = 0.0;
        for (uint64_t c = lane; c < ncols; c += kWave) {
            const float cv = x[ord_index(xv, base + c)] - mean;
            var += static_cast<double>(cv) * static_cast<double>(cv);
        }
        var = wave_sum(var);
        const float variance = static_cast<float>(var / static_cast<double>(ncols));
        const float k = 1.0f / __builtin_sqrtf(variance + eps);
        for (uint64_t c = lane; c < ncols; c += kWave)
            y[ord_index(yv, base + c)] = (x[ord_index(xv, base + c)] - mean) * k;
    }
}

// Dense-sum soft_max over general layouts (wave per row, f64 sum).  With
// kExt the element is first scaled and the f16 mask added (the soft_max_ext
// composition); kExt requires x and y to share extents.
template <bool kExt>
__global__ __launch_bounds__(kBlock) void k_softmax_generic(OrdView xv, OrdView yv, uint64_t rows, uint64_t ncols,
                                                             const float *x, float *y, MaskGeo mg, float scale)
{
    __shared__ uint64_t lds[32];
    if (threadIdx.x < 32) lds[threadIdx.x] = kExp2Table[threadIdx.x];
    __syncthreads();
    const uint32_t wave = threadIdx.x / kWave;
    const uint32_t lane = threadIdx.x % kWave;
    const uint64_t r = static_cast<uint64_t>(blockIdx.x) * (kBlock / kWave) + wave;
    if (r >= rows) return;
    const uint64_t base = r * ncols;
    const uint16_t *mr = nullptr;
    if (kExt && mg.p) {
        const uint64_t i1 = r % xv.ne[1];
        const uint64_t i2 = (r / xv.ne[1]) % xv.ne[2];
        const uint64_t i3 = r / (xv.ne[1] * xv.ne[2]);
        mr = mg.p + ((i3 % mg.m3.d) * mg.m2.d + (i2 % mg.m2.d)) * static_cast<uint64_t>(mg.ne1) * ncols + i1 * ncols;
    }
    auto load = [&](uint64_t c) {
        float v = x[ord_index(xv, base + c)];
        if constexpr (kExt) {
            v = v * scale;
            if (mr) v = v + hw_fp16_to_f32(mr[c]);
        }
        return v;
    };
    float mx = -__builtin_inff();
    for (uint64_t c = lane; c < ncols; c += kWave) mx = __builtin_fmaxf(mx, load(c));
    mx = wave_max(mx);
    double acc = 0.0;
    for (uint64_t c = lane; c < ncols; c += kWave) {
        const float e = emel_expf_nonpos(load(c) - mx, lds);
        y[ord_index(yv, base + c)] = e;
        acc += static_cast<double>(e);
    }
    acc = wave_sum(acc);
    const double recip = 1.0 / static_cast<double>(static_cast<float>(acc));
    for (uint64_t c = lane; c < ncols; c += kWave) {
        const int64_t o = ord_index(yv, base + c);
        y[o] = div_by_recip(y[o], recip);
    }
}

// Strided soft_max (reductions.rs:603-638) and the generic envelope's
// soft_max (generic.rs:1948-1986): the row sum is the sequential f32 sum
// s_k = RN(s_{k-1} + e_k) in column order.  One workgroup of NT threads per
// row:
//   1. the row maximum, all threads (the order does not matter: NaN never
//      wins, and a NaN or an infinity turns the row into NaN through its sum
//      in either formulation);
//   2. per tile of NT * SEG columns, every thread computes its e = expf(x -
//      max) and stages it in LDS in column order; the tile is then added to
//      the running sum exactly (seq_tile_sum below);
//   3. y = e / sum, the correctly rounded quotient (div_by_recip, sum >= 1).
// Column c of row r is ordinal r * ncols + c of each view; x has ncols ==
// ne[0], so its offset is the row's offset plus c * st[0].  y shares that
// form when its ne[0] is ncols (kYRow), else its ordinal is decoded.
// Rows of at most kSeqShort columns take one lane each instead: the
// reference's own loop, short enough that a workgroup per row would idle.
constexpr uint64_t kSeqShort = 64;

__device__ __forceinline__ int64_t row_offset(const OrdView &v, uint64_t r)
{
    const uint64_t i1 = r % v.ne[1];
    const uint64_t q = r / v.ne[1];
    return static_cast<int64_t>(i1) * v.st[1] + static_cast<int64_t>(q % v.ne[2]) * v.st[2] +
           static_cast<int64_t>(q / v.ne[2]) * v.st[3];
}

__global__ __launch_bounds__(kBlock) void k_softmax_lane(OrdView xv, OrdView yv, uint64_t rows, uint64_t ncols,
                                                          const float *x, float *y)
{
    __shared__ uint64_t tab[32];
    if (threadIdx.x < 32) tab[threadIdx.x] = kExp2Table[threadIdx.x];
    __syncthreads();
    const uint64_t r = static_cast<uint64_t>(blockIdx.x) * kBlock + threadIdx.x;
    if (r >= rows) return;
    const uint64_t base = r * ncols;
    float mx = x[ord_index(xv, base)];
    for (uint64_t c = 1; c < ncols; ++c) {
        const float v = x[ord_index(xv, base + c)];
        if (v > mx) mx = v;
    }
    float sum = 0.0f;
    for (uint64_t c = 0; c < ncols; ++c) {
        const float e = emel_expf_nonpos(x[ord_index(xv, base + c)] - mx, tab);
        y[ord_index(yv, base + c)] = e;
        sum += e;
    }
    const double recip = 1.0 / static_cast<double>(sum);
    for (uint64_t c = 0; c < ncols; ++c) {
        const int64_t o = ord_index(yv, base + c);
        y[o] = div_by_recip(y[o], recip);
    }
}

// The exact sequential sum of one staged tile (seqsum.hpp), in two steps.
//
// Predict, all threads: thread t owns the tile's addends SEG t .. SEG t +
// SEG - 1 (segment t).  The running sum before them is within
// seq_rel_bound of the exact value s_prev + (f64 prefix of the tile),
// s_prev being the exact running sum before the tile.  When that interval,
// widened to the end of the segment, lies in one binade [2^(E-1), 2^E) and
// no addend is a rounding tie on its grid 2^u (u = E - 24), every addition
// inside the segment adds round(e / 2^u) units: the segment is predictable
// and its contribution is an integer.  Its units are scanned over the
// tile, and the unpredictable segments are listed in order.
//
// Combine, wave 0: between two unpredictable segments lies a run of
// predictable ones.  When the run lies in one binade with the running sum
// (the grids of its first and last segments equal the state's), the run
// adds an exact multiple of 2^u: its scanned unit count times 2^u, an f32
// value, so one f32 addition adds the whole run exactly.  Each
// unpredictable segment is added one f32 addition at a time, the
// reference's own arithmetic.  So the combine is one flat sequence of f32
// additions -- per unpredictable segment, its run then its addends -- with
// each run's binade checked before and after its addition (a check that
// fails falls back to adding the whole tile one addend at a time).  A row
// takes SEG + 1 additions per binade crossing and per segment holding a
// tie.  The sequence is read from LDS records, the next record loaded while
// the current one is added: a handful of instructions per addition, where
// a loop that rebuilt the state (m, u) per segment cost several times more.
constexpr int32_t kNoGrid = -1000; // u of an unpredictable segment

// The i-th unpredictable segment f in one 16-byte-aligned record: its
// addends, the scanned units before it and the grids on either side of it
// (the last segment of the run before it, the first of the run after it).
// Record nfail is a sentinel: zero addends after the tile's last run.
template <uint32_t SEG>
struct alignas(16) FailRec {
    float e[SEG];     // segment f's addends (+0 in the sentinel)
    uint32_t units;   // predictable units before segment f (the tile's total in the sentinel)
    int32_t u_before; // u[f - 1]: the run's last grid; kNoGrid when the run before f is empty
    int32_t u_after;  // u[f + 1]: the next run's first grid; kNoGrid when it is empty
    uint32_t pad;
};

template <uint32_t NT, uint32_t SEG>
struct SeqScratch {
    int32_t u[NT]; // grid exponent per segment, kNoGrid if unpredictable
    FailRec<SEG> rec[NT + 1];
    uint32_t wave_units[NT / kWave];
    uint32_t wave_fail[NT / kWave];
    double wave_sum[NT / kWave];
};

// Adds segment g's addends to acc one by one.
template <uint32_t SEG>
__device__ __forceinline__ float walk_segment(const float *s_e, uint32_t g, float acc)
{
    const float4 *q = reinterpret_cast<const float4 *>(s_e + SEG * g);
#pragma unroll
    for (uint32_t j = 0; j < SEG / 4; ++j) {
        const float4 v = q[j];
        acc += v.x;
        acc += v.y;
        acc += v.z;
        acc += v.w;
    }
    return acc;
}

template <uint32_t NT, uint32_t SEG>
__device__ __forceinline__ void seq_tile_sum(const float *s_e, SeqScratch<NT, SEG> &sc, float s_prev, SumState &st)
{
    constexpr uint32_t NW = NT / kWave;
    const uint32_t t = threadIdx.x;
    const uint32_t wave = t / kWave, lane = t % kWave;
    float e[SEG];
#pragma unroll
    for (uint32_t j = 0; j < SEG; j += 4) {
        const float4 q = *reinterpret_cast<const float4 *>(&s_e[SEG * t + j]);
        e[j] = q.x;
        e[j + 1] = q.y;
        e[j + 2] = q.z;
        e[j + 3] = q.w;
    }
    double part[4]; // four partial sums: a short dependency chain
#pragma unroll
    for (uint32_t j = 0; j < 4; ++j) part[j] = static_cast<double>(e[j]);
#pragma unroll
    for (uint32_t j = 4; j < SEG; ++j) part[j % 4] += static_cast<double>(e[j]);
    const double seg = (part[0] + part[1]) + (part[2] + part[3]);
    const double incl = wave_incl_scan_f64(seg);
    if (lane == kWave - 1) sc.wave_sum[wave] = incl;
    __syncthreads();
    // the exclusive prefix as a sum of whole segments (never incl - seg,
    // whose cancellation error is not relative to the prefix): positive
    // terms, so its f64 error is relative, within seq_rel_bound's slack
    const double up = __shfl_up(incl, 1, kWave);
    double pre = lane == 0 ? 0.0 : up;
    for (uint32_t w = 0; w < wave; ++w) pre += sc.wave_sum[w];
    const double base = static_cast<double>(s_prev) + pre;
    const double lo = base * (1.0 - seq_rel_bound(static_cast<double>(SEG * t)));
    const double hi = (base + seg) * (1.0 + seq_rel_bound(static_cast<double>(SEG * t + SEG)));
    int elo = 0, ehi = 0;
    (void)__builtin_frexp(lo, &elo);
    (void)__builtin_frexp(hi, &ehi);
    bool ok = lo >= 0x1p-126 && hi < 0x1p127 && lo <= hi && elo == ehi;
    const int32_t u = elo - 1 - 23;
    // seq_units of each addend, specialised to a segment in one binade:
    // every addend is below 2^24 units there (no clamp needed, never NaN),
    // each t - round(t) is exact, and every partial unit sum is an integer
    // below 2^24, so four f32 partial sums hold them exactly.  A tie is
    // |t - round(t)| == 1/2, taken from the largest distance.
    uint32_t units = 0;
    if (ok) {
        float part[4];
        float dist = 0.0f;
#pragma unroll
        for (uint32_t j = 0; j < SEG; ++j) {
            const float tj = __builtin_ldexpf(e[j], -u);
            const float rj = __builtin_rintf(tj);
            part[j % 4] = j < 4 ? rj : part[j % 4] + rj;
            dist = __builtin_fmaxf(dist, __builtin_fabsf(tj - rj));
        }
        units = static_cast<uint32_t>((part[0] + part[1]) + (part[2] + part[3]));
        ok = dist != 0.5f;
    }
    units = ok ? units : 0u;
    sc.u[t] = ok ? u : kNoGrid;
    // scan of units and compaction of the unpredictable segments
    const uint32_t uincl = wave_incl_scan(units);
    const uint64_t failing = __ballot(!ok);
    if (lane == kWave - 1) {
        sc.wave_units[wave] = uincl;
        sc.wave_fail[wave] = static_cast<uint32_t>(__builtin_popcountll(failing));
    }
    __syncthreads();
    uint32_t ubase = 0, fbase = 0, nfail = 0, total = 0;
#pragma unroll
    for (uint32_t w = 0; w < NW; ++w) {
        const uint32_t wu = sc.wave_units[w], wf = sc.wave_fail[w];
        ubase += w < wave ? wu : 0u;
        fbase += w < wave ? wf : 0u;
        nfail += wf;
        total += wu;
    }
    if (!ok) {
        FailRec<SEG> &r = sc.rec[fbase + static_cast<uint32_t>(__builtin_popcountll(failing & ((uint64_t{1} << lane) - 1)))];
        r.units = ubase + uincl; // units contributes 0
        r.u_before = t > 0 ? sc.u[t - 1] : kNoGrid;
        r.u_after = t + 1 < NT ? sc.u[t + 1] : kNoGrid;
#pragma unroll
        for (uint32_t j = 0; j < SEG; ++j) r.e[j] = e[j];
    }
    if (t == NT - 1) {
        FailRec<SEG> &r = sc.rec[nfail];
        r.units = total;
        r.u_before = ok ? u : kNoGrid;
        r.u_after = kNoGrid;
#pragma unroll
        for (uint32_t j = 0; j < SEG; ++j) r.e[j] = 0.0f;
    }
    __syncthreads();
    if (wave != 0 || !st.finite) return;

    // The flat walk, uniform across wave 0.  Record i's run is the
    // segments between the previous record's segment and its own: its
    // units are the difference of the two scanned counts, its first grid
    // the previous record's u_after (u[0] for the first).  grid(): the
    // exponent of the f32 spacing around a value >= +0 (2^-149 below the
    // normal range).
    auto grid = [](float v) {
        const int32_t be = static_cast<int32_t>(__builtin_bit_cast(uint32_t, v) >> 23);
        return (be > 0 ? be : 1) - 150;
    };
    const uint32_t nrec = static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(nfail)));
    float acc = s_prev;
    bool bad = false;
    uint32_t prev_units = 0;
    int32_t prev_after = sc.u[0];
    FailRec<SEG> cur = sc.rec[0];
    for (uint32_t i = 0; i <= nrec; ++i) {
        const FailRec<SEG> ahead = sc.rec[i < nrec ? i + 1 : nrec];
        const bool has_run = cur.u_before != kNoGrid;
        const float run = has_run ? __builtin_ldexpf(static_cast<float>(cur.units - prev_units), cur.u_before) : 0.0f;
        const float after = acc + run; // exact when the run stays in the state's binade
        bad = bad || (has_run && !(grid(acc) == prev_after && prev_after == cur.u_before && grid(after) == cur.u_before));
        acc = after;
#pragma unroll
        for (uint32_t j = 0; j < SEG; ++j) acc += cur.e[j];
        prev_units = cur.units;
        prev_after = cur.u_after;
        cur = ahead;
    }
    acc = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, acc)));
    if (!(acc < __builtin_inff())) { // NaN (the addends are at most 1: never +inf): final whatever the checks say
        st.finite = false;
        st.special = acc;
        return;
    }
    if (__builtin_amdgcn_readfirstlane(static_cast<int>(bad)) == 0) {
        const SeqState h = seq_state(acc);
        st.m = h.m;
        st.u = h.u;
        return;
    }
    // Not expected (the predictions carry a proven bound): the whole tile
    // again from its exact starting value, one addition at a time.
    acc = s_prev;
    for (uint32_t g = 0; g < NT; ++g) acc = walk_segment<SEG>(s_e, g, acc);
    acc = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, acc)));
    if (!(acc < __builtin_inff())) {
        st.finite = false;
        st.special = acc;
        return;
    }
    const SeqState h = seq_state(acc);
    st.m = h.m;
    st.u = h.u;
}

// kOneTile: the row fits one tile (ncols <= NT * SEG), so each thread keeps
// its exponentials in registers across the walk and writes y once.  Every
// pass issues a thread's SEG loads before using any of them (a store to y
// between loads would otherwise wait for each load in turn: x and y may be
// the same memory).
template <uint32_t NT, uint32_t SEG, bool kYRow, bool kOneTile>
__global__ __launch_bounds__(NT) void k_softmax_seq(OrdView xv, OrdView yv, uint64_t ncols, const float *x, float *y)
{
    constexpr uint32_t TILE = NT * SEG;
    constexpr uint32_t NW = NT / kWave;
    __shared__ uint64_t tab[32];
    __shared__ __align__(16) float s_e[TILE];
    __shared__ SeqScratch<NT, SEG> s_seq;
    __shared__ float s_red[NW];
    __shared__ float s_total;
    const uint32_t wave = threadIdx.x / kWave;
    const uint32_t lane = threadIdx.x % kWave;
    // the expf table: loaded by wave 0 ahead of the row, written to LDS after
    // the row's loads (the barrier after the maximum orders the table)
    uint64_t tab_word = 0;
    if (wave == 0) tab_word = kExp2Table[lane % 32];
    const uint64_t r = blockIdx.x;
    const int64_t xrow = row_offset(xv, r);
    const int64_t yrow = kYRow ? row_offset(yv, r) : 0;
    const int64_t xs0 = xv.st[0], ys0 = yv.st[0];
    auto yoff = [&](uint64_t c) { return kYRow ? yrow + static_cast<int64_t>(c) * ys0 : ord_index(yv, r * ncols + c); };
    // column j of this thread in the tile at t0 (clamped to the tile's first
    // column past its end: the loads stay unconditional and in bounds)
    auto col = [&](uint64_t t0, uint32_t n, uint32_t j) {
        const uint32_t c = threadIdx.x + NT * j;
        return t0 + (c < n ? c : 0u);
    };
    auto tile_n = [&](uint64_t t0) { return ncols - t0 < TILE ? static_cast<uint32_t>(ncols - t0) : TILE; };

    // 1. maximum (NaN never wins; NaN and infinities reach the sum instead)
    float v[SEG];
    float mx = -__builtin_inff();
    // Unit column strides (rows apart, columns contiguous: the common
    // strided case) address a row from one uniform base with 32-bit offsets.
    const bool unit = xs0 == 1 && (!kYRow || ys0 == 1);
    for (uint64_t t0 = 0; t0 < ncols; t0 += TILE) {
        const uint32_t n = tile_n(t0);
        if (unit) {
            const float *xp = x + xrow + static_cast<int64_t>(t0);
#pragma unroll
            for (uint32_t j = 0; j < SEG; ++j) {
                const uint32_t c = threadIdx.x + NT * j;
                v[j] = xp[c < n ? c : 0u];
            }
        } else {
#pragma unroll
            for (uint32_t j = 0; j < SEG; ++j) v[j] = x[xrow + static_cast<int64_t>(col(t0, n, j)) * xs0];
        }
#pragma unroll
        for (uint32_t j = 0; j < SEG; ++j) mx = threadIdx.x + NT * j < n ? __builtin_fmaxf(mx, v[j]) : mx;
    }
    if (threadIdx.x < 32) tab[threadIdx.x] = tab_word;
    mx = wave_max_dpp(mx);
    if (lane == 0) s_red[wave] = mx;
    __syncthreads();
    mx = s_red[0];
#pragma unroll
    for (uint32_t w = 1; w < NW; ++w) mx = __builtin_fmaxf(mx, s_red[w]);

    // 2. exponentials and the sequential sum
    SumState st{0u, -149, true, 0.0f};
    for (uint64_t t0 = 0; t0 < ncols; t0 += TILE) {
        const uint32_t n = tile_n(t0);
        if constexpr (!kOneTile) {
#pragma unroll
            for (uint32_t j = 0; j < SEG; ++j) v[j] = x[xrow + static_cast<int64_t>(col(t0, n, j)) * xs0];
        }
#pragma unroll
        for (uint32_t j = 0; j < SEG; ++j) {
            const uint32_t c = threadIdx.x + NT * j;
            // +0 past the row's end adds nothing to a sum that is never -0.
            // The exponential is computed for every lane (the clamped
            // column is in bounds) and selected: a branch per element would
            // serialise the table reads of the SEG exponentials.
            float ej = emel_expf_nonpos(v[j] - mx, tab);
            asm("" : "+v"(ej));
            v[j] = c < n ? ej : 0.0f;
            s_e[c] = v[j];
            if (!kOneTile && c < n) y[yoff(t0 + c)] = v[j];
        }
        if (threadIdx.x == 0) s_total = st.finite ? seq_value(st.m, st.u) : st.special; // the sum before the tile
        __syncthreads();
        const float s_prev = s_total;
        if (s_prev == s_prev) seq_tile_sum<NT, SEG>(s_e, s_seq, s_prev, st); // a NaN sum is final
        __syncthreads(); // s_e, s_seq and s_total are rewritten next
    }
    if (threadIdx.x == 0) s_total = st.finite ? seq_value(st.m, st.u) : st.special;
    __syncthreads();

    // 3. y = e / sum (sum >= 1, or NaN)
    const double recip = 1.0 / static_cast<double>(s_total);
    if constexpr (kOneTile) {
        const uint32_t n = static_cast<uint32_t>(ncols);
        if (unit && n == TILE) { // every column of every thread in the row: no per-element test
            float *yp = y + yrow;
#pragma unroll
            for (uint32_t j = 0; j < SEG; ++j) yp[threadIdx.x + NT * j] = div_by_recip(v[j], recip);
        } else {
#pragma unroll
            for (uint32_t j = 0; j < SEG; ++j) {
                const uint32_t c = threadIdx.x + NT * j;
                if (c < n) y[yoff(c)] = div_by_recip(v[j], recip);
            }
        }
    } else {
        for (uint64_t t0 = 0; t0 < ncols; t0 += TILE) {
            const uint32_t n = tile_n(t0);
#pragma unroll
            for (uint32_t j = 0; j < SEG; ++j) v[j] = y[yoff(col(t0, n, j))];
#pragma unroll
            for (uint32_t j = 0; j < SEG; ++j) {
                const uint32_t c = threadIdx.x + NT * j;
                if (c < n) y[yoff(t0 + c)] = div_by_recip(v[j], recip);
            }
        }
    }
}

// ---- host-side selection ---------------------------------------------------

bool contiguous(const Operand &p)
{
    int64_t expect = 1;
    for (int d = 0; d < 4; ++d) {
        if (p.ne[d] != 1 && p.st[d] != expect) return false;
        expect *= static_cast<int64_t>(p.ne[d]);
    }
    return true;
}

bool same_ne(const Operand &a, const Operand &b)
{
    for (int d = 0; d < 4; ++d)
        if (a.ne[d] != b.ne[d]) return false;
    return true;
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

OrdView ord_view(const Operand &p)
{
    OrdView v;
    for (int d = 0; d < 4; ++d) {
        v.ne[d] = p.ne[d];
        v.st[d] = p.st[d];
    }
    return v;
}

template <uint32_t NT, uint32_t SEG>
void launch_softmax_seq_nt(const Operand &x, const Operand &y, uint64_t rows, hipStream_t s)
{
    const uint64_t ncols = x.ne[0];
    const float *xp = static_cast<const float *>(x.data);
    float *yp = static_cast<float *>(y.data);
    const dim3 grid(static_cast<uint32_t>(rows));
    const bool one = ncols <= NT * SEG;
    if (y.ne[0] == ncols) {
        if (one) k_softmax_seq<NT, SEG, true, true><<<grid, NT, 0, s>>>(ord_view(x), ord_view(y), ncols, xp, yp);
        else k_softmax_seq<NT, SEG, true, false><<<grid, NT, 0, s>>>(ord_view(x), ord_view(y), ncols, xp, yp);
    } else {
        if (one) k_softmax_seq<NT, SEG, false, true><<<grid, NT, 0, s>>>(ord_view(x), ord_view(y), ncols, xp, yp);
        else k_softmax_seq<NT, SEG, false, false><<<grid, NT, 0, s>>>(ord_view(x), ord_view(y), ncols, xp, yp);
    }
}


template <RowOp OP, int NW, int NV, bool FULL>
void launch_vec(const RowGeo &g, const RowArgs &a, const MaskGeo &mg, hipStream_t s)
{
    constexpr uint32_t rows_per_block = kBlock / (NW * kWave);
    const uint32_t blocks = (g.rows + rows_per_block - 1) / rows_per_block;
    const float *x = static_cast<const float *>(a.x.data);
    float *y = static_cast<float *>(a.y.data);
    if (OP == RowOp::SoftMaxExt && mg.p)
        k_row_vec<OP, NW, NV, FULL, true><<<dim3(blocks), kBlock, 0, s>>>(g, x, y, a.w, mg, a.eps, a.scale);
    else
        k_row_vec<OP, NW, NV, FULL, false><<<dim3(blocks), kBlock, 0, s>>>(g, x, y, a.w, mg, a.eps, a.scale);
}

template <RowOp OP, int NW, int NV>
void launch_fit(const RowGeo &g, const RowArgs &a, const MaskGeo &mg, hipStream_t s)
{
    if (g.ncols / 4 == static_cast<uint32_t>(NW * kWave * NV)) launch_vec<OP, NW, NV, true>(g, a, mg, s);
    else launch_vec<OP, NW, NV, false>(g, a, mg, s);
}

// One wave per row in a 64-thread workgroup, the row exactly NV float4 per
// lane (the normalisations only: no mask).
template <RowOp OP, int NV>
void launch_wave_rows(const RowGeo &g, const RowArgs &a, hipStream_t s)
{
    k_row_vec<OP, 1, NV, true, false, kWave><<<dim3(g.rows), kWave, 0, s>>>(
        g, static_cast<const float *>(a.x.data), static_cast<float *>(a.y.data), a.w, MaskGeo{}, a.eps, a.scale);
}

// Rows of up to 1024 columns: a wave per row; up to 16384 columns: a
// workgroup per row with the row in registers; wider: a workgroup per row
// streaming in passes.  Measured on MI355X: the normalisations of 1536 to
// 4096 rows of exactly 2048, 4096 or 8192 columns run faster with one wave
// per row in 64-thread workgroups (11.3 against 12.9 us for rms_norm at
// [4096, 2048]; 1.5 to 4 waves per SIMD, each with its whole row in
// flight).  Fewer rows leave SIMDs idle and more rows favour four
// waves per row, and the softmaxes' two reductions and exponentials favour
// four waves per row at every row count.
template <RowOp OP>
void launch_vec_nv(const RowGeo &g, const RowArgs &a, const MaskGeo &mg, hipStream_t s)
{
    const uint32_t nv = g.ncols / 4;
    if constexpr (kRmsOp<OP> || kNormOp<OP>) {
        if (g.rows >= 1536 && g.rows <= 4096) {
            if (nv == 8 * kWave) return launch_wave_rows<OP, 8>(g, a, s);
            if (nv == 16 * kWave) return launch_wave_rows<OP, 16>(g, a, s);
            if (nv == 32 * kWave) return launch_wave_rows<OP, 32>(g, a, s);
        }
    }
    if (nv <= 1 * kWave) launch_fit<OP, 1, 1>(g, a, mg, s);
    else if (nv <= 2 * kWave) launch_fit<OP, 1, 2>(g, a, mg, s);
    else if (nv <= 4 * kWave) launch_fit<OP, 1, 4>(g, a, mg, s);
    else if (nv <= 2 * kBlock) launch_fit<OP, 4, 2>(g, a, mg, s);
    else if (nv <= 4 * kBlock) launch_fit<OP, 4, 4>(g, a, mg, s);
    else if (nv <= 8 * kBlock) launch_fit<OP, 4, 8>(g, a, mg, s);
    else if (nv <= 16 * kBlock) launch_fit<OP, 4, 16>(g, a, mg, s);
    else launch_vec<OP, 4, 0, false>(g, a, mg, s);
}

} // namespace

hipError_t launch_softmax_seq(const Operand &x, const Operand &y, hipStream_t s)
{
    const uint64_t ncols = x.ne[0];
    uint64_t count = 1;
    for (int d = 0; d < 4; ++d) count *= x.ne[d];
    if (count == 0 || ncols == 0) return hipSuccess;
    const uint64_t rows = count / ncols;
    if (ncols <= kSeqShort) {
        const uint64_t blocks = (rows + kBlock - 1) / kBlock;
        if (blocks > 0x7fffffffull) return hipErrorInvalidValue;
        k_softmax_lane<<<dim3(static_cast<uint32_t>(blocks)), kBlock, 0, s>>>(
            ord_view(x), ord_view(y), rows, ncols, static_cast<const float *>(x.data), static_cast<float *>(y.data));
        return hipGetLastError();
    }
    if (rows > 0x7fffffffull) return hipErrorInvalidValue; // one workgroup per row
    // (threads, addends per segment) by row width, measured on MI355X: one
    // tile covers rows up to 16384 columns, wider rows stream tiles of 16384
    if (ncols <= 512) launch_softmax_seq_nt<64, 8>(x, y, rows, s);
    else if (ncols <= 1024) launch_softmax_seq_nt<64, 16>(x, y, rows, s);
    else if (ncols <= 2048) launch_softmax_seq_nt<256, 8>(x, y, rows, s);
    else if (ncols <= 4096) launch_softmax_seq_nt<256, 16>(x, y, rows, s);
    else if (ncols <= 8192) launch_softmax_seq_nt<512, 16>(x, y, rows, s);
    else launch_softmax_seq_nt<1024, 16>(x, y, rows, s);
    return hipGetLastError();
}

hipError_t launch_rows(const RowArgs &a, hipStream_t s)
{
    const bool soft = a.op == RowOp::SoftMax || a.op == RowOp::SoftMaxExt;
    const uint64_t ncols = a.x.ne[0];
    uint64_t count = 1;
    for (int d = 0; d < 4; ++d) count *= a.x.ne[d];
    if (count == 0 || ncols == 0) return hipSuccess;
    const uint64_t rows = count / ncols;

    // The strided soft_max keeps the reference's sequential f32 sum.
    if (a.op == RowOp::SoftMax && !a.dense_sum) return launch_softmax_seq(a.x, a.y, s);

    // Vectorized rows: contiguous dim 0, 16-byte aligned row starts, and the
    // destination row r holding the same columns as the source row r.
    auto strides4 = [](const Operand &p) {
        for (int d = 1; d < 4; ++d)
            if (p.ne[d] != 1 && p.st[d] % 4 != 0) return false;
        return true;
    };
    const bool rows_match = same_ne(a.x, a.y) || (contiguous(a.x) && contiguous(a.y));
    const bool w_ok = a.op != RowOp::RmsNormMul || (a.w_st0 == 1 && aligned16(a.w));
    const bool mask_ok = a.op != RowOp::SoftMaxExt || a.mask == nullptr || (reinterpret_cast<uintptr_t>(a.mask) & 7u) == 0;
    const bool vec = ncols % 4 == 0 && a.x.st[0] == 1 && a.y.st[0] == 1 && strides4(a.x) && strides4(a.y) &&
                     aligned16(a.x.data) && aligned16(a.y.data) && rows_match && w_ok && mask_ok &&
                     rows < 0xffffffffull && ncols < 0xffffffffull;
    if (vec) {
        // When x and y differ in shape but are both dense, row r of each is
        // the same linear range: describe both with x's extents.
        RowGeo g{};
        g.rows = static_cast<uint32_t>(rows);
        g.ncols = static_cast<uint32_t>(ncols);
        g.ne1 = FastDiv(static_cast<uint32_t>(a.x.ne[1]));
        g.ne2 = FastDiv(static_cast<uint32_t>(a.x.ne[2]));
        const bool linear = !same_ne(a.x, a.y);
        for (int d = 0; d < 4; ++d) {
            g.x_st[d] = a.x.st[d];
            g.y_st[d] = linear ? a.x.st[d] : a.y.st[d];
        }
        if (linear) { // both dense: use x's row-major strides for y
            int64_t e = 1;
            for (int d = 0; d < 4; ++d) {
                g.x_st[d] = e;
                g.y_st[d] = e;
                e *= static_cast<int64_t>(a.x.ne[d]);
            }
        }
        MaskGeo mg{};
        mg.m2 = FastDiv(1);
        mg.m3 = FastDiv(1);
        if (a.op == RowOp::SoftMaxExt) {
            mg.p = a.mask;
            mg.ne1 = static_cast<uint32_t>(a.x.ne[1]);
            mg.m2 = FastDiv(static_cast<uint32_t>(a.mask_ne2 ? a.mask_ne2 : 1));
            mg.m3 = FastDiv(static_cast<uint32_t>(a.mask_ne3 ? a.mask_ne3 : 1));
        }
        switch (a.op) {
        case RowOp::RmsNorm: launch_vec_nv<RowOp::RmsNorm>(g, a, mg, s); break;
        case RowOp::RmsNormMul: launch_vec_nv<RowOp::RmsNormMul>(g, a, mg, s); break;
        case RowOp::Norm: launch_vec_nv<RowOp::Norm>(g, a, mg, s); break;
        case RowOp::SoftMax: launch_vec_nv<RowOp::SoftMax>(g, a, mg, s); break;
        case RowOp::SoftMaxExt: launch_vec_nv<RowOp::SoftMaxExt>(g, a, mg, s); break;
        case RowOp::GenRmsNorm: launch_vec_nv<RowOp::GenRmsNorm>(g, a, mg, s); break;
        case RowOp::GenNorm: launch_vec_nv<RowOp::GenNorm>(g, a, mg, s); break;
        }
        return hipGetLastError();
    }
    // the generic envelope's norms take this path only for vectorisable
    // rows; their caller has a kernel for every other layout
    if (a.op == RowOp::GenRmsNorm || a.op == RowOp::GenNorm) return hipErrorNotSupported;

    const uint64_t blocks = (rows + (kBlock / kWave) - 1) / (kBlock / kWave);
    if (blocks > 0x7fffffffull) return hipErrorInvalidConfiguration;
    const dim3 grid(static_cast<uint32_t>(blocks));
    const float *x = static_cast<const float *>(a.x.data);
    float *y = static_cast<float *>(a.y.data);
    if (soft) {
        MaskGeo mg{};
        if (a.op == RowOp::SoftMaxExt) {
            mg.p = a.mask;
            mg.ne1 = static_cast<uint32_t>(a.x.ne[1]);
            mg.m2 = FastDiv(static_cast<uint32_t>(a.mask_ne2 ? a.mask_ne2 : 1));
            mg.m3 = FastDiv(static_cast<uint32_t>(a.mask_ne3 ? a.mask_ne3 : 1));
            k_softmax_generic<true><<<grid, kBlock, 0, s>>>(ord_view(a.x), ord_view(a.y), rows, ncols, x, y, mg,
                                                             a.scale);
        } else {
            k_softmax_generic<false><<<grid, kBlock, 0, s>>>(ord_view(a.x), ord_view(a.y), rows, ncols, x, y, mg,
                                                              1.0f);
        }
    } else if (a.op == RowOp::RmsNorm) {
        k_row_generic<RowOp::RmsNorm><<<grid, kBlock, 0, s>>>(ord_view(a.x), ord_view(a.y), rows, ncols, x, y, a.w,
                                                               a.w_st0, a.eps);
    } else if (a.op == RowOp::RmsNormMul) {
        k_row_generic<RowOp::RmsNormMul><<<grid, kBlock, 0, s>>>(ord_view(a.x), ord_view(a.y), rows, ncols, x, y,
                                                                  a.w, a.w_st0, a.eps);
    } else {
        k_row_generic<RowOp::Norm><<<grid, kBlock, 0, s>>>(ord_view(a.x), ord_view(a.y), rows, ncols, x, y, a.w,
                                                            a.w_st0, a.eps);
    }
    return hipGetLastError();
}

// ---- OpGroupNorm (group_norm.rs:197-241) -----------------------------------------
//
// One workgroup per (batch, group).  The group's W*H*(C/groups) elements are
// visited three times -- f64 sum, f64 sum of the squared f32-centered
// values, then (x - mean) * scale -- at their (column, row, channel, batch)
// offsets, so any element strides work; the later passes hit L2.  The f64
// sums run as a tree instead of the reference's sequential loop, the same
// trade as rms_norm.

namespace {

struct GroupGeo {
    uint32_t groups;
    uint32_t cpg;          // channels per group
    uint64_t n;            // elements per group
    FastDiv w, wh;         // W and W*H
    int64_t x_st[4], y_st[4];
};

__device__ __forceinline__ double block_sum4(double v, double *lds)
{
    v = wave_sum_dpp(v);
    const uint32_t wave = threadIdx.x / kWave;
    if (threadIdx.x % kWave == 0) lds[wave] = v;
    __syncthreads();
    const double t = (lds[0] + lds[1]) + (lds[2] + lds[3]);
    __syncthreads(); // lds is reused by the next reduction
    return t;
}

__global__ __launch_bounds__(kBlock) void k_group_norm(GroupGeo g, const float *x, float *y, float eps)
{
    static_assert(kBlock == 4 * kWave, "block_sum4 combines four waves");
    __shared__ double lds[kBlock / kWave];
    const uint32_t b = blockIdx.x / g.groups;
    const uint32_t grp = blockIdx.x - b * g.groups;
    const uint32_t ch0 = grp * g.cpg;
    auto offset = [&](const int64_t *st, uint32_t e) {
        const uint32_t c = g.wh.div(e);
        const uint32_t rem = e - c * g.wh.d;
        const uint32_t row = g.w.div(rem);
        const uint32_t col = rem - row * g.w.d;
        return static_cast<int64_t>(col) * st[0] + static_cast<int64_t>(row) * st[1] +
               static_cast<int64_t>(ch0 + c) * st[2] + static_cast<int64_t>(b) * st[3];
    };
    const uint32_t n = static_cast<uint32_t>(g.n);
    double sum = 0.0;
    for (uint32_t e = threadIdx.x; e < n; e += kBlock) sum += static_cast<double>(x[offset(g.x_st, e)]);
    sum = block_sum4(sum, lds);
    const float mean = static_cast<float>(sum / static_cast<double>(g.n));
    double var = 0.0;
    for (uint32_t e = threadIdx.x; e < n; e += kBlock) {
        const float c = x[offset(g.x_st, e)] - mean;
        var += static_cast<double>(c) * static_cast<double>(c);
    }
    var = block_sum4(var, lds);
    const float scale = 1.0f / __builtin_sqrtf(static_cast<float>(var / static_cast<double>(g.n)) + eps);
    for (uint32_t e = threadIdx.x; e < n; e += kBlock) y[offset(g.y_st, e)] = (x[offset(g.x_st, e)] - mean) * scale;
}

} // namespace

hipError_t launch_group_norm(const Operand &x, const Operand &y, uint32_t groups, float eps, hipStream_t s)
{
    const uint64_t w = x.ne[0], h = x.ne[1], c = x.ne[2], bt = x.ne[3];
    if (groups == 0 || c % groups != 0) return hipErrorInvalidValue;
    GroupGeo g{};
    g.groups = groups;
    g.cpg = static_cast<uint32_t>(c / groups);
    g.n = w * h * g.cpg;
    const uint64_t blocks = static_cast<uint64_t>(groups) * bt;
    if (w * h >= 0xffffffffull || g.n >= 0xffffffffull || blocks >= 0x7fffffffull) return hipErrorInvalidValue;
    g.w = FastDiv(static_cast<uint32_t>(w));
    g.wh = FastDiv(static_cast<uint32_t>(w * h));
    for (int d = 0; d < 4; ++d) {
        g.x_st[d] = x.st[d];
        g.y_st[d] = y.st[d];
    }
    k_group_norm<<<dim3(static_cast<uint32_t>(blocks)), kBlock, 0, s>>>(g, static_cast<const float *>(x.data),
                                                                         static_cast<float *>(y.data), eps);
    return hipGetLastError();
}

} // namespace emel
