// reduce.hip -- gfx950 kernels for sum_rows (reductions.rs:684-700),
// per-row argmax (one OpArgmax per row, reductions.rs:715-730) and the
// whole-tensor sum / mean / argmax (reductions.rs:670-730).
//
// Long rows (the 151,936-wide logits rows) are split into `chunks` column
// ranges, one workgroup each, so the grid fills all 256 CUs.  Each
// workgroup reduces its range (f64 sums; (value, index) maxima) and writes
// one partial; a second kernel with one wave per row combines the row's
// partials in a fixed tree order.  The kernel boundary makes the partials
// visible across XCDs without in-kernel fences: an agent-scope fence costs
// an L2 write-back and invalidate per workgroup on gfx950, and a single pass
// that hands partials over through agent-scope atomics measured 1.3-3.6x
// slower than the second launch (contention on the per-row counter).
// Results are deterministic run to run.
//
// argmax keeps the reference's sequential strict-> scan semantics: the
// winner is the lowest index among the maximal non-NaN values, NaNs never
// win, and a NaN in column 0 makes the result 0 (nothing compares greater
// than the initial NaN).
#include <type_traits>

#include "common.hpp"
#include "launch.hpp"

namespace emel {
namespace {

struct ArgPart {
    float v;
    uint32_t i;
};

struct RedGeo {
    uint32_t rows;
    uint32_t chunks;
    uint64_t ncols;       // columns per row (whole tensor: the element count)
    uint64_t chunk_cols;  // columns per chunk (a multiple of 4 when vectorized)
    FastDiv ne1, ne2;     // row -> (i1, i2, i3)
    int64_t x_st[4];
    int64_t d_st[4];
    uint64_t ne[4];       // source extents (ordinal mode)
    uint32_t mode;        // 0: float4 rows, 1: scalar rows (x_st[0]), 2: ordinal decode (rows == 1)
};

enum : uint32_t { kModeVec = 0, kModeScalar = 1, kModeOrdinal = 2 };

__device__ __forceinline__ int64_t ordinal_offset(const RedGeo &g, uint64_t k)
{
    int64_t off = 0;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        off += static_cast<int64_t>(k % g.ne[d]) * g.x_st[d];
        k /= g.ne[d];
    }
    return off;
}

template <RedOp OP>
struct Acc {
    static constexpr bool kArg = OP == RedOp::ArgmaxRows || OP == RedOp::Argmax;
};

// Per-thread accumulation over [c0, c1) of row r.
template <RedOp OP>
__device__ __forceinline__ void accumulate(const RedGeo &g, const float *x, int64_t base, uint64_t c0, uint64_t c1,
                                           double &sum, float &bv, uint32_t &bi)
{
    constexpr bool kArg = Acc<OP>::kArg;
    auto take = [&](float v, uint64_t c) {
        if constexpr (kArg) {
            if (v > bv) { // lanes scan their columns in increasing order
                bv = v;
                bi = static_cast<uint32_t>(c);
            }
        } else {
            sum += static_cast<double>(v);
        }
    };
    if (g.mode == kModeVec) {
        const float4 *x4 = reinterpret_cast<const float4 *>(x + base);
        auto take4 = [&](const float4 &q, uint64_t c) {
            if constexpr (kArg) {
                take(q.x, c);
                take(q.y, c + 1);
                take(q.z, c + 2);
                take(q.w, c + 3);
            } else {
                sum += (static_cast<double>(q.x) + static_cast<double>(q.y)) +
                       (static_cast<double>(q.z) + static_cast<double>(q.w));
            }
        };
        // kUnroll non-temporal loads in flight per thread (each byte is read
        // once), then taken in column order
        constexpr int kUnroll = 4;
        const uint64_t vend = c1 / 4;
        uint64_t v = c0 / 4 + threadIdx.x;
        for (; v + (kUnroll - 1) * kBlock < vend; v += kUnroll * kBlock) {
            float4 q[kUnroll];
#pragma unroll
            for (int j = 0; j < kUnroll; ++j) q[j] = ld_nt(x4 + v + j * kBlock);
#pragma unroll
            for (int j = 0; j < kUnroll; ++j) take4(q[j], 4 * (v + j * kBlock));
        }
        for (; v < vend; v += kBlock) take4(ld_nt(x4 + v), 4 * v);
    } else if (g.mode == kModeScalar) {
        for (uint64_t c = c0 + threadIdx.x; c < c1; c += kBlock) take(x[base + static_cast<int64_t>(c) * g.x_st[0]], c);
    } else {
        for (uint64_t c = c0 + threadIdx.x; c < c1; c += kBlock) take(x[ordinal_offset(g, c)], c);
    }
}

// Writes the row result from its combined (sum | (value, index)) word.
// argmax: `first` is the row's column 0 (a NaN there makes the result 0).
template <RedOp OP>
__device__ __forceinline__ void write_result(const RedGeo &g, float first, void *dst, uint32_t row, uint64_t packed)
{
    constexpr bool kArg = Acc<OP>::kArg;
    uint32_t i1 = 0, i2 = 0, i3 = 0;
    if (g.mode != kModeOrdinal) {
        const uint32_t t = g.ne1.div(row);
        i1 = row - t * g.ne1.d;
        i3 = g.ne2.div(t);
        i2 = t - i3 * g.ne2.d;
    }
    const int64_t doff = static_cast<int64_t>(i1) * g.d_st[1] + static_cast<int64_t>(i2) * g.d_st[2] +
                         static_cast<int64_t>(i3) * g.d_st[3];
    if constexpr (kArg) {
        const ArgPart p = __builtin_bit_cast(ArgPart, packed);
        // column 0 NaN: the sequential scan never replaces it
        const uint64_t idx = (first != first || p.i == 0xffffffffu) ? 0 : p.i;
        const float fidx = static_cast<float>(idx); // the reference stores the index as f32
        if constexpr (OP == RedOp::ArgmaxRows) static_cast<int32_t *>(dst)[doff] = static_cast<int32_t>(fidx);
        else static_cast<float *>(dst)[doff] = fidx;
    } else {
        const double t = __builtin_bit_cast(double, packed);
        if constexpr (OP == RedOp::Mean)
            static_cast<float *>(dst)[doff] = static_cast<float>(t / static_cast<double>(g.ncols));
        else
            static_cast<float *>(dst)[doff] = static_cast<float>(t);
    }
}

// Pass 1: workgroup (row, chunk) reduces its column range.  With one chunk
// per row it writes the result; otherwise it writes its partial word.
template <RedOp OP>
__global__ __launch_bounds__(kBlock) void k_reduce(RedGeo g, const float *x, void *dst, uint64_t *part)
{
    constexpr bool kArg = Acc<OP>::kArg;
    __shared__ double s_sum[kBlock / kWave];
    __shared__ float s_v[kBlock / kWave];
    __shared__ uint32_t s_i[kBlock / kWave];

    const uint32_t row = blockIdx.x / g.chunks;
    const uint32_t chunk = blockIdx.x - row * g.chunks;
    const uint32_t wave = threadIdx.x / kWave;
    const uint32_t lane = threadIdx.x % kWave;

    int64_t base = 0;
    if (g.mode != kModeOrdinal) {
        const uint32_t t = g.ne1.div(row);
        const uint32_t i1 = row - t * g.ne1.d;
        const uint32_t i3 = g.ne2.div(t);
        const uint32_t i2 = t - i3 * g.ne2.d;
        base = static_cast<int64_t>(i1) * g.x_st[1] + static_cast<int64_t>(i2) * g.x_st[2] +
               static_cast<int64_t>(i3) * g.x_st[3];
    }
    const uint64_t c0 = static_cast<uint64_t>(chunk) * g.chunk_cols;
    const uint64_t c1 = c0 + g.chunk_cols < g.ncols ? c0 + g.chunk_cols : g.ncols;

    // argmax: the row's column 0, read by the chunk-0 workgroup while its
    // range loads are in flight (a NaN there decides the row)
    float first = 0.0f;
    if constexpr (kArg) {
        if (chunk == 0 && threadIdx.x == 0) first = g.mode == kModeOrdinal ? x[ordinal_offset(g, 0)] : x[base];
    }

    double sum = 0.0;
    float bv = -__builtin_inff();
    uint32_t bi = 0xffffffffu; // "no candidate": loses every tie on index
    accumulate<OP>(g, x, base, c0, c1, sum, bv, bi);

    if constexpr (kArg) {
        wave_argmax(bv, bi);
        if (lane == 0) {
            s_v[wave] = bv;
            s_i[wave] = bi;
        }
    } else {
        sum = wave_sum(sum);
        if (lane == 0) s_sum[wave] = sum;
    }
    __syncthreads();
    if (threadIdx.x != 0) return;
    uint64_t packed;
    if constexpr (kArg) {
        for (int w = 1; w < kBlock / kWave; ++w) argmax_merge(s_v[0], s_i[0], s_v[w], s_i[w]);
        packed = __builtin_bit_cast(uint64_t, ArgPart{s_v[0], s_i[0]});
        // Split rows: a NaN in column 0 makes chunk 0's partial (+inf, 0),
        // which every other partial loses to (greater value, or equal value
        // and higher index), so the combined index is 0.
        if (g.chunks > 1 && chunk == 0 && first != first)
            packed = __builtin_bit_cast(uint64_t, ArgPart{__builtin_inff(), 0u});
    } else {
        double t = s_sum[0];
        for (int w = 1; w < kBlock / kWave; ++w) t += s_sum[w];
        packed = __builtin_bit_cast(uint64_t, t);
    }
    if (g.chunks == 1) write_result<OP>(g, first, dst, row, packed);
    else part[blockIdx.x] = packed;
}

// Pass 2: one wave per row combines the row's partials (lane l takes
// chunks l, l+64, ...; then a fixed butterfly) and writes the result.
template <RedOp OP>
__global__ __launch_bounds__(kBlock) void k_reduce_finish(RedGeo g, void *dst, const uint64_t *part)
{
    constexpr bool kArg = Acc<OP>::kArg;
    const uint32_t row = blockIdx.x * (kBlock / kWave) + threadIdx.x / kWave;
    const uint32_t lane = threadIdx.x % kWave;
    if (row >= g.rows) return;
    double tsum = 0.0;
    float tv = -__builtin_inff();
    uint32_t ti = 0xffffffffu;
    for (uint32_t c = lane; c < g.chunks; c += kWave) {
        const uint64_t q = part[static_cast<uint64_t>(row) * g.chunks + c];
        if constexpr (kArg) {
            const ArgPart p = __builtin_bit_cast(ArgPart, q);
            argmax_merge(tv, ti, p.v, p.i);
        } else {
            tsum += __builtin_bit_cast(double, q);
        }
    }
    uint64_t packed;
    if constexpr (kArg) {
        wave_argmax(tv, ti);
        packed = __builtin_bit_cast(uint64_t, ArgPart{tv, ti});
    } else {
        tsum = wave_sum(tsum);
        packed = __builtin_bit_cast(uint64_t, tsum);
    }
    // column 0 was folded into chunk 0's partial by pass 1
    if (lane == 0) write_result<OP>(g, 0.0f, dst, row, packed);
}

constexpr uint32_t kTargetBlocks = 2048; // 8 workgroups per CU on 256 CUs
constexpr uint64_t kMinChunkCols = 4 * kBlock; // one float4 per thread at least

bool plan(const RedArgs &a, RedGeo &g)
{
    g = RedGeo{};
    const bool whole = a.op == RedOp::Sum || a.op == RedOp::Mean || a.op == RedOp::Argmax;
    uint64_t count = 1;
    for (int d = 0; d < 4; ++d) {
        g.ne[d] = a.x.ne[d];
        g.x_st[d] = a.x.st[d];
        g.d_st[d] = a.dst_view.st[d];
        count *= a.x.ne[d];
    }
    // contiguous row-major (extent-1 strides ignored)
    bool dense = true;
    int64_t e = 1;
    for (int d = 0; d < 4; ++d) {
        if (a.x.ne[d] != 1 && a.x.st[d] != e) dense = false;
        e *= static_cast<int64_t>(a.x.ne[d]);
    }
    const bool aligned = (reinterpret_cast<uintptr_t>(a.x.data) & 15u) == 0;
    if (whole) {
        g.rows = 1;
        g.ncols = count;
        g.ne1 = FastDiv(1);
        g.ne2 = FastDiv(1);
        for (int d = 0; d < 4; ++d) g.d_st[d] = 0;
        if (dense) {
            g.x_st[0] = 1;
            g.x_st[1] = g.x_st[2] = g.x_st[3] = 0;
            g.mode = (aligned && count % 4 == 0) ? kModeVec : kModeScalar;
        } else {
            g.mode = kModeOrdinal;
        }
    } else {
        const uint64_t rows = count / a.x.ne[0];
        if (rows >= 0xffffffffull || a.x.ne[1] >= 0xffffffffull || a.x.ne[2] >= 0xffffffffull) return false;
        g.rows = static_cast<uint32_t>(rows);
        g.ncols = a.x.ne[0];
        g.ne1 = FastDiv(static_cast<uint32_t>(a.x.ne[1]));
        g.ne2 = FastDiv(static_cast<uint32_t>(a.x.ne[2]));
        bool st4 = true;
        for (int d = 1; d < 4; ++d)
            if (a.x.ne[d] != 1 && a.x.st[d] % 4 != 0) st4 = false;
        g.mode = (a.x.st[0] == 1 && g.ncols % 4 == 0 && aligned && st4) ? kModeVec : kModeScalar;
    }
    if ((a.op == RedOp::ArgmaxRows || a.op == RedOp::Argmax) && g.ncols >= 0xffffffffull) return false;
    uint64_t want = (kTargetBlocks + g.rows - 1) / g.rows;
    uint64_t chunk = (g.ncols + want - 1) / want;
    if (chunk < kMinChunkCols) chunk = kMinChunkCols;
    chunk = (chunk + 3) & ~uint64_t{3};
    uint64_t chunks = (g.ncols + chunk - 1) / chunk;
    if (chunks == 0) chunks = 1;
    if (static_cast<uint64_t>(g.rows) * chunks > 0x7fffffffull) return false;
    g.chunks = static_cast<uint32_t>(chunks);
    g.chunk_cols = chunk;
    return true;
}

} // namespace

uint64_t reduce_workspace_bytes(const RedArgs &a)
{
    RedGeo g;
    if (!plan(a, g) || g.chunks == 1) return 0;
    return static_cast<uint64_t>(g.rows) * g.chunks * sizeof(uint64_t);
}

hipError_t launch_reduce(const RedArgs &a, hipStream_t s)
{
    RedGeo g;
    if (!plan(a, g)) return hipErrorInvalidValue;
    const float *x = static_cast<const float *>(a.x.data);
    uint64_t *part = static_cast<uint64_t *>(a.workspace);
    if (g.chunks > 1 && !part) return hipErrorInvalidValue;
    const dim3 grid(g.rows * g.chunks);
    const dim3 fgrid((g.rows + (kBlock / kWave) - 1) / (kBlock / kWave));
    auto run = [&](auto op_tag) {
        constexpr RedOp OP = decltype(op_tag)::value;
        k_reduce<OP><<<grid, kBlock, 0, s>>>(g, x, a.dst, part);
        if (g.chunks > 1) k_reduce_finish<OP><<<fgrid, kBlock, 0, s>>>(g, a.dst, part);
    };
    switch (a.op) {
    case RedOp::SumRows: run(std::integral_constant<RedOp, RedOp::SumRows>{}); break;
    case RedOp::ArgmaxRows: run(std::integral_constant<RedOp, RedOp::ArgmaxRows>{}); break;
    case RedOp::Sum: run(std::integral_constant<RedOp, RedOp::Sum>{}); break;
    case RedOp::Mean: run(std::integral_constant<RedOp, RedOp::Mean>{}); break;
    case RedOp::Argmax: run(std::integral_constant<RedOp, RedOp::Argmax>{}); break;
    }
    return hipGetLastError();
}

} // namespace emel
