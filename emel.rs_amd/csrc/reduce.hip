// reduce.hip -- gfx950 kernels for sum_rows (reductions.rs:684-700),
// per-row argmax (one OpArgmax per row, reductions.rs:715-730) and the
// whole-tensor sum / mean / argmax (reductions.rs:670-730).
//
// One launch.  Long rows (the 151,936-wide logits rows) are split into
// `chunks` column ranges, one workgroup each, so the grid fills all 256 CUs.
// Each workgroup reduces its range (f64 sums; (value, index) maxima) and
// publishes one partial word; the last workgroup of a row to finish merges
// the row's partials and writes the result.
//
// The hand-over uses agent-scope relaxed atomics only, no fences:
//   - a partial is stored with an agent-scope store (global_store ... sc1,
//     written through to the coherence point every XCD reads from), and
//     `s_waitcnt vmcnt(0)` waits for its acknowledgement;
//   - then the workgroup adds 1 to its row's arrival counter (agent-scope
//     atomic add with return).  The workgroup that sees count - 1 is last:
//     every other partial of the row was acknowledged before its writer's
//     increment, which came before this one;
//   - the last workgroup reads the partials with agent-scope loads (sc1,
//     served from the coherence point), merges them in a fixed lane order
//     (so the result does not depend on which workgroup came last), writes
//     the result and stores 0 back into the counter for the next launch.
// This is the release/acquire pair with the L2 write-back and invalidate
// left out: every value handed over is itself written and read at the
// coherence point, so nothing else needs to be made visible.
//
// Counters live on separate cache lines (a line sees about 32 increments
// per launch): increments of one line are serialised at the coherence
// point, and 64 row counters packed into 256 bytes measured 2x slower.  A
// row with more than 64 chunks merges in two levels: groups of up to 64
// chunks, then the groups.
//
// argmax keeps the reference's sequential strict-> scan semantics: the
// winner is the lowest index among the maximal non-NaN values, NaNs never
// win, and a NaN in column 0 makes the result 0 (nothing compares greater
// than the initial NaN).
#include <mutex>
#include <type_traits>

#include "common.hpp"
#include "launch.hpp"

namespace emel {
namespace {

struct ArgPart {
    float v;
    uint32_t i;
};

constexpr uint32_t kMaxGroup = kWave;          // chunks merged by one wave
constexpr uint32_t kMaxChunks = kMaxGroup * kMaxGroup;
constexpr uint32_t kLineWords = 64;            // 256 bytes of u32 counters
#ifndef RED_BATCH
constexpr int kRedBatch = 5;                   // float4 loads in flight per thread
#else
constexpr int kRedBatch = RED_BATCH;
#endif

struct RedGeo {
    uint32_t rows;
    uint32_t chunks;      // chunks per row
    uint32_t groups;      // first-level groups per row (1: one level)
    uint32_t group_size;  // chunks per group (<= 64)
    uint32_t cstride;     // first-level counter stride, in u32 words
    uint64_t ncols;       // columns per row (whole tensor: the element count)
    uint64_t chunk_cols;  // columns per chunk (a multiple of 4 when vectorized)
    FastDiv ne1, ne2;     // row -> (i1, i2, i3)
    int64_t x_st[4];
    int64_t d_st[4];
    uint64_t ne[4];       // source extents (ordinal mode)
    uint32_t mode;        // 0: float4 rows, 1: scalar rows (x_st[0]), 2: ordinal decode (rows == 1)
    // scratch layout: byte offsets of the two partial arrays in the partials
    // buffer, and of the two counter arrays in the counters buffer
    uint64_t off_part1, off_part2, off_cnt1, off_cnt2;
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

// Per-thread accumulation over [c0, c1) of row r.  `first` receives the
// first element the thread reads (for thread 0 of the row's chunk 0: column
// 0, which the argmax NaN rule needs).
template <RedOp OP>
__device__ __forceinline__ void accumulate(const RedGeo &g, const float *x, int64_t base, uint64_t c0, uint64_t c1,
                                           double &sum, float &bv, uint32_t &bi, float &first)
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
    if (!kArg && g.mode == kModeVec) { // argmax's vector mode is argmax_chunk_vec
        // The range is read through a buffer descriptor bounded to it: a
        // load past its end returns zeros without touching memory.  Each
        // batch issues kBatch non-temporal 128-bit loads per thread
        // unconditionally (one round trip; no lane-dependent branches, which
        // would serialise the loads).  Zeros leave a sum unchanged: a partial
        // sum that starts at +0.0 is never -0.0.
        constexpr int kBatch = kRedBatch;
        const uint32_t nvec = static_cast<uint32_t>((c1 - c0) / 4);
        const BufRsrc r = buffer_rsrc(x + base + c0, nvec * 16u);
        for (uint32_t v0 = 0; v0 < nvec; v0 += kBatch * kBlock) {
            float4 q[kBatch];
#pragma unroll
            for (int j = 0; j < kBatch; ++j) q[j] = ld_buf_nt(r, (v0 + j * kBlock + threadIdx.x) * 16u);
#pragma unroll
            for (int j = 0; j < kBatch; ++j)
                sum += (static_cast<double>(q[j].x) + static_cast<double>(q[j].y)) +
                       (static_cast<double>(q[j].z) + static_cast<double>(q[j].w));
        }
    } else if (g.mode == kModeScalar) {
        for (uint64_t c = c0 + threadIdx.x; c < c1; c += kBlock) {
            const float v = x[base + static_cast<int64_t>(c) * g.x_st[0]];
            if (c == c0 + threadIdx.x) first = v;
            take(v, c);
        }
    } else {
        for (uint64_t c = c0 + threadIdx.x; c < c1; c += kBlock) {
            const float v = x[ordinal_offset(g, c)];
            if (c == c0 + threadIdx.x) first = v;
            take(v, c);
        }
    }
}

// ---- argmax over a 128-bit-vectorised chunk ----------------------------------
//
// The per-element form above (compare, then select value and index) is a
// dependent chain of 3 instructions per element.  The vector path splits it:
//   1. each lane takes the maximum of its batch's non-NaN values with a
//      v_max3_f32 tree (independent operations, ~1 instruction per 2
//      elements);
//   2. the workgroup forms the chunk maximum M of those lane maxima;
//   3. only lanes whose maximum equals M look for the first column holding
//      a value equal to M (usually one lane per chunk).
// This is the reference's strict-> scan: its winner is the first column
// whose value equals the maximum of the non-NaN values (float equality, so
// -0.0 and +0.0 tie and the earlier column wins), since every earlier value
// is smaller and no later equal value is strictly greater.

// v_max3_f32 as the instruction, without the canonicalising v_max_f32 that
// clang puts in front of every operand of fmaxf.  In IEEE mode a quiet NaN
// operand is ignored and a signalling one makes the result a quiet NaN;
// lane_max rescans exactly whenever the tree yields NaN.
__device__ __forceinline__ float max3_raw(float a, float b, float c)
{
    float r;
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}

template <int N>
__device__ __forceinline__ float max3_tree(const float (&v)[N])
{
    constexpr int M = (N + 2) / 3;
    float w[M];
#pragma unroll
    for (int i = 0; i < M; ++i) {
        const float a = v[3 * i];
        if (3 * i + 1 >= N) {
            w[i] = a; // a lone leftover goes up a level as it is
        } else {
            const float b = v[3 * i + 1];
            const float c = 3 * i + 2 < N ? v[3 * i + 2] : a;
            w[i] = max3_raw(a, b, c);
        }
    }
    if constexpr (M == 1) return w[0];
    else return max3_tree(w);
}

template <int B>
__device__ __forceinline__ void flatten(const float4 (&q)[B], float (&v)[4 * B])
{
#pragma unroll
    for (int j = 0; j < B; ++j) {
        v[4 * j] = q[j].x;
        v[4 * j + 1] = q[j].y;
        v[4 * j + 2] = q[j].z;
        v[4 * j + 3] = q[j].w;
    }
}

// Maximum of the lane's non-NaN values, -inf when it has none.
template <int B>
__device__ __forceinline__ float lane_max(const float (&v)[4 * B])
{
    float m = max3_tree(v);
    if (m != m) { // a signalling NaN, or no non-NaN value at all
        m = -__builtin_inff();
#pragma unroll
        for (int i = 0; i < 4 * B; ++i) m = v[i] > m ? v[i] : m;
    }
    return m;
}

// Position (float4 j * 4 + component) of the lane's first value equal to m,
// or 0xffffffff.
template <int B>
__device__ __forceinline__ uint32_t lane_first(const float (&v)[4 * B], float m)
{
    uint32_t p = 0xffffffffu;
#pragma unroll
    for (int i = 4 * B - 1; i >= 0; --i) p = v[i] == m ? static_cast<uint32_t>(i) : p;
    return p;
}

// Total order on non-NaN floats as signed integers (-0.0 just below +0.0).
__device__ __forceinline__ int32_t f32_order(float f)
{
    const int32_t b = __builtin_bit_cast(int32_t, f);
    return b ^ ((b >> 31) & 0x7fffffff);
}

__device__ __forceinline__ float f32_from_order(int32_t k)
{
    return __builtin_bit_cast(float, k ^ ((k >> 31) & 0x7fffffff));
}

__device__ __forceinline__ int32_t wave_max_dpp_i32(int32_t v)
{
    const auto step = [](int32_t a, int32_t b) { return a > b ? a : b; };
    v = step(v, static_cast<int32_t>(dpp32<kDppXor1>(static_cast<uint32_t>(v))));
    v = step(v, static_cast<int32_t>(dpp32<kDppXor2>(static_cast<uint32_t>(v))));
    v = step(v, static_cast<int32_t>(dpp32<kDppHalfMirror>(static_cast<uint32_t>(v))));
    v = step(v, static_cast<int32_t>(dpp32<kDppMirror>(static_cast<uint32_t>(v))));
    const int32_t a = static_cast<int32_t>(lane_u32(static_cast<uint32_t>(v), 0));
    const int32_t b = static_cast<int32_t>(lane_u32(static_cast<uint32_t>(v), 16));
    const int32_t c = static_cast<int32_t>(lane_u32(static_cast<uint32_t>(v), 32));
    const int32_t d = static_cast<int32_t>(lane_u32(static_cast<uint32_t>(v), 48));
    return step(step(a, b), step(c, d));
}

// The (value, column) candidate of columns [c0, c0 + 4 nvec) of the row at
// x + base, with 16-byte aligned rows; every thread of the workgroup calls
// it.  Wave 0 returns true with the candidate in `out` (uniform); the other
// waves return false and have nothing more to do.  `nan0` is true when the
// chunk's first column holds a NaN.  Thread t reads float4 t, t + 256, ...
// of each batch, like the sums.  (Measured at config 5: giving each wave a
// contiguous quarter of the chunk, or letting the wave that holds the
// maximum publish without the second barrier, were both 0.2 us slower.)
__device__ __forceinline__ bool argmax_chunk_vec(const float *x, int64_t base, uint64_t c0, uint32_t nvec,
                                                 ArgPart &out, bool &nan0)
{
    constexpr int kBatch = kRedBatch;
    constexpr uint32_t kSpan = kBatch * kBlock; // float4 per batch
    constexpr uint32_t kWaves = kBlock / kWave;
    __shared__ int32_t s_key[kWaves];
    __shared__ uint32_t s_col[kWaves];
    __shared__ uint32_t s_nan0;
    const uint32_t t = threadIdx.x;
    const uint32_t wave = t / kWave;
    const BufRsrc r = buffer_rsrc(x + base + c0, nvec * 16u);
    const auto col = [&](uint32_t v0, uint32_t p) { return (v0 + (p >> 2) * kBlock + t) * 4u + (p & 3u); };

    // Batches before the last, all in range: the lane's running candidate
    // (value, chunk-relative column), replaced only by a strictly greater one.
    float run_v = -__builtin_inff();
    uint32_t run_c = 0xffffffffu;
    uint32_t v0 = 0;
    float first = 0.0f; // thread 0: column c0
    float4 q[kBatch];
    float v[4 * kBatch];
    for (; v0 + kSpan < nvec; v0 += kSpan) {
#pragma unroll
        for (int j = 0; j < kBatch; ++j) q[j] = ld_buf_nt(r, (v0 + j * kBlock + t) * 16u);
        if (v0 == 0) first = q[0].x;
        flatten(q, v);
        const float bm = lane_max<kBatch>(v);
        if (bm > run_v) {
            run_c = col(v0, lane_first<kBatch>(v, bm));
            run_v = bm;
        }
    }
    // The last batch.  A lane's float4 index past the chunk is clamped to its
    // last float4 (nvec >= 1: every chunk holds a column): the duplicate
    // cannot change the maximum, and the column it reports, computed from
    // the unclamped index, is above that of the lane that holds the float4,
    // so the minimum over lanes never takes it.
#pragma unroll
    for (int j = 0; j < kBatch; ++j) q[j] = ld_buf_nt(r, min(v0 + j * kBlock + t, nvec - 1) * 16u);
    if (v0 == 0) first = q[0].x;
    flatten(q, v);
    const float bm = lane_max<kBatch>(v);
    const float lm = bm > run_v ? bm : run_v;

    // chunk maximum
    const int32_t wk = wave_max_dpp_i32(f32_order(lm));
    if (t % kWave == 0) s_key[wave] = wk;
    if (t == 0) s_nan0 = first != first;
    __syncthreads();
    int32_t mk = s_key[0];
#pragma unroll
    for (int w = 1; w < kWaves; ++w) mk = mk > s_key[w] ? mk : s_key[w];
    const float m = f32_from_order(mk);

    // first column holding it: an earlier batch's (lower) column, else the
    // last batch's
    uint32_t c = 0xffffffffu;
    if (lm == m) {
        if (run_v == m) {
            c = run_c;
        } else {
            const uint32_t p = lane_first<kBatch>(v, m);
            if (p != 0xffffffffu) c = col(v0, p);
        }
    }
    c = wave_min_dpp(c);
    if (t % kWave == 0) s_col[wave] = c;
    __syncthreads();
    nan0 = s_nan0 != 0;
    if (wave != 0) return false;
    c = min(min(s_col[0], s_col[1]), min(s_col[2], s_col[3]));
    out = ArgPart{m, c == 0xffffffffu ? c : static_cast<uint32_t>(c0) + c};
    return true;
}

// Writes the row result from its combined (sum | (value, index)) word.
template <RedOp OP>
__device__ __forceinline__ void write_result(const RedGeo &g, void *dst, uint32_t row, uint64_t packed)
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
        const uint64_t idx = p.i == 0xffffffffu ? 0 : p.i; // no candidate: every value was NaN or -inf
        const float fidx = static_cast<float>(idx);         // the reference stores the index as f32
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

// Merges n <= 64 partial words across the wave: lane l contributes `own`
// when l == self, else the word at slots[l] (read at the coherence point).
// Returns the merged word, uniform.
template <RedOp OP>
__device__ __forceinline__ uint64_t merge_slots(const uint64_t *slots, uint32_t n, uint32_t self, uint64_t own)
{
    constexpr bool kArg = Acc<OP>::kArg;
    const uint32_t lane = threadIdx.x % kWave;
    uint64_t q = own;
    if (lane < n && lane != self) q = __hip_atomic_load(slots + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if constexpr (kArg) {
        const ArgPart p = __builtin_bit_cast(ArgPart, q);
        float v = lane < n ? p.v : -__builtin_inff();
        uint32_t i = lane < n ? p.i : 0xffffffffu;
        wave_argmax_dpp(v, i);
        return __builtin_bit_cast(uint64_t, ArgPart{v, i});
    } else {
        const double t = wave_sum_dpp(lane < n ? __builtin_bit_cast(double, q) : 0.0);
        return __builtin_bit_cast(uint64_t, t);
    }
}

// Publishes `packed` into `slot` and counts the arrival; true for the last of
// `n` arrivals (uniform).  Lane 0 of the calling wave does the memory
// operations.
__device__ __forceinline__ bool arrive(uint64_t *slot, uint32_t *counter, uint32_t n, uint64_t packed)
{
    const bool lead = threadIdx.x % kWave == 0;
    uint32_t prev = 0;
    if (lead) {
        __hip_atomic_store(slot, packed, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); // the partial is at the coherence point
        prev = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    prev = __builtin_amdgcn_readfirstlane(prev);
    if (prev != n - 1) return false;
    if (lead) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return true;
}

// Workgroup (row, chunk) reduces its column range; with one chunk per row it
// writes the result, otherwise it hands its partial over (see above).
template <RedOp OP>
__global__ __launch_bounds__(kBlock) void k_reduce(RedGeo g, const float *x, void *dst, char *parts, char *counts)
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

    double sum = 0.0;
    float bv = -__builtin_inff();
    uint32_t bi = 0xffffffffu; // "no candidate": loses every tie on index
    float first = 0.0f;        // thread 0 of chunk 0: the row's column 0
    bool vec_arg = false;
    bool nan0 = false; // the chunk's first column is NaN (vector argmax)
    if constexpr (kArg) {
        if (g.mode == kModeVec) {
            ArgPart p;
            if (!argmax_chunk_vec(x, base, c0, static_cast<uint32_t>((c1 - c0) / 4), p, nan0)) return;
            bv = p.v;
            bi = p.i;
            vec_arg = true;
        }
    }
    if (!vec_arg) {
        accumulate<OP>(g, x, base, c0, c1, sum, bv, bi, first);
        if constexpr (kArg) {
            wave_argmax_dpp(bv, bi);
            if (lane == 0) {
                s_v[wave] = bv;
                s_i[wave] = bi;
            }
        } else {
            sum = wave_sum_dpp(sum);
            if (lane == 0) s_sum[wave] = sum;
        }
        __syncthreads();
    }
    // wave 0 alone from here on: the partial is uniform across it
    if (!vec_arg && wave != 0) return; // (argmax_chunk_vec returned the other waves)
    uint64_t packed;
    if constexpr (kArg) {
        float v = bv;
        uint32_t i = bi;
        if (!vec_arg) {
            v = s_v[0];
            i = s_i[0];
            for (int w = 1; w < kBlock / kWave; ++w) argmax_merge(v, i, s_v[w], s_i[w]);
            first = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, first))); // thread 0
            nan0 = first != first;
        }
        // A NaN in column 0 decides the row: chunk 0's partial becomes
        // (+inf, 0), which every other candidate loses to (equal value and a
        // higher index, or a lower value).
        if (chunk == 0 && nan0) {
            v = __builtin_inff();
            i = 0;
        }
        packed = __builtin_bit_cast(uint64_t, ArgPart{v, i});
    } else {
        packed = __builtin_bit_cast(uint64_t, (s_sum[0] + s_sum[1]) + (s_sum[2] + s_sum[3]));
    }
    if (g.chunks == 1) {
        if (lane == 0) write_result<OP>(g, dst, row, packed);
        return;
    }
    uint64_t *part1 = reinterpret_cast<uint64_t *>(parts + g.off_part1);
    uint32_t *cnt1 = reinterpret_cast<uint32_t *>(counts + g.off_cnt1);
    const uint32_t grp = chunk / g.group_size;
    const uint32_t gfirst = grp * g.group_size;
    const uint32_t gn = g.chunks - gfirst < g.group_size ? g.chunks - gfirst : g.group_size;
    uint64_t *gslots = part1 + static_cast<uint64_t>(row) * g.chunks + gfirst;
    if (!arrive(gslots + (chunk - gfirst), cnt1 + (static_cast<uint64_t>(row) * g.groups + grp) * g.cstride, gn, packed))
        return;
    packed = merge_slots<OP>(gslots, gn, chunk - gfirst, packed);
    if (g.groups > 1) {
        uint64_t *rslots = reinterpret_cast<uint64_t *>(parts + g.off_part2) + static_cast<uint64_t>(row) * g.groups;
        uint32_t *cnt2 = reinterpret_cast<uint32_t *>(counts + g.off_cnt2) + static_cast<uint64_t>(row) * kLineWords;
        if (!arrive(rslots + grp, cnt2, g.groups, packed)) return;
        packed = merge_slots<OP>(rslots, g.groups, grp, packed);
    }
    if (lane == 0) write_result<OP>(g, dst, row, packed);
}

constexpr uint32_t kTargetBlocks = 2048; // 8 workgroups per CU on 256 CUs
constexpr uint64_t kMinChunkCols = 4 * kBlock; // one float4 per thread at least

uint64_t align256(uint64_t b) { return (b + 255) & ~uint64_t{255}; }

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
    const uint64_t min_for_cap = (g.ncols + kMaxChunks - 1) / kMaxChunks;
    if (chunk < min_for_cap) chunk = min_for_cap;
    chunk = (chunk + 3) & ~uint64_t{3};
    uint64_t chunks = (g.ncols + chunk - 1) / chunk;
    if (chunks == 0) chunks = 1;
    if (chunks > kMaxChunks || static_cast<uint64_t>(g.rows) * chunks > 0x7fffffffull) return false;
    g.chunks = static_cast<uint32_t>(chunks);
    g.chunk_cols = chunk;
    if (g.mode == kModeVec && chunk * 4 > 0x7fffffffull) g.mode = kModeScalar; // buffer offsets are 32-bit
    g.groups = (g.chunks + kMaxGroup - 1) / kMaxGroup;
    g.group_size = (g.chunks + g.groups - 1) / g.groups;
    // first-level counters: about 32 increments per 128-byte line
    uint32_t cs = 1;
    while (cs < g.group_size && cs < kLineWords) cs <<= 1;
    g.cstride = cs;
    if (g.chunks > 1) {
        const uint64_t rows = g.rows;
        g.off_part1 = 0;
        g.off_part2 = align256(rows * g.chunks * sizeof(uint64_t));
        g.off_cnt1 = 0;
        g.off_cnt2 = align256(rows * g.groups * g.cstride * sizeof(uint32_t));
    }
    return true;
}

RedScratch scratch_bytes(const RedGeo &g)
{
    RedScratch r{0, 0};
    if (g.chunks <= 1) return r;
    r.partials = g.off_part2 + (g.groups > 1 ? align256(uint64_t{g.rows} * g.groups * sizeof(uint64_t)) : 0);
    r.counters = g.off_cnt2 + (g.groups > 1 ? align256(uint64_t{g.rows} * kLineWords * sizeof(uint32_t)) : 0);
    return r;
}

// ---- the allocation-free entry point's scratch -------------------------------
//
// One array per device, in the code object's zero-initialised data: the
// first 64 KiB hold arrival counters, the next 64 KiB partials.  Every plan
// above needs at most 24 KiB of counters and 32 KiB of partials (rows below
// 2048 split into at most 2048 + rows chunks in total; more rows need no
// scratch).  In host code `scratch` names a host-side stand-in: the device
// address comes from hipGetSymbolAddress, once per device.
constexpr uint64_t kStaticCounterBytes = 64u << 10;
constexpr uint64_t kStaticPartialBytes = 64u << 10;
static __device__ __align__(256) unsigned char scratch[kStaticCounterBytes + kStaticPartialBytes];

__global__ __launch_bounds__(kBlock) void k_clear_words(uint32_t *p, uint32_t n)
{
    const uint32_t i = blockIdx.x * kBlock + threadIdx.x;
    if (i < n) p[i] = 0u;
}

constexpr int kMaxDevices = 64;
std::mutex g_static_lock;
char *g_static_base[kMaxDevices]; // device address of `scratch`, per device (null until set up)

} // namespace

hipError_t reduce_static_scratch(RedArgs &a, hipStream_t stream)
{
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    char *base = nullptr;
    {
        std::lock_guard<std::mutex> g(g_static_lock);
        if (!g_static_base[dev]) {
            // set-up on this device's first call, with the device current
            void *ptr = nullptr;
            e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
            if (e != hipSuccess) return e;
            if (!ptr) return hipErrorInvalidSymbol;
            // The counters must start at zero (launches leave them zero).  A
            // fill kernel, not a memset node, so a captured first call
            // replays correctly.
            constexpr uint32_t words = kStaticCounterBytes / 4;
            k_clear_words<<<(words + kBlock - 1) / kBlock, kBlock, 0, stream>>>(static_cast<uint32_t *>(ptr), words);
            e = hipGetLastError();
            if (e != hipSuccess) return e;
            g_static_base[dev] = static_cast<char *>(ptr);
        }
        base = g_static_base[dev];
    }
    const RedScratch need = reduce_scratch_bytes(a);
    if (need.counters > kStaticCounterBytes || need.partials > kStaticPartialBytes) return hipErrorOutOfMemory;
    a.counters = base;
    a.partials = base + kStaticCounterBytes;
    a.scratch = RedScratch{kStaticPartialBytes, kStaticCounterBytes};
    return hipSuccess;
}

RedScratch reduce_scratch_bytes(const RedArgs &a)
{
    RedGeo g;
    if (!plan(a, g)) return RedScratch{0, 0};
    return scratch_bytes(g);
}

hipError_t launch_reduce(const RedArgs &a, hipStream_t s)
{
    RedGeo g;
    if (!plan(a, g)) return hipErrorInvalidValue;
    const float *x = static_cast<const float *>(a.x.data);
    const RedScratch need = scratch_bytes(g);
    char *parts = static_cast<char *>(a.partials);
    char *counts = static_cast<char *>(a.counters);
    if (need.partials > a.scratch.partials || need.counters > a.scratch.counters) return hipErrorInvalidValue;
    if (g.chunks > 1 && (!parts || !counts)) return hipErrorInvalidValue;
    const dim3 grid(g.rows * g.chunks);
    auto run = [&](auto op_tag) {
        constexpr RedOp OP = decltype(op_tag)::value;
        k_reduce<OP><<<grid, kBlock, 0, s>>>(g, x, a.dst, parts, counts);
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
