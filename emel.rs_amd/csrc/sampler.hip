// sampler.hip -- gfx950 kernels for emel-logits' native temperature/top-k
// sampler (Sampler::sample_temperature_top_k, crates/emel-logits/src/
// sampler/sm.rs:380-392, effects :759-847) and its candidate validator
// (Validator::process_event(Build), crates/emel-logits/src/validator/sm.rs).
//
// A request is one row of `card` logits; a launch serves `rows` independent
// requests.  Per row, as the reference computes it:
//   v = x * (1/T)                          (f32, in place)
//   m = max over v, NaN ignored            (f32::max fold from -inf)
//   e = expf(v - m)                        (glibc expf, in place)
//   S = e_0 + e_1 + ... sequentially, f32  (the rounding of every step kept)
//   p = e / S                              (in place: the caller's logits end as p)
//   rank by p descending (f32::total_cmp), keep the first top_k
//   race_j = p_j / -logf(u_j), u_j from the Park-Miller sequence; the first
//   maximal race wins.
//
// Kernels, in launch order (the same sequence for every request; rows that
// finish a stage early skip the later ones):
//   k_smp_max     (row, chunk) workgroups: chunk maxima of v; for chunks of
//                 at most 8192 columns also each 512-element sub-chunk's
//                 maximum and approximate sum of exp(v - that maximum).
//   k_smp_expseg  (row, chunk), chunks of at most 8192 columns: e written
//                 in place, and each sub-chunk's exact contribution in units
//                 of the binade (or each of the two binades) predicted from
//                 the approximate sums.  One head workgroup per row, first in
//                 the grid, adds the row's first sub-chunk one by one (the
//                 walk's starting state) and finds e_thr, the top_k-th
//                 largest e among the row's sub-chunk maxima (fast candidate
//                 list, top_k <= 8192).
//   k_smp_exp and k_smp_seg, wider chunks, the same in two passes: e and
//                 the chunk's f64 sum, then the predictions from exact f64
//                 prefixes.
//   k_smp_sum     one wave per row: the exact sequential sum (seqsum.hpp),
//                 taking a sub-chunk's predicted contribution when the exact
//                 state confirms it, walking the other sub-chunks from
//                 registers or from LDS.  A second wave stages the
//                 sub-chunks that probably cross a binade into LDS ahead of
//                 the walk, with their lane unit scans at both binades, so
//                 that a crossing takes one step.  The walk ends with the
//                 fast threshold p_thr = e_thr / S.
//   k_smp_div     (row, chunk): p written in place, plus the histogram of the
//                 top 11 bits of p's total-order key, and the list of every
//                 p >= p_thr.  A row whose list fits 8192 entries is ranked
//                 from it.
//   k_smp_tail    (when the fast list applies: top_k at most the row's
//                 sub-chunk count) one 1024-thread workgroup per row, in one
//                 launch:
//                 - rows the fast list did not resolve: radix selection of
//                   the top_k-th key, 11, 11, 10 key bits (the first digit
//                   from k_smp_div's histogram, later ones from scans of the
//                   row), stopping as soon as every key at or above the
//                   current prefix fits the kCap candidates one workgroup
//                   sorts; at 32 bits the threshold key T is exact.  Then the
//                   candidate list (key, index) in column order: every key >=
//                   prefix, or every key > T plus the lowest-index ties at T
//                   up to top_k;
//                 - every row: sort of the candidates in LDS (key descending
//                   then index ascending: register runs merged by merge
//                   path), the ranked outputs, then the race selection.
// Otherwise, for top_k <= kCap (the bucket path), the exponential pass also
// counts e's first digits, k_smp_sum turns the digit holding the top_k-th
// largest e into a bracket [blo, bhi] of p's keys, and k_smp_div lists the
// keys above bhi (A) into the candidate list and those in the bracket (B)
// into the bucket list; then
//   k_smp_rank    a few 1024-thread workgroups per row: groups of whole first
//                 digits of A, each sorted in LDS at its known offset, and B,
//                 cut by digits of its own histograms and sorted, after them;
//                 each races its own slots and the row's last workgroup
//                 writes the selection.  A row whose lists do not select
//                 (|A| < top_k <= |A| + |B| fails, or B overflows) takes the
//                 radix selection from scans of the row in one workgroup.
// For top_k > kCap the selection runs as k_smp_resolve (one workgroup per
// row, the ties at T counted per chunk) and k_smp_collect ((row, chunk)
// workgroups), and the list is sorted as kCap tiles (k_smp_tile_sort),
// merged pairwise (k_smp_merge), and finished by k_smp_finish.
//
// Ties of p: the reference sorts with sort_unstable_by, which leaves the
// order of equal probabilities unspecified; here they rank by ascending
// index, the order the CPU oracle uses.
#include <type_traits>

#include "common.hpp"
#include "launch.hpp"
#include "libm_replica.hpp"
#include "seqsum.hpp"

namespace emel {
namespace {

constexpr uint32_t kCap = 8192;          // candidates sorted in LDS by one workgroup
constexpr uint32_t kRankThreads = 1024;
constexpr uint32_t kBins = 2048;         // 11-bit radix digits
constexpr uint32_t kNone = 0xffffffffu;
constexpr uint32_t kModulus = 2147483647u;   // sampler/sm.rs:22
constexpr uint64_t kMultiplier = 16807u;     // sampler/sm.rs:23
constexpr int32_t kInvalidRequest = 13;      // EMEL_ERR_INVALID_REQUEST

// Per-row selection state (workspace).
struct RowSel {
    float total;      // the sequential sum S
    uint32_t mode;    // 0 open, 1 collect keys >= prefix, 2 collect keys > T + ties,
                      // 3 the list k_smp_div wrote (keys >= fast_key)
    uint32_t prefix;  // resolved top `depth` bits of the key (T when depth == 32)
    uint32_t depth;
    uint32_t need;    // elements still to take from the prefix region
    uint32_t above;   // elements whose key prefix is greater (all taken)
    uint32_t count;   // candidates collected
    uint32_t written; // collect cursor
    uint32_t fast_on;    // k_smp_div lists the keys >= fast_key
    uint32_t fast_key;   // key of p_thr (k_smp_sum)
    uint32_t fast_count; // keys >= fast_key found; > kCap: the radix path decides
    uint32_t ethr_on;    // e_thr found (k_smp_expseg's head workgroup)
    uint32_t ethr_key;   // key of e_thr
    uint32_t bon;        // the bucket path's bracket [blo, bhi] is set (k_smp_sum)
    uint32_t blo, bhi;   // keys: A above bhi, B in [blo, bhi] (k_smp_div lists both)
    uint32_t gdone;      // k_smp_rank: workgroups of the row finished
    uint64_t gfill;      // k_smp_div: words listed, A (low half) and B (high half)
};
constexpr uint32_t kMaxGroups = 8; // k_smp_rank workgroups per row
// One k_smp_rank workgroup's result: its greatest race_word and the token of
// that slot.
struct GroupBest {
    uint64_t word;
    uint64_t idx;
};
constexpr uint32_t kBucketCap = 16384; // words a row's bucket list (B) holds

struct SmpGeo {
    uint32_t rows;
    uint32_t chunks;
    uint64_t card;
    uint64_t chunk_cols; // multiple of 4
    int64_t ld;          // logits row stride, elements
    uint32_t vec;        // 16-byte aligned rows: float4 paths
    uint32_t top_k;
    float scale;
    uint32_t cand_ld;    // candidate slots per row
};

// A sub-chunk's contribution to the row's exact sum, computed ahead of the
// walk at a predicted binade (k_smp_seg): units (+1 when `tie` and the
// running units plus `par` are odd) of 2^u, when ok.
constexpr uint32_t kSub = 512;   // elements per sub-chunk (one walk round)
constexpr uint32_t kPer = kSub / kWave; // elements per lane of a sub-chunk
constexpr uint32_t kMaxSub = 64; // sub-chunks a chunk predicts; later ones are walked
// When the sub-chunk's bounds span two binades, it is counted at both: u for
// the lower one and u + 1 for the upper one (units1 and flag bits 4-6); the
// walk takes the count of whichever binade its exact state is in.
struct SegInfo {
    uint32_t units;  // at 2^u; large counts saturate: the walk rejects anything >= 2^24
    int32_t u;
    uint32_t flags;  // bit 0 ok at 2^u, bit 1 one tie, bit 2 its parity, bit 3 empty slot,
                     // bits 4-6 the same at 2^(u+1), bit 7 likely walked (stage it)
    uint32_t units1; // at 2^(u+1), when bit 4 is set
};
constexpr uint32_t kSegEmpty = 8u;
constexpr uint32_t kSegUpper = 4u;     // shift of the 2^(u+1) bits
constexpr uint32_t kSegWalk = 0x80u;
// A row's first slot holds the running sum after it instead (the walk starts
// there): units = m and u, or with kSegSpecial a NaN or +inf sum whose bits
// are in units1.  It is also empty: the walk adds nothing for it.
constexpr uint32_t kSegState = 0x100u;
constexpr uint32_t kSegSpecial = 0x200u;
constexpr uint32_t kSegHasU = 0x400u; // u names the lower binade of a usable plan
// Chunks of at most kFuseSubs sub-chunks (kFuseCols columns) take the fused
// path: k_smp_max<true> also leaves an approximate sum of exp(v - m_k) per
// sub-chunk (m_k its maximum), and k_smp_expseg writes e and predicts each
// sub-chunk from those sums in one pass.  Wider chunks run k_smp_max<false>,
// k_smp_exp and k_smp_seg, which predict from exact f64 sums of e.
constexpr uint32_t kFuseSubs = 16;
constexpr uint32_t kFusePerWave = kFuseSubs / (kBlock / kWave);
constexpr uint64_t kFuseCols = uint64_t{kFuseSubs} * kSub;
static_assert(kFusePerWave * (kBlock / kWave) == kFuseSubs, "sub-chunks split evenly over the waves");
struct SubSum {
    float m; // maximum of v over the sub-chunk (-inf when it has none)
    float s; // ~ sum of exp(v - m) over the sub-chunk; 0 when m is -inf
};

struct SmpWs {
    float *part;   // rows * chunks chunk maxima
    double *psum;  // rows * chunks f64 sums of e per chunk (binade prediction);
                   // fused path: ~ sums of exp(v - chunk maximum)
    SubSum *sub;   // rows * chunks * subs per chunk (fused path)
    SegInfo *seg;  // rows * chunks * subs per chunk
    RowSel *sel;   // rows
    uint32_t *hist; // rows * kBins
    uint32_t *ties; // rows * chunks
    uint64_t *cand; // rows * cand_ld
    uint64_t *cand2; // rows * cand_ld (merge ping-pong, top_k > kCap)
    uint32_t *ehist;  // rows * kBins: first-digit histogram of e (the bucket path)
    uint64_t *bucket; // rows * kBucketCap (B lists; the bucket path only)
    GroupBest *gbest; // rows * kMaxGroups (the bucket path only)
};

// f32::total_cmp as an unsigned key (larger key = later in total order).
__device__ __forceinline__ uint32_t total_key(float f)
{
    const uint32_t b = f32_to_bits(f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float from_key(uint32_t k)
{
    return bits_to_f32((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}
// Sort word: key descending, then index ascending, as one descending u64.
__device__ __forceinline__ uint64_t cand_word(uint32_t key, uint32_t idx)
{
    return (static_cast<uint64_t>(key) << 32) | static_cast<uint64_t>(~idx);
}

// a * b mod (2^31 - 1) for a < 2^32, b < 2^31: since 2^31 == 1 (mod 2^31 - 1),
// folding the high bits onto the low ones twice leaves r < 2 (2^31 - 1), and
// one conditional subtraction gives the remainder.
__host__ __device__ __forceinline__ constexpr uint32_t mulmod(uint32_t a, uint32_t b)
{
    const uint64_t x = static_cast<uint64_t>(a) * b;
    uint64_t r = (x & kModulus) + (x >> 31);
    r = (r & kModulus) + (r >> 31);
    return static_cast<uint32_t>(r >= kModulus ? r - kModulus : r);
}

// 16807^(t+1) mod (2^31 - 1) for t < kRankThreads: the Park-Miller draw
// multiplier of slot t (state_j = s0 16807^(j+1)); slot t + m kRankThreads
// multiplies by kPmStride^m more.
struct PmPowers {
    uint32_t v[kRankThreads];
};
constexpr PmPowers make_pm_powers()
{
    PmPowers p{};
    uint32_t x = 1;
    for (uint32_t t = 0; t < kRankThreads; ++t) {
        x = mulmod(x, static_cast<uint32_t>(kMultiplier));
        p.v[t] = x;
    }
    return p;
}
static constexpr PmPowers kPmPowers = make_pm_powers();
constexpr uint32_t kPmStride = kPmPowers.v[kRankThreads - 1]; // 16807^kRankThreads
static_assert(kPmPowers.v[0] == 16807u && kPmPowers.v[1] == 282475249u && kPmPowers.v[2] == 1622650073u,
              "Park-Miller powers: 16807, 16807^2, 16807^3 mod 2^31 - 1");

// 16807^n mod (2^31 - 1) by squaring: the draw state of slot j - 1 from s0
// is s0 16807^j, so a workgroup ranking the slots from j0 starts from
// s0 pm_power(j0).
__host__ __device__ constexpr uint32_t pm_power(uint32_t n)
{
    uint32_t r = 1, b = static_cast<uint32_t>(kMultiplier);
    for (; n; n >>= 1) {
        if (n & 1u) r = mulmod(r, b);
        b = mulmod(b, b);
    }
    return r;
}
static_assert(pm_power(1) == kPmPowers.v[0] && pm_power(3) == kPmPowers.v[2] && pm_power(kRankThreads) == kPmStride,
              "pm_power agrees with the power table");

// Visits the columns [c0, c1) of one row: float4 steps when the row is
// 16-byte aligned, then a scalar tail.  A step issues U loads per thread
// before any is used; loads past the range re-read its last float4 (in
// bounds, from cache) and are not visited, so a chunk of up to U float4 per
// thread costs one memory round trip.  The order of the visits is
// unspecified: callers only reduce order-independently or write
// elementwise.  f(float &v, uint64_t col) may modify v; WRITE stores it back.
template <bool WRITE, int U = 8, class F>
__device__ __forceinline__ void visit(const SmpGeo &g, float *row, uint64_t c0, uint64_t c1, F f)
{
    uint64_t c = c0;
    if (g.vec) {
        float4 *r4 = reinterpret_cast<float4 *>(row);
        const uint64_t v1 = c1 / 4;
        const uint64_t bs = blockDim.x;
        auto apply = [&](float4 &q, uint64_t vi) {
            f(q.x, 4 * vi);
            f(q.y, 4 * vi + 1);
            f(q.z, 4 * vi + 2);
            f(q.w, 4 * vi + 3);
        };
        for (uint64_t v = c0 / 4 + threadIdx.x; v < v1; v += U * bs) {
            float4 q[U];
#pragma unroll
            for (int j = 0; j < U; ++j) {
                const uint64_t i = v + j * bs;
                q[j] = r4[i < v1 ? i : v1 - 1];
            }
#pragma unroll
            for (int j = 0; j < U; ++j) {
                const uint64_t i = v + j * bs;
                if (i < v1) {
                    apply(q[j], i);
                    if constexpr (WRITE) r4[i] = q[j];
                }
            }
        }
        c = v1 * 4 > c0 ? v1 * 4 : c0;
    }
    for (uint64_t k = c + threadIdx.x; k < c1; k += blockDim.x) {
        float v = row[k];
        f(v, k);
        if constexpr (WRITE) row[k] = v;
    }
}

__device__ __forceinline__ void chunk_range(const SmpGeo &g, uint32_t chunk, uint64_t &c0, uint64_t &c1)
{
    c0 = static_cast<uint64_t>(chunk) * g.chunk_cols;
    c1 = c0 + g.chunk_cols < g.card ? c0 + g.chunk_cols : g.card;
}

__device__ __forceinline__ uint32_t subs_per_chunk(const SmpGeo &g)
{
    return static_cast<uint32_t>((g.chunk_cols + kSub - 1) / kSub);
}

// Block reduction of a float maximum (NaN-free operands), 256 threads.
__device__ __forceinline__ float block_max256(float v)
{
    __shared__ float s[kBlock / kWave];
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) {
        const float o = __shfl_xor(v, off, kWave);
        v = o > v ? o : v;
    }
    if (threadIdx.x % kWave == 0) s[threadIdx.x / kWave] = v;
    __syncthreads();
    float r = s[0];
    for (int w = 1; w < kBlock / kWave; ++w) r = s[w] > r ? s[w] : r;
    return r;
}

// ---- stage 1: chunk maxima of v = x * scale ---------------------------------

// The fused path's lane layout of a sub-chunk starting at column a0: lane l
// holds columns a0 + 4 l .. a0 + 4 l + 3 and a0 + kSub / 2 + 4 l .. + 3
// (elements 0-3 and 4-7 of its kPer), so each 128-bit load or store
// instruction of a wave covers 1 KiB contiguously.
constexpr uint32_t kSplit = 2; // groups of a lane's elements
static_assert(kPer == 4 * kSplit, "one float4 per group");
__device__ __forceinline__ uint64_t split_col(uint64_t a0, uint32_t lane, uint32_t q)
{
    return a0 + (q / 4) * (kSub / kSplit) + 4 * lane + (q % 4);
}

// Lane `lane`'s elements of the sub-chunk at a0 (zeros past c1, or everywhere
// when !valid).
// WHOLE: test a whole sub-chunk once (wave-uniform) before the per-float4
// tests.
template <bool WHOLE = false>
__device__ __forceinline__ void load_split(const SmpGeo &g, const float *x, uint64_t a0, uint64_t c1, uint32_t lane,
                                           bool valid, float (&v)[kPer])
{
    if (WHOLE && valid && g.vec && a0 + kSub <= c1) { // uniform: a whole sub-chunk of an aligned row
#pragma unroll
        for (uint32_t h = 0; h < kSplit; ++h) {
            // plain loads: later passes re-read these lines from cache
            const float4 t = *reinterpret_cast<const float4 *>(x + split_col(a0, lane, 4 * h));
            v[4 * h] = t.x;
            v[4 * h + 1] = t.y;
            v[4 * h + 2] = t.z;
            v[4 * h + 3] = t.w;
        }
        return;
    }
#pragma unroll
    for (uint32_t h = 0; h < kSplit; ++h) {
        const uint64_t col = split_col(a0, lane, 4 * h);
        if (valid && g.vec && col + 4 <= c1) {
            // plain loads: later passes re-read these lines from cache
            const float4 t = *reinterpret_cast<const float4 *>(x + col);
            v[4 * h] = t.x;
            v[4 * h + 1] = t.y;
            v[4 * h + 2] = t.z;
            v[4 * h + 3] = t.w;
        } else {
#pragma unroll
            for (uint32_t q = 0; q < 4; ++q) v[4 * h + q] = valid && col + q < c1 ? x[col + q] : 0.0f;
        }
    }
}

// exp(x) for the binade predictions only, never for a result: one hardware
// 2^x of x log2(e).  The f32 product's rounding and v_exp_f32's own error
// leave it within about (1 + |x|) 2^-23 of exp(x).
__device__ __forceinline__ float approx_exp(float x)
{
    return __builtin_amdgcn_exp2f(x * 1.44269504088896341f);
}

// FUSED (chunks of at most kFuseSubs sub-chunks) reads the chunk as
// k_smp_expseg does, lane l of a wave holding elements kPer l .. kPer l +
// kPer - 1 of a sub-chunk, and also leaves each sub-chunk's maximum and
constexpr uint32_t kFastPer = 8;         // sub-chunk maxima per lane for the fast threshold

// Whether a launch's rows can take the fast list: the fused path, top_k
// within kCap and within the row's sub-chunk count, at most kFastPer
// sub-chunks per lane.
__host__ __device__ inline bool fast_list_possible(const SmpGeo &g)
{
    const uint64_t spc = (g.chunk_cols + kSub - 1) / kSub, nslots = uint64_t{g.chunks} * spc;
    const uint64_t last = g.card - uint64_t{g.chunks - 1} * g.chunk_cols;
    const uint64_t nsub = uint64_t{g.chunks - 1} * spc + (last + kSub - 1) / kSub; // sub-chunks with elements
    return g.chunk_cols <= kFuseCols && g.top_k <= kCap && nslots <= kWave * kFastPer && nsub >= g.top_k;
}

// The bucket path: top_k <= kCap without the fast list.
__host__ __device__ inline bool bucket_path(const SmpGeo &g) { return g.top_k <= kCap && !fast_list_possible(g); }

// Adds the LDS histogram of a workgroup to the row's global histogram, bin b
// to dst[(b + rot) mod nbins] (nbins a power of two).
__device__ __forceinline__ void flush_hist(uint32_t *s_hist, uint32_t nbins, uint32_t *dst, uint32_t rot = 0)
{
    __syncthreads();
    for (uint32_t b = threadIdx.x; b < nbins; b += blockDim.x) {
        const uint32_t c = s_hist[b];
        if (c) atomicAdd(dst + ((b + rot) & (nbins - 1)), c);
    }
}

// approximate sum of exp(v - that maximum) in sub, and in psum the chunk's
// approximate sum of exp(v - chunk maximum): k_smp_expseg's binade
// predictions start from them.
template <bool FUSED>
__global__ __launch_bounds__(kBlock) void k_smp_max(SmpGeo g, float *logits, SmpWs w)
{
    const uint32_t row = blockIdx.x / g.chunks, chunk = blockIdx.x % g.chunks;
    float *x = logits + static_cast<int64_t>(row) * g.ld;
    if (chunk == 0) {
        // fresh per-row state for this call
        for (uint32_t b = threadIdx.x; b < kBins; b += blockDim.x) {
            w.hist[static_cast<uint64_t>(row) * kBins + b] = 0;
            w.ehist[static_cast<uint64_t>(row) * kBins + b] = 0;
        }
        if (threadIdx.x == 0) {
            RowSel s{};
            s.need = g.top_k;
            w.sel[row] = s;
        }
    }
    uint64_t c0, c1;
    chunk_range(g, chunk, c0, c1);
    const float scale = g.scale;
    if constexpr (!FUSED) {
        float m = -__builtin_inff();
        visit<false>(g, x, c0, c1, [&](float &v, uint64_t) {
            const float s = v * scale;
            m = s > m ? s : m; // f32::max: a NaN operand is never taken
        });
        m = block_max256(m);
        if (threadIdx.x == 0) w.part[blockIdx.x] = m;
    } else {
        const uint32_t lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
        const uint32_t spc = subs_per_chunk(g);
        const uint32_t nsub = static_cast<uint32_t>((c1 - c0 + kSub - 1) / kSub); // <= kFuseSubs
        float v[kFusePerWave][kPer];
#pragma unroll
        for (uint32_t j = 0; j < kFusePerWave; ++j) {
            const uint32_t k = wave + (kBlock / kWave) * j;
            load_split<true>(g, x, c0 + static_cast<uint64_t>(k) * kSub, c1, lane, k < nsub, v[j]);
        }
        // per lane: its maximum lm over its elements of each sub-chunk and
        // la = sum of exp(v - lm), so the exponentials need no wave
        // reduction first; then per sub-chunk the wave maximum m_k and
        // sum of la exp(lm - m_k), the four sub-chunks' reductions
        // independent of one another
        float lm[kFusePerWave], la[kFusePerWave];
#pragma unroll
        for (uint32_t j = 0; j < kFusePerWave; ++j) {
            const uint32_t k = wave + (kBlock / kWave) * j;
            const uint64_t a0 = c0 + static_cast<uint64_t>(k) * kSub;
            lm[j] = -__builtin_inff();
            la[j] = 0.0f;
            // only a row's last sub-chunk can end early: the others skip the
            // per-element column checks
            auto stats = [&](auto full_tag) {
                constexpr bool kFull = decltype(full_tag)::value;
                float m = -__builtin_inff(), a = 0.0f;
#pragma unroll
                for (uint32_t q = 0; q < kPer; ++q) {
                    const float t = v[j][q] * scale;
                    v[j][q] = t;
                    const bool in = kFull || split_col(a0, lane, q) < c1;
                    m = in && t > m ? t : m; // f32::max: a NaN operand is never taken
                }
                if (m > -__builtin_inff()) {
#pragma unroll
                    for (uint32_t q = 0; q < kPer; ++q) {
                        const bool in = kFull || split_col(a0, lane, q) < c1;
                        a += in ? approx_exp(v[j][q] - m) : 0.0f; // a NaN or +inf makes it NaN
                    }
                }
                lm[j] = m;
                la[j] = a;
            };
            if (k < nsub) { // wave-uniform
                if (a0 + kSub <= c1) stats(std::true_type{});
                else stats(std::false_type{});
            }
        }
        float wm = -__builtin_inff(); // this wave's maximum
        float mk[kFusePerWave], sk[kFusePerWave];
#pragma unroll
        for (uint32_t j = 0; j < kFusePerWave; ++j)
            mk[j] = wave + (kBlock / kWave) * j < nsub ? wave_max_dpp(lm[j]) : -__builtin_inff(); // uniform
#pragma unroll
        for (uint32_t j = 0; j < kFusePerWave; ++j) {
            sk[j] = 0.0f;
            if (wave + (kBlock / kWave) * j < nsub) { // uniform
                // every prediction from a NaN sum fails
                const float t = la[j] != 0.0f ? la[j] * approx_exp(lm[j] - mk[j]) : 0.0f;
                sk[j] = wave_sum_dpp(t); // f32 tree: within 6 2^-24, far inside kApproxRel
            }
        }
#pragma unroll
        for (uint32_t j = 0; j < kFusePerWave; ++j) {
            const uint32_t k = wave + (kBlock / kWave) * j;
            if (k < nsub) {
                if (lane == 0) w.sub[static_cast<uint64_t>(blockIdx.x) * spc + k] = SubSum{mk[j], sk[j]};
                wm = mk[j] > wm ? mk[j] : wm;
            } else {
                mk[j] = -__builtin_inff();
                sk[j] = 0.0f;
            }
        }
        const float mc = block_max256(wm);
        double t = 0.0;
#pragma unroll
        for (uint32_t j = 0; j < kFusePerWave; ++j)
            if (sk[j] != 0.0f) t += static_cast<double>(sk[j] * approx_exp(mk[j] - mc));
        __shared__ double s_acc[kBlock / kWave];
        if (lane == 0) s_acc[wave] = t;
        __syncthreads();
        if (threadIdx.x == 0) {
            w.part[blockIdx.x] = mc;
            w.psum[blockIdx.x] = (s_acc[0] + s_acc[1]) + (s_acc[2] + s_acc[3]);
        }
    }
}

__device__ __forceinline__ float row_max(const SmpGeo &g, const SmpWs &w, uint32_t row)
{
    float m = -__builtin_inff();
    for (uint32_t c = threadIdx.x; c < g.chunks; c += blockDim.x) {
        const float p = w.part[static_cast<uint64_t>(row) * g.chunks + c];
        m = p > m ? p : m;
    }
    return block_max256(m);
}

// ---- stage 2: e = expf(v - m) in place --------------------------------------

template <bool EH> // the bucket path: also the histogram of e's first digits
__global__ __launch_bounds__(kBlock) void k_smp_exp(SmpGeo g, float *logits, SmpWs w)
{
    const uint32_t row = blockIdx.x / g.chunks, chunk = blockIdx.x % g.chunks;
    float *x = logits + static_cast<int64_t>(row) * g.ld;
    // expf's 2^(i/32) table in LDS and the e histogram's reset, ordered by
    // row_max's barrier
    __shared__ uint64_t s_tab[32];
    __shared__ uint32_t s_eh[EH ? kBins : 1];
    constexpr bool eh = EH;
    if (threadIdx.x < 32) s_tab[threadIdx.x] = kExp2Table[threadIdx.x];
    if constexpr (eh)
        for (uint32_t b = threadIdx.x; b < kBins; b += blockDim.x) s_eh[b] = 0;
    const float m = row_max(g, w, row);
    uint64_t c0, c1;
    chunk_range(g, chunk, c0, c1);
    const float scale = g.scale;
    const ExpfConsts ec = expf_consts_in_vgprs();
    double acc = 0.0;
    // 4 float4 per step: the expf replica's registers leave room for no more
    // at full occupancy
    visit<true, 4>(g, x, c0, c1, [&](float &v, uint64_t) {
        const float s = v * scale;
        v = emel_expf(s - m, s_tab, ec);
        acc += static_cast<double>(v);
        if constexpr (eh) atomicAdd(&s_eh[__builtin_bit_cast(uint32_t, v) >> 21], 1u);
    });
    if constexpr (eh) flush_hist(s_eh, kBins, w.ehist + static_cast<uint64_t>(row) * kBins, kBins / 2);
    // f64 chunk sum: only a prediction of where the exact sum's binades
    // change (k_smp_seg); never part of a result
    __shared__ double s_acc[kBlock / kWave];
    acc = wave_sum(acc);
    if (threadIdx.x % kWave == 0) s_acc[threadIdx.x / kWave] = acc;
    __syncthreads();
    if (threadIdx.x == 0) w.psum[blockIdx.x] = (s_acc[0] + s_acc[1]) + (s_acc[2] + s_acc[3]);
}

// ---- stage 2b: chunk contributions at a predicted binade --------------------
//
// The exact running sum at the start of chunk c is the f64 prefix P of the
// chunk sums up to the accumulated rounding of the steps before it: each
// step rounds by at most 2^-24 of the running sum, which never decreases,
// so the true value lies within P (1 +- (c0 2^-24 + 2^-30)) -- and likewise
// at the chunk's end.  When both bounds share one binade, the chunk adds a
// whole number of units of that binade; when they span two, it adds a whole
// number of units of either, unless it crosses from one into the other.
// This kernel counts them.  The walk (k_smp_sum) takes a count only after
// checking, on the exact state, that its binade is the state's and that
// the units fit below 2^24: the bound steers the work, the checks decide
// correctness.


// A sub-chunk's units of 2^u (seq_units) and its tie flags (bits 0-2 of
// SegInfo::flags: ok when it holds at most one tie, that tie, its parity).
// Lane l holds kPer of its elements (zeros past its end) in H groups of
// kPer / H consecutive ones, group h starting at element h kSub / H + l kPer
// / H: H = 1 is eight consecutive elements per lane, H = 2 two float4 of a
// wave-contiguous layout.  Called by a whole wave; the result is the same in
// every lane.
template <uint32_t H>
__device__ __forceinline__ void count_units(const float (&e)[kPer], int32_t u, uint32_t &units_out, uint32_t &flags_out)
{
    constexpr uint32_t G = kPer / H;
    static_assert(G * H == kPer, "groups split a lane's elements evenly");
    // Units of 2^u (seq_units): t = e / 2^u, floor(t) plus one when the
    // fraction is above 1/2; a tie (fraction exactly 1/2) counts its lower
    // neighbour here and sets its bit in tmask.
    auto units = [&](float x, uint32_t &q, float &f) {
        float t = __builtin_ldexpf(x, -u);
        t = __builtin_fminf(t, 16777216.0f); // IEEE minNum: also NaN -> 2^24
        f = __builtin_amdgcn_fractf(t);      // t - floor(t), exact for 0 <= t <= 2^24
        q = static_cast<uint32_t>(t);        // floor for t >= 0
    };
    uint32_t gs[H], tmask = 0; // per group at most 8 (2^24 + 1) units: no overflow
#pragma unroll
    for (uint32_t h = 0; h < H; ++h) {
        gs[h] = 0;
#pragma unroll
        for (uint32_t i = 0; i < G; ++i) {
            uint32_t q;
            float f;
            units(e[h * G + i], q, f);
            gs[h] += q + (f > 0.5f ? 1u : 0u);
            tmask |= static_cast<uint32_t>(f == 0.5f) << (h * G + i);
        }
    }
    uint32_t incl[H], total = 0;
#pragma unroll
    for (uint32_t h = 0; h < H; ++h) {
        incl[h] = wave_incl_scan(gs[h] < kSeqLimit ? gs[h] : kSeqLimit);
        total += static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(incl[h]), kWave - 1));
    }
    const uint32_t lane_ties = static_cast<uint32_t>(__builtin_popcount(tmask));
    const uint64_t tl_mask = __ballot(tmask != 0u);
    uint32_t nties = 0;
    for (uint64_t m = tl_mask; m; m &= m - 1)
        nties += static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(lane_ties), __builtin_ctzll(m)));
    units_out = total;
    flags_out = 0u;
    if (nties == 0) {
        flags_out = 1u;
    } else if (nties == 1) { // uniform; the tie sits in lane tl, element ti of group th
        const int tl = __builtin_ctzll(tl_mask);
        const uint32_t ti = tmask ? static_cast<uint32_t>(__builtin_ctz(tmask)) : 0u;
        const uint32_t th = ti / G;
        // units before the tie: the groups before th, this group's lanes
        // before tl, then this lane's elements of group th before ti
        uint32_t before = 0, tq = 0;
#pragma unroll
        for (uint32_t h = 0; h < H; ++h) {
            const uint32_t tot_h = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(incl[h]), kWave - 1));
            const uint32_t excl_h = incl[h] - (gs[h] < kSeqLimit ? gs[h] : kSeqLimit);
            before += h < th ? tot_h : (h == th ? excl_h : 0u);
        }
#pragma unroll
        for (uint32_t i = 0; i < kPer; ++i) {
            uint32_t q;
            float f;
            units(e[i], q, f);
            if (i / G == th && i < ti) before += q + (f > 0.5f ? 1u : 0u);
            if (i == ti) tq = q;
        }
        const uint32_t par = (before + tq) & 1u;
        flags_out = 1u | 2u | (static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(par), tl)) << 2);
    }
}

// A steering margin, not a bound: how far predictions assume the running f32
// sum after `a` roundings strays from the exact prefix, relatively.  Each
// rounding moves it by at most 2^-24 of itself, either way; without a bias in
// the rounding direction the moves mostly cancel, and their total stays near
// sqrt(a) 2^-24 (seq_rel_bound is the worst case, a 2^-24).  A sub-chunk whose
// range under this margin spans a binade boundary probably crosses it.
__device__ __forceinline__ double steer_margin(double a)
{
    return 8.0 * __builtin_sqrt(a) * 0x1p-24;
}

// The plan of one sub-chunk's prediction, packed in 32 bits: its exact
// running sum before and after lies in [lo, hi] (the rounding bound), and
// probably in [wlo, whi] (the steering margin).  When both bounds lie in
// normal f32 binades, one or two adjacent ones, it is counted at the lower
// binade [2^(b-1), 2^b) (u = b - 24) and, for two, at the upper one: bits
// 0-1 hold the number of binades (0: not usable), bit 2 is set when
// [wlo, whi] spans a binade boundary (the sub-chunk probably crosses it and
// is walked), bits 8-31 hold u + kPlanBias.
constexpr int32_t kPlanBias = 512;
__device__ __forceinline__ uint32_t plan_sub(double lo, double hi, double wlo, double whi)
{
    int elo = 0, ehi = 0, wl = 0, wh = 0;
    (void)__builtin_frexp(lo, &elo);
    (void)__builtin_frexp(hi, &ehi);
    (void)__builtin_frexp(wlo, &wl);
    (void)__builtin_frexp(whi, &wh);
    if (!(lo >= 0x1p-126 && hi < 0x1p127 && lo <= hi && ehi - elo <= 1)) return 0u;
    const uint32_t walk = wl != wh ? 4u : 0u;
    return (ehi != elo ? 2u : 1u) | walk | (static_cast<uint32_t>(elo - 1 - 23 + kPlanBias) << 8);
}

// The prediction of one sub-chunk by its plan (wave-uniform): its counts at
// one or two binades, else not usable; the likely-walked bit when the plan
// says so or neither count is usable.
template <uint32_t H>
__device__ __forceinline__ SegInfo predict_sub(const float (&e)[kPer], uint32_t plan)
{
    SegInfo info{0, 0, kSegWalk, 0};
    const uint32_t nb = plan & 3u;
    if (nb == 0) return info;
    info.u = static_cast<int32_t>(plan >> 8) - kPlanBias;
    info.flags = kSegHasU;
    // one copy of the count, run once per binade: the two counts never hold
    // registers at the same time
#pragma nounroll
    for (uint32_t b = 0; b < nb; ++b) {
        uint32_t units, flags;
        count_units<H>(e, info.u + static_cast<int32_t>(b), units, flags);
        if (b == 0) info.units = units;
        else info.units1 = units;
        info.flags |= flags << (b * kSegUpper);
    }
    if ((plan & 4u) || (info.flags & (1u | (1u << kSegUpper))) == 0u) info.flags |= kSegWalk;
    return info;
}

// The row's first sub-chunk, added one element at a time by lane 0: the
// reference's own arithmetic.  At the start of a row the running sum is
// comparable to its addends, and a binade crossing or a tie comes every few
// elements, each of which would cost the walk a round.  Returns slot 0's
// SegInfo: the state after it.  e is this lane's part of the sub-chunk in
// predict_sub's layout H (+0 past the row's end, which leaves the never -0
// running sum unchanged); s_buf is kSub floats of this wave's LDS.  Called
// by a whole wave.
template <uint32_t H>
__device__ __forceinline__ SegInfo head_state(const float (&e)[kPer], float4 *s_buf)
{
    constexpr uint32_t G = kPer / H;
    static_assert(G % 4 == 0, "whole float4 per group");
    const uint32_t lane = threadIdx.x % kWave;
#pragma unroll
    for (uint32_t h = 0; h < H; ++h)
#pragma unroll
        for (uint32_t j = 0; j < G / 4; ++j)
            s_buf[(h * (kSub / H) + lane * G) / 4 + j] =
                make_float4(e[h * G + 4 * j], e[h * G + 4 * j + 1], e[h * G + 4 * j + 2], e[h * G + 4 * j + 3]);
    // this wave's LDS writes before lane 0's reads
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    float acc = 0.0f;
    if (lane == 0) {
#pragma unroll 8
        for (uint32_t j = 0; j < kSub / 4; ++j) {
            const float4 q = s_buf[j];
            acc += q.x;
            acc += q.y;
            acc += q.z;
            acc += q.w;
        }
    }
    acc = __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, acc)));
    SegInfo info{0, 0, kSegEmpty | kSegState, 0};
    if (!(acc < __builtin_inff())) { // NaN or +inf
        info.flags |= kSegSpecial;
        info.units1 = __builtin_bit_cast(uint32_t, acc);
    } else {
        const SeqState st = seq_state(acc);
        info.units = st.m;
        info.u = st.u;
    }
    return info;
}

// One 256-thread workgroup per (row, chunk); wave w predicts sub-chunks
// w, w + 4, ... from its kPer elements per lane.  A sub-chunk with one tie is
// still usable: the tie rounds its sum to an even number of units, so it
// adds q or q + 1 units depending on the parity of the units before it,
// recorded as `par`.
__global__ __launch_bounds__(kBlock) void k_smp_seg(SmpGeo g, float *logits, SmpWs w)
{
    __shared__ double s_red[kBlock / kWave];
    __shared__ double s_sub[kMaxSub];
    __shared__ float4 s_head[kSub / 4]; // wave 0 of a row's first chunk: the head
    const uint32_t row = blockIdx.x / g.chunks, chunk = blockIdx.x % g.chunks;
    const uint32_t lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    double pre = 0.0;
    for (uint32_t c = threadIdx.x; c < chunk; c += blockDim.x) pre += w.psum[static_cast<uint64_t>(row) * g.chunks + c];
    pre = wave_sum(pre);
    if (lane == 0) s_red[wave] = pre;
    __syncthreads();
    const double P = (s_red[0] + s_red[1]) + (s_red[2] + s_red[3]);
    uint64_t c0, c1;
    chunk_range(g, chunk, c0, c1);
    const uint32_t spc = subs_per_chunk(g);
    const uint32_t nsub = static_cast<uint32_t>((c1 - c0 + kSub - 1) / kSub);
    const uint32_t npred = nsub < kMaxSub ? nsub : kMaxSub;
    SegInfo *out = w.seg + (static_cast<uint64_t>(row) * g.chunks + chunk) * spc;
    const float *x = logits + static_cast<int64_t>(row) * g.ld;
    auto load_sub = [&](uint32_t k, float (&e)[kPer]) {
        const uint64_t first = c0 + static_cast<uint64_t>(k) * kSub + kPer * lane;
        if (g.vec && first + kPer <= c1) {
            const float4 *p4 = reinterpret_cast<const float4 *>(x + first);
#pragma unroll
            for (uint32_t j = 0; j < kPer / 4; ++j) {
                const float4 q = p4[j];
                e[4 * j] = q.x;
                e[4 * j + 1] = q.y;
                e[4 * j + 2] = q.z;
                e[4 * j + 3] = q.w;
            }
        } else {
#pragma unroll
            for (uint32_t j = 0; j < kPer; ++j) e[j] = first + j < c1 ? x[first + j] : 0.0f;
        }
    };
    // pass A: f64 sum of every sub-chunk
    for (uint32_t k = wave; k < npred; k += kBlock / kWave) {
        float e[kPer];
        load_sub(k, e);
        double acc = 0.0;
#pragma unroll
        for (uint32_t j = 0; j < kPer; ++j) acc += static_cast<double>(e[j]);
        acc = wave_sum(acc);
        if (lane == 0) s_sub[k] = acc;
    }
    __syncthreads();
    // slots past the chunk's last sub-chunk (only in a shorter last chunk)
    // are empty: they add nothing, whatever the state
    for (uint32_t k = nsub + threadIdx.x; k < spc; k += blockDim.x) out[k] = SegInfo{0, 0, kSegEmpty, 0};
    // pass B: the prediction per sub-chunk
    for (uint32_t k = wave; k < nsub; k += kBlock / kWave) {
        SegInfo info{0, 0, kSegWalk, 0}; // past kMaxSub: walked
        const uint64_t a0 = c0 + static_cast<uint64_t>(k) * kSub;
        const uint64_t a1 = a0 + kSub < c1 ? a0 + kSub : c1;
        if (k < npred) {
            double Pk = P;
            for (uint32_t i = 0; i < k; ++i) Pk += s_sub[i];
            const double end = Pk + s_sub[k];
            const uint32_t plan = plan_sub(Pk * (1.0 - seq_rel_bound(static_cast<double>(a0))),
                                           end * (1.0 + seq_rel_bound(static_cast<double>(a1))),
                                           Pk * (1.0 - steer_margin(static_cast<double>(a0))),
                                           end * (1.0 + steer_margin(static_cast<double>(a1))));
            float e[kPer];
            load_sub(k, e);
            // the row's first sub-chunk: the walk's starting state instead
            info = chunk == 0 && k == 0 ? head_state<1>(e, s_head) : predict_sub<1>(e, plan);
        }
        if (lane == 0) out[k] = info;
    }
}

// ---- stages 2 and 2b in one pass (chunks of at most kFuseSubs sub-chunks) ---
//
// e = expf(v - m) in place, as k_smp_exp computes it, and each sub-chunk's
// prediction as k_smp_seg makes it, from the e still in registers.  The sum
// of e before a sub-chunk, and the sub-chunk's own, come from
// k_smp_max<true>'s approximate sums (of the chunks before this one, then
// of this chunk's sub-chunks before it), rescaled from their maxima to the
// row's; the bounds widen by kApproxRel for their error.  Every wave works
// on its own: no barrier, and the next sub-chunk's loads are in flight while
// the current one is computed.  The walk's checks on the exact state decide
// every prediction, so an approximate sum can only cost walks.
//
// Relative error of those sums, bounded with a wide margin: an approximate
// exponential is within (1 + |x|) 2^-23 of exp(x) and the exact e within
// (1 + |x|) 2^-24 of exp(v - m) (x = v - the maximum it is taken from, so
// |x| grows only as e shrinks); weighted by size, a sum of N terms is then
// within (2 + ln N) 2^-23, about 2^-19 for a 151,936-token row.  The f32
// sums inside a sub-chunk (8 terms per lane, then a six-level wave tree) and
// the f32 stores add at most 15 2^-24 more.
constexpr double kApproxRel = 0x1p-14;

__device__ __forceinline__ double readlane_f64(double v, uint32_t l)
{
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(b)), l));
    const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(b >> 32)), l));
    return __builtin_bit_cast(double, (static_cast<uint64_t>(hi) << 32) | lo);
}

constexpr uint32_t kFastBits = 14;       // low key bits the fast threshold leaves 0 (2^-9 of e_thr at most)

// The fast candidate threshold, by one wave.  The top_k largest sub-chunk
// maxima are top_k distinct elements; with e_thr the top_k-th largest of
// their e (computed as k_smp_expseg computes e), at least top_k elements
// have e >= e_thr, so p >= p_thr = e_thr / S (the division k_smp_div uses,
// correctly rounded and so monotone), and every element of the top_k by p
// -- ties at the boundary included -- has p >= p_thr.  k_smp_div then lists
// those elements directly.  Returns false when the row cannot take it
// (three-pass chunks, top_k above kCap or above the sub-chunk count, more
// than kFastPer sub-chunks per lane).
__device__ bool fast_threshold(const SmpGeo &g, const SmpWs &w, uint32_t row, uint32_t lane, const uint64_t *tab,
                               uint32_t &ethr_key)
{
    const uint32_t spc = subs_per_chunk(g), nslots = g.chunks * spc;
    if (!fast_list_possible(g)) return false;
    const SubSum *sub = w.sub + static_cast<uint64_t>(row) * nslots;
    // only the last chunk can hold empty slots: its first `tail` slots are written
    const uint32_t last = (g.chunks - 1) * spc;
    const uint32_t tail = static_cast<uint32_t>((g.card - static_cast<uint64_t>(g.chunks - 1) * g.chunk_cols + kSub - 1) / kSub);
    float mv[kFastPer];
    bool valid[kFastPer];
    float M = -__builtin_inff();
#pragma unroll
    for (uint32_t j = 0; j < kFastPer; ++j) {
        const uint32_t slot = lane + kWave * j;
        valid[j] = slot < nslots && (slot < last || slot - last < tail); // written by k_smp_max<true>
        mv[j] = valid[j] ? sub[slot].m : -__builtin_inff();
        M = mv[j] > M ? mv[j] : M;
    }
    M = wave_max_dpp(M); // the row maximum: every element lies in a sub-chunk
    const ExpfConsts ec = expf_consts_in_vgprs();
    uint32_t key[kFastPer];
    uint32_t nvalid = 0;
#pragma unroll
    for (uint32_t j = 0; j < kFastPer; ++j) {
        key[j] = valid[j] ? total_key(emel_expf(mv[j] - M, tab, ec)) : 0u; // valid keys are > 0
        nvalid += static_cast<uint32_t>(__builtin_popcountll(__ballot(valid[j])));
    }
    if (nvalid < g.top_k) return false;
    // The largest t with top_k keys >= t, bit by bit from the top; the bits
    // below kFastBits stay 0, which only lowers t (a lower threshold lists a
    // few more candidates, never fewer).
    uint32_t t = 0;
    for (int b = 31; b >= static_cast<int>(kFastBits); --b) {
        const uint32_t c = t | (1u << b);
        uint32_t n = 0;
#pragma unroll
        for (uint32_t j = 0; j < kFastPer; ++j) n += static_cast<uint32_t>(__builtin_popcountll(__ballot(key[j] >= c)));
        if (n >= g.top_k) t = c;
    }
    ethr_key = t;
    return true;
}

// The row maximum of v, from the chunk maxima (every lane of a wave).
__device__ __forceinline__ float row_max_wave(const SmpGeo &g, const SmpWs &w, uint32_t row, uint32_t lane)
{
    const uint64_t rbase = static_cast<uint64_t>(row) * g.chunks;
    float m = -__builtin_inff();
    for (uint32_t c = lane; c < g.chunks; c += kWave) {
        const float p = w.part[rbase + c];
        m = p > m ? p : m;
    }
    return wave_max_dpp(m);
}

// A head workgroup of k_smp_expseg (one per row, first in the grid): its
// first wave computes the row's first sub-chunk's e, as the (row, 0)
// workgroup does, and adds them one by one (head_state) into slot 0.  Its
// own workgroup, dispatched before the others, keeps this serial chain off
// the tail of the pass.
__device__ __forceinline__ void expseg_head(const SmpGeo &g, const float *logits, const SmpWs &w, uint32_t row,
                                            uint64_t *tab, float4 *s_head)
{
    const uint32_t lane = threadIdx.x % kWave;
    const float *x = logits + static_cast<int64_t>(row) * g.ld;
    uint64_t c0, c1;
    chunk_range(g, 0, c0, c1);
    float v[kPer];
    load_split(g, x, c0, c1, lane, true, v);
    const float m = row_max_wave(g, w, row, lane);
    const ExpfConsts ec = expf_consts_in_vgprs();
    if (lane < 32) tab[lane] = kExp2Table[lane];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
#pragma unroll
    for (uint32_t q = 0; q < kPer; ++q)
        v[q] = split_col(c0, lane, q) < c1 ? emel_expf(v[q] * g.scale - m, tab, ec) : 0.0f;
    const SegInfo head = head_state<kSplit>(v, s_head);
    if (lane == 0) w.seg[static_cast<uint64_t>(row) * g.chunks * subs_per_chunk(g)] = head;
}

// Grid: g.rows head workgroups (expseg_head), then one per (row, chunk).
template <bool EH> // the bucket path: also the histogram of e's first digits
__global__ __launch_bounds__(kBlock) void k_smp_expseg(SmpGeo g, float *logits, SmpWs w)
{
    const uint32_t lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    // each wave's own copy of expf's 2^(i/32) table in LDS: no workgroup barrier
    __shared__ uint64_t s_tab[kBlock / kWave][32];
    if (blockIdx.x < g.rows) {
        __shared__ float4 s_head[kSub / 4];
        if (wave == 0) expseg_head(g, logits, w, blockIdx.x, s_tab[0], s_head);
        if (wave == 1) { // beside it: e_thr for the fast candidate list
            if (lane < 32) s_tab[1][lane] = kExp2Table[lane];
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
            uint32_t key = 0;
            const bool ok = fast_threshold(g, w, blockIdx.x, lane, s_tab[1], key);
            if (lane == 0) {
                w.sel[blockIdx.x].ethr_key = key;
                w.sel[blockIdx.x].ethr_on = ok ? 1u : 0u;
            }
        }
        return;
    }
    const uint32_t b = blockIdx.x - g.rows;
    const uint32_t row = b / g.chunks, chunk = b % g.chunks;
    float *x = logits + static_cast<int64_t>(row) * g.ld;
    uint64_t c0, c1;
    chunk_range(g, chunk, c0, c1);
    // the bucket path: the histogram of e's first digits (flushed at the end).
    // e is +0 or more, or NaN, so its key is its bits with the top bit set and
    // the bins count bits >> 21, which the flush moves up by kBins / 2.
    __shared__ uint32_t s_eh[EH ? kBins : 1];
    constexpr bool eh = EH;
    if constexpr (eh) {
        for (uint32_t d = threadIdx.x; d < kBins; d += blockDim.x) s_eh[d] = 0;
        __syncthreads();
    }
    const uint32_t spc = subs_per_chunk(g);
    const uint32_t nsub = static_cast<uint32_t>((c1 - c0 + kSub - 1) / kSub); // <= kFuseSubs
    auto sub_col = [&](uint32_t k) { return c0 + static_cast<uint64_t>(k) * kSub; };
    // the first sub-chunk's loads go out before the row state is read
    float cur[kPer];
    load_split(g, x, sub_col(wave), c1, lane, wave < nsub, cur);
    const uint64_t rbase = static_cast<uint64_t>(row) * g.chunks;
    const float m = row_max_wave(g, w, row, lane);
    double pre = 0.0; // ~ sum of e over the chunks before this one
    for (uint32_t c = lane; c < chunk; c += kWave) {
        const double sc = w.psum[rbase + c];
        // m = +inf makes it NaN (inf - inf), and every prediction fails
        if (sc != 0.0) pre += sc * exp(static_cast<double>(w.part[rbase + c]) - static_cast<double>(m));
    }
    pre = wave_sum_dpp(pre);
    double term = 0.0; // lane i: ~ sum of e over sub-chunk i of this chunk
    if (lane < nsub) {
        const SubSum ss = w.sub[(rbase + chunk) * spc + lane];
        if (ss.s != 0.0f) term = static_cast<double>(ss.s) * exp(static_cast<double>(ss.m) - static_cast<double>(m));
    }
    const double incl = wave_incl_scan_f64(term);
    // lane i: sub-chunk i's prediction plan, from the sums before and at it
    uint32_t plan = 0;
    if (lane < nsub) {
        const double before = pre + (incl - term);
        const double end = before + term;
        const uint64_t a0 = sub_col(lane);
        const double a1 = static_cast<double>(a0 + kSub < c1 ? a0 + kSub : c1);
        const double lo = before * (1.0 - kApproxRel), hi = end * (1.0 + kApproxRel);
        plan = plan_sub(lo * (1.0 - seq_rel_bound(static_cast<double>(a0))), hi * (1.0 + seq_rel_bound(a1)),
                        lo * (1.0 - steer_margin(static_cast<double>(a0))), hi * (1.0 + steer_margin(a1)));
    }
    SegInfo *out = w.seg + (rbase + chunk) * spc;
    // slots past the chunk's last sub-chunk (only in a shorter last chunk)
    // are empty: they add nothing, whatever the state
    for (uint32_t k = nsub + threadIdx.x; k < spc; k += blockDim.x) out[k] = SegInfo{0, 0, kSegEmpty, 0};
    const float scale = g.scale;
    const ExpfConsts ec = expf_consts_in_vgprs();
    if (lane < 32) s_tab[wave][lane] = kExp2Table[lane];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    const uint64_t *tab = s_tab[wave];
#pragma unroll
    for (uint32_t j = 0; j < kFusePerWave; ++j) {
        const uint32_t k = wave + (kBlock / kWave) * j;
        if (k >= nsub) break; // wave-uniform
        float nxt[kPer];
        if (j + 1 < kFusePerWave)
            load_split(g, x, sub_col(k + kBlock / kWave), c1, lane, k + kBlock / kWave < nsub, nxt);
        const uint64_t a0 = sub_col(k);
        if (a0 + kSub <= c1) { // only a row's last sub-chunk can end early
#pragma unroll
            for (uint32_t q = 0; q < kPer; ++q) cur[q] = emel_expf(cur[q] * scale - m, tab, ec);
            if constexpr (eh)
#pragma unroll
                for (uint32_t q = 0; q < kPer; ++q) atomicAdd(&s_eh[__builtin_bit_cast(uint32_t, cur[q]) >> 21], 1u);
        } else {
#pragma unroll
            for (uint32_t q = 0; q < kPer; ++q) {
                const bool in = split_col(a0, lane, q) < c1;
                cur[q] = in ? emel_expf(cur[q] * scale - m, tab, ec) : 0.0f;
                if constexpr (eh)
                    if (in) atomicAdd(&s_eh[__builtin_bit_cast(uint32_t, cur[q]) >> 21], 1u);
            }
        }
#pragma unroll
        for (uint32_t h = 0; h < kSplit; ++h) {
            const uint64_t col = split_col(a0, lane, 4 * h);
            if (g.vec && col + 4 <= c1) {
                *reinterpret_cast<float4 *>(x + col) = make_float4(cur[4 * h], cur[4 * h + 1], cur[4 * h + 2], cur[4 * h + 3]);
            } else {
#pragma unroll
                for (uint32_t q = 0; q < 4; ++q)
                    if (col + q < c1) x[col + q] = cur[4 * h + q];
            }
        }
        const SegInfo info =
            predict_sub<kSplit>(cur, static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(plan), k)));
        // the row's first slot holds the head workgroup's state instead
        if (lane == 0 && (chunk != 0 || k != 0)) out[k] = info;
        if (j + 1 < kFusePerWave) {
#pragma unroll
            for (uint32_t q = 0; q < kPer; ++q) cur[q] = nxt[q];
        }
    }
    if constexpr (eh) flush_hist(s_eh, kBins, w.ehist + static_cast<uint64_t>(row) * kBins, kBins / 2);
}

// ---- stage 3: the exact sequential sum of e ----------------------------------
//
// One wave per row walks the row's sub-chunks in order.  A sub-chunk whose
// predicted contribution (k_smp_seg) holds on the exact state -- the same
// binade, and the units stay below 2^24, so no element inside it can cross
// (units never decrease) -- is added in one step.  Any other sub-chunk is
// walked as one tile of 64 lanes x kPer elements: a round computes the
// tile's units at the current binade and their wave prefix sum, and either
// commits the rest of the tile (no event) or finds the first event
// element, adds it with one f32 addition and starts the next round after
// it.  Each round commits at least one element, so the rounds end.

constexpr uint32_t kFastWg = 256;        // fast candidates a k_smp_div workgroup buffers
constexpr uint32_t kStage = 24;          // walked sub-chunks k_smp_sum's second wave stages in LDS


// One wave per row walks (wave 0); wave 1 stages sub-chunks for it, and on
// the bucket path a third wave picks e's first digit holding the top_k-th
// largest e, both off the walk's path.  The sub-chunks' predictions are
// read a batch at a time (lane i holds sub-chunk kb + i's).  A sub-chunk
// whose predicted contribution holds on the exact state -- the same binade,
// and the units (its one tie resolved by the current parity) stay below
// 2^24, so no element inside it can cross (units never decrease) -- is
// added in one step.  Any other sub-chunk is loaded straight into the
// walk's registers (lane l holds its elements kPer l .. kPer l + kPer - 1,
// 128-bit loads in flight) and walked: one round, plus one per event.
// Per lane of a staged sub-chunk with a usable plan (lower binade u), left
// by k_smp_sum's second wave: the inclusive wave scans of the lane unit
// totals at u and at u + 1 (each total capped at 2^24, as the walk's rounds
// cap them) and whether the lane holds a tie at u (bit 0) or u + 1 (bit 1).
struct LaneScan {
    uint32_t incl0, incl1, ties, pad;
};

// A lane's unit total at 2^u of its elements (capped at 2^24; NaN counts
// 2^24) and whether one of them is a tie (seq_units).
__device__ __forceinline__ uint32_t lane_units(const float (&e)[kPer], int32_t u, bool &tie)
{
    uint32_t lsum = 0;
    float dmax = 0.0f;
#pragma unroll
    for (uint32_t j = 0; j < kPer; ++j) {
        float t = __builtin_ldexpf(e[j], -u);
        t = __builtin_fminf(t, 16777216.0f);
        const float rt = __builtin_rintf(t);
        lsum += static_cast<uint32_t>(rt);
        dmax = __builtin_fmaxf(dmax, __builtin_fabsf(t - rt));
    }
    tie = dmax == 0.5f;
    return lsum < kSeqLimit ? lsum : kSeqLimit;
}

// One step for a sub-chunk whose walk starts in its lower binade u (s.u ==
// u), from its lane scans (ls, this lane's) and its elements in LDS (st, the
// walk's register layout).  The first event
// at u -- a tie, or the element whose units reach 2^24 -- lies in the first
// lane whose tie bit is set or whose scan reaches 2^24 - m; that lane's
// elements are spread over lanes 0-7 and resolved there, and the event is
// added with one f32 addition.  When it is the crossing into u + 1, and the
// rest of the sub-chunk holds no tie at u + 1 and its units there keep the
// state below 2^24, the state after the sub-chunk follows from the scans at
// u + 1.  Returns kStepDone with s the state after the sub-chunk, kStepEvent
// with s the state after element k (the caller walks the elements after
// it), or kStepNone with s unchanged (a NaN or +inf sum: the caller walks the
// whole sub-chunk).
constexpr uint32_t kStepDone = 0, kStepEvent = 1, kStepNone = 2;

// Inclusive prefix sum over lanes 0-7 (row shifts of 1, 2, 4 inside the
// first row of 16 lanes; the other lanes' results are not used).
__device__ __forceinline__ uint32_t scan8(uint32_t v)
{
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x111, 0xf, 0xf, true)); // row_shr:1
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x112, 0xf, 0xf, true)); // row_shr:2
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x114, 0xf, 0xf, true)); // row_shr:4
    return v;
}

__device__ __forceinline__ uint32_t crossing_step(const LaneScan ls, const float4 (&st)[kPer / 4][kWave], int32_t u,
                                                  SumState &s, uint32_t &k)
{
    static_assert(kPer == 8, "a lane's elements spread over lanes 0-7");
    const uint32_t lane = threadIdx.x % kWave;
    const uint64_t emask = __ballot((ls.ties & 1u) || s.m + ls.incl0 >= kSeqLimit);
    if (emask == 0) { // no event at u: the sub-chunk adds its units
        s.m += static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(ls.incl0), kWave - 1));
        return kStepDone;
    }
    const int fl = __builtin_ctzll(emask);
    // lane fl's elements, element i in lane i (i < 8): one LDS read each
    const uint32_t i = lane % kPer;
    const float *stf = reinterpret_cast<const float *>(&st[0][0]);
    const float ev = stf[((i / 4) * kWave + static_cast<uint32_t>(fl)) * 4 + (i % 4)];
    const float ei = lane < kPer ? ev : 0.0f;
    const uint32_t before = fl == 0 ? 0u : static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(ls.incl0), fl - 1));
    // their units and t - rint(t) at u and at u + 1, with in-lane prefixes
    auto units = [&](int32_t b, float &d) {
        float t = __builtin_ldexpf(ei, -b);
        t = __builtin_fminf(t, 16777216.0f); // also NaN -> 2^24
        const float rt = __builtin_rintf(t);
        d = t - rt;
        return static_cast<uint32_t>(rt);
    };
    float d0, d1;
    const uint32_t r0 = units(u, d0), r1 = units(u + 1, d1);
    const uint32_t p0 = scan8(r0), p1 = scan8(r1);
    const uint32_t base = s.m + before;
    const uint64_t jmask = __ballot(lane < kPer && (__builtin_fabsf(d0) == 0.5f || base + p0 >= kSeqLimit));
    if (jmask == 0) return kStepNone; // unreachable: lane fl holds an event
    const int jc = __builtin_ctzll(jmask);
    const uint32_t run_k = base + static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(p0 - r0), jc));
    const float e_k = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, ei), jc));
    const float sn = seq_value(run_k, u) + e_k; // the event element: one f32 addition
    if (!(sn < __builtin_inff())) return kStepNone;
    const SeqState nx = seq_state(sn);
    k = kPer * static_cast<uint32_t>(fl) + static_cast<uint32_t>(jc);
    s.m = nx.m;
    s.u = nx.u;
    if (nx.u != u + 1) return kStepEvent;
    // the rest at u + 1: lane fl's elements after jc, then the lanes after fl
    const uint32_t in_lane = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(p1), kPer - 1)) -
                             static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(p1), jc));
    const uint32_t total1 = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(ls.incl1), kWave - 1));
    const uint32_t upto1 = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(ls.incl1), fl));
    const uint64_t t1in = __ballot(lane < kPer && __builtin_fabsf(d1) == 0.5f) >> (jc + 1);
    const uint64_t t1out = __ballot(lane > static_cast<uint32_t>(fl) && (ls.ties & 2u));
    const uint64_t rest = static_cast<uint64_t>(in_lane) + (total1 - upto1);
    if (t1in != 0 || t1out != 0 || s.m + rest >= kSeqLimit) return kStepEvent;
    s.m += static_cast<uint32_t>(rest);
    return kStepDone;
}

constexpr uint32_t kSumThreads = 3 * kWave; // the third wave on the bucket path only

__global__ __launch_bounds__(kSumThreads) void k_smp_sum(SmpGeo g, const float *logits, SmpWs w)
{
    // wave 1 stages the walk-marked sub-chunks: s_stage[i] holds the i-th
    // of them (in slot order) as the walk's registers hold it (float4 q of
    // lane l at [i][q][l]); s_ready counts the staged ones (release /
    // acquire)
    __shared__ float4 s_stage[kStage][kPer / 4][kWave];
    __shared__ LaneScan s_lanes[kStage][kWave]; // with a usable plan: the lane scans (crossing_step)
    __shared__ float4 s_own[kPer / 4][kWave];   // wave 0: a sub-chunk it loaded, for crossing_step
    __shared__ uint32_t s_ready;
    __shared__ uint32_t s_edig; // the bucket path: e's first digit holding the top_k-th largest e
    const uint32_t row = blockIdx.x;
    const uint32_t lane = threadIdx.x % kWave;
    const float *x = logits + static_cast<int64_t>(row) * g.ld;
    const uint32_t spc = subs_per_chunk(g);
    const uint64_t card4 = g.card & ~uint64_t{3};
    // The row's predictions form one list of chunks * spc slots; they are
    // read 64 at a time (lane i holds slot base + i), the next batch in
    // flight while this one is used.
    const uint32_t nslots = g.chunks * spc;
    const SegInfo *seg = w.seg + static_cast<uint64_t>(row) * nslots;
    // the walk starts from the state after the row's first sub-chunk (its
    // head, added one by one by the prediction pass)
    SumState s{0u, -149, true, 0.0f};
    {
        const SegInfo h = seg[0];
        if (h.flags & kSegSpecial) {
            s.finite = false;
            s.special = __builtin_bit_cast(float, h.units1);
        } else {
            s.m = h.units;
            s.u = h.u;
        }
    }
    // A sub-chunk's element count (1 .. kSub) and first column.
    auto slot_range = [&](uint32_t slot, uint64_t &a0) {
        uint64_t c0, c1;
        chunk_range(g, slot / spc, c0, c1);
        a0 = c0 + static_cast<uint64_t>(slot % spc) * kSub;
        const uint64_t a1 = a0 + kSub < c1 ? a0 + kSub : c1;
        return static_cast<uint32_t>(a1 - a0);
    };
    // A sub-chunk's elements kPer lane .. kPer lane + kPer - 1 into e (+0 past
    // its end); every address is clamped into the sub-chunk, so the loads
    // are unconditional.
    auto load_slot = [&](uint32_t slot, float (&e)[kPer], uint32_t &n) {
        uint64_t a0;
        n = slot_range(slot, a0);
        const uint64_t a1 = a0 + n;
        const uint32_t c = kPer * lane;
        if (g.vec && a1 <= card4) { // a0 and n are multiples of 4: whole float4s
            const float4 *x4 = reinterpret_cast<const float4 *>(x + a0);
            float4 q[kPer / 4];
#pragma unroll
            for (uint32_t j = 0; j < kPer / 4; ++j) q[j] = x4[c + 4 * j < n ? c / 4 + j : 0u];
#pragma unroll
            for (uint32_t j = 0; j < kPer / 4; ++j) {
                const bool in = c + 4 * j < n;
                e[4 * j] = in ? q[j].x : 0.0f;
                e[4 * j + 1] = in ? q[j].y : 0.0f;
                e[4 * j + 2] = in ? q[j].z : 0.0f;
                e[4 * j + 3] = in ? q[j].w : 0.0f;
            }
        } else {
#pragma unroll
            for (uint32_t j = 0; j < kPer; ++j) e[j] = x[a0 + (c + j < n ? c + j : 0u)];
#pragma unroll
            for (uint32_t j = 0; j < kPer; ++j) e[j] = c + j < n ? e[j] : 0.0f;
        }
    };
    if (threadIdx.x == 0) {
        s_ready = 0;
        s_edig = kNone;
    }
    __syncthreads();
    if (threadIdx.x >= 2 * kWave) { // wave 2 (the bucket path)
        // e's first digit holding the top_k-th largest e (every e counted
        // once by the exponential pass), 32 digits per lane
        const uint4 *eh = reinterpret_cast<const uint4 *>(w.ehist + static_cast<uint64_t>(row) * kBins) + 8 * lane;
        uint32_t c[32], local = 0;
#pragma unroll
        for (uint32_t i = 0; i < 8; ++i) {
            const uint4 h = eh[i];
            c[4 * i] = h.x;
            c[4 * i + 1] = h.y;
            c[4 * i + 2] = h.z;
            c[4 * i + 3] = h.w;
        }
#pragma unroll
        for (uint32_t i = 0; i < 32; ++i) local += c[i];
        const uint32_t incl = wave_incl_scan(local);
        uint32_t cum = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(incl), kWave - 1)) - incl;
#pragma unroll
        for (int i = 31; i >= 0; --i) {
            if (cum < g.top_k && g.top_k <= cum + c[i]) s_edig = 32 * lane + static_cast<uint32_t>(i);
            cum += c[i];
        }
    } else if (threadIdx.x >= kWave) { // wave 1
        // Stage, in slot order, the sub-chunks marked as probably walked
        // (almost every sub-chunk the walk loads).  The walk takes a staged
        // sub-chunk from LDS when it is ready and loads it itself otherwise,
        // so it never waits.
        uint32_t nst = 0;
        for (uint32_t kb = 0; kb < nslots && nst < kStage; kb += kWave) {
            const uint32_t sl = kb + lane;
            SegInfo si{0, 0, kSegEmpty, 0};
            if (sl < nslots && sl != 0) si = seg[sl];
            uint64_t m = __ballot((si.flags & (kSegWalk | kSegEmpty)) == kSegWalk);
            while (m != 0 && nst < kStage) {
                const int bit = __builtin_ctzll(m);
                const uint32_t slot = kb + static_cast<uint32_t>(bit);
                m &= m - 1;
                float e[kPer];
                uint32_t n;
                load_slot(slot, e, n);
#pragma unroll
                for (uint32_t q = 0; q < kPer / 4; ++q)
                    s_stage[nst][q][lane] = make_float4(e[4 * q], e[4 * q + 1], e[4 * q + 2], e[4 * q + 3]);
                const uint32_t sf = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(si.flags), bit));
                if (sf & kSegHasU) { // the lane scans at its two binades
                    const int32_t su = __builtin_amdgcn_readlane(si.u, bit);
                    bool t0, t1;
                    const uint32_t x0 = lane_units(e, su, t0);
                    const uint32_t x1 = lane_units(e, su + 1, t1);
                    s_lanes[nst][lane] = LaneScan{wave_incl_scan(x0), wave_incl_scan(x1),
                                                  static_cast<uint32_t>(t0) | (static_cast<uint32_t>(t1) << 1), 0u};
                }
                ++nst;
                if (lane == 0) __hip_atomic_store(&s_ready, nst, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_WORKGROUP);
            }
        }
    } else { // wave 0: the walk
    bool nan_final = false;
    uint32_t marked = 0; // walk-marked slots before this batch: wave 1 stages them in this order
    uint32_t ready = 0;  // staged slots known to be ready (s_ready only grows)
    uint32_t pre_slot = kNone; // prefetched into pre_e
    float pre_e[kPer];
    SegInfo nxt{0, 0, kSegEmpty, 0};
    if (lane < nslots) nxt = seg[lane];
    for (uint32_t kb = 0; kb < nslots && !nan_final; kb += kWave) {
        const SegInfo mine = nxt;
        if (kb + kWave + lane < nslots) nxt = seg[kb + kWave + lane];
        const uint32_t nb = nslots - kb < kWave ? nslots - kb : kWave;
        const uint64_t wmask =
            __ballot(lane < nb && kb + lane != 0 && (mine.flags & (kSegWalk | kSegEmpty)) == kSegWalk);
        if (kb == 0 && wmask != 0) { // the first walk-marked slot: usually reached before wave 1 stages it
            pre_slot = static_cast<uint32_t>(__builtin_ctzll(wmask));
            uint32_t n;
            load_slot(pre_slot, pre_e, n);
        }
        uint32_t i = 0; // next slot of the batch
        while (i < nb) {
            // Take the run of slots from i on that need no decision: empty
            // ones, and usable sub-chunks counted at the current binade,
            // their units below 2^24 -- one wave prefix sum finds where the
            // run ends.
            bool fail = false, tie = false;
            uint32_t add = 0, par = 0;
            if (lane >= i && lane < nb) {
                const bool empty = (mine.flags & kSegEmpty) != 0;
                const bool upper = mine.u + 1 == s.u;
                const uint32_t fb = mine.flags >> (upper ? kSegUpper : 0u); // the state's binade's bits
                const bool easy = empty || (s.finite && (fb & 1u) && (upper || mine.u == s.u));
                add = easy && !empty ? (upper ? mine.units1 : mine.units) : 0u;
                tie = easy && !empty && (fb & 2u);
                par = (fb >> 2) & 1u;
                fail = !easy;
            }
            const uint32_t x = add < kSeqLimit ? add : kSeqLimit;
            uint32_t incl = wave_incl_scan(x);
            // A slot with one tie adds one more unit when the running units
            // before it plus its tie's parity bit are odd (round to even).
            // Its correction moves the slots after it, so they are settled
            // in order, on the scalar unit: at most a few per batch.
            const uint64_t tmask = __ballot(tie);
            if (tmask) {
                const uint32_t excl = incl - x;
                uint64_t cmask = 0;
                uint32_t cacc = 0;
                for (uint64_t m = tmask; m; m &= m - 1) {
                    const int tl = __builtin_ctzll(m);
                    const uint32_t c = (s.m + static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(excl), tl)) +
                                        cacc + static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(par), tl))) &
                                       1u;
                    cmask |= static_cast<uint64_t>(c) << tl;
                    cacc += c;
                }
                // the corrections at and before this lane
                incl += __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(cmask >> 32),
                                                  __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(cmask), 0u)) +
                        static_cast<uint32_t>((cmask >> lane) & 1u);
            }
            fail = fail || (lane >= i && lane < nb && static_cast<uint64_t>(s.m) + incl >= kSeqLimit);
            const uint64_t fmask = __ballot(fail);
            const uint32_t f = fmask ? static_cast<uint32_t>(__builtin_ctzll(fmask)) : nb;
            if (f > i) s.m += static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(incl), f - 1));
            if (f >= nb) break;
            i = f + 1;
            if (!s.finite && s.special != s.special) { // NaN is final
                nan_final = true;
                break;
            }
            // slot f is walked: from LDS when wave 1 has staged it (the
            // staged slots are the walk-marked ones, in slot order), else
            // from the prefetch or a load of its own
            float e[kPer];
            bool staged = false;
            const uint32_t sidx = marked + static_cast<uint32_t>(__builtin_popcountll(wmask & ((uint64_t{1} << f) - 1u)));
            if ((wmask >> f) & 1u) {
                if (sidx >= ready) ready = __hip_atomic_load(&s_ready, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP);
                staged = sidx < ready;
            }
            // in its lower binade, a sub-chunk with a usable plan crosses in
            // one step (crossing_step)
            const int32_t su = __builtin_amdgcn_readlane(mine.u, f);
            const uint32_t sf = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(mine.flags), f));
            const bool one_step = (sf & kSegHasU) && s.finite && su == s.u;
            uint32_t k = kSub;
            uint32_t step = kStepNone;
            if (staged) {
                if (one_step) {
                    const uint4 lv = *reinterpret_cast<const uint4 *>(&s_lanes[sidx][lane]); // one 128-bit read
                    step = crossing_step(LaneScan{lv.x, lv.y, lv.z, lv.w}, s_stage[sidx], su, s, k);
                }
                if (step == kStepDone) continue;
#pragma unroll
                for (uint32_t q = 0; q < kPer / 4; ++q) {
                    const float4 v = s_stage[sidx][q][lane];
                    e[4 * q] = v.x;
                    e[4 * q + 1] = v.y;
                    e[4 * q + 2] = v.z;
                    e[4 * q + 3] = v.w;
                }
            } else {
                if (kb + f == pre_slot) {
#pragma unroll
                    for (uint32_t j = 0; j < kPer; ++j) e[j] = pre_e[j];
                } else {
                    uint32_t n;
                    load_slot(kb + f, e, n);
                }
                if (one_step) { // the lane scans here; the elements into s_own for the spread
#pragma unroll
                    for (uint32_t q = 0; q < kPer / 4; ++q)
                        s_own[q][lane] = make_float4(e[4 * q], e[4 * q + 1], e[4 * q + 2], e[4 * q + 3]);
                    bool t0, t1;
                    const uint32_t x0 = lane_units(e, su, t0);
                    const uint32_t x1 = lane_units(e, su + 1, t1);
                    const LaneScan ls{wave_incl_scan(x0), wave_incl_scan(x1),
                                      static_cast<uint32_t>(t0) | (static_cast<uint32_t>(t1) << 1), 0u};
                    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
                    __builtin_amdgcn_wave_barrier();
                    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
                    step = crossing_step(ls, s_own, su, s, k);
                }
            }
            if (step == kStepDone || (step == kStepEvent && k + 1 >= kSub)) continue;
            if (step == kStepEvent) { // the elements after k remain
                const int32_t kk = static_cast<int32_t>(k) - static_cast<int32_t>(kPer * lane);
#pragma unroll
                for (uint32_t j = 0; j < kPer; ++j) e[j] = static_cast<int32_t>(j) <= kk ? 0.0f : e[j];
            }
            sum_tile<kPer>(e, s);
        }
        marked += static_cast<uint32_t>(__builtin_popcountll(wmask));
    }
    } // wave 0
    __syncthreads(); // wave 2's digit of e
    if (threadIdx.x == 0) {
        const float S = s.finite ? seq_value(s.m, s.u) : s.special;
        const double recip = 1.0 / static_cast<double>(S);
        w.sel[row].total = S;
        // p_thr = e_thr / S, as k_smp_div divides (a NaN or +inf sum takes the radix path)
        if (w.sel[row].ethr_on && s.finite) {
            w.sel[row].fast_key = total_key(div_by_recip(from_key(w.sel[row].ethr_key), recip));
            w.sel[row].fast_on = 1u;
        }
        // The bucket path's bracket: p's keys of the digit's least e and of
        // the next digit's least e.  p is monotone in e, so the top_k-th
        // largest p lies in [blo, bhi] and fewer than top_k keys exceed bhi;
        // k_smp_rank relies on neither and checks the counts of its lists.
        const uint32_t d = s_edig;
        if (d != kNone && s.finite) {
            w.sel[row].blo = total_key(div_by_recip(from_key(d << 21), recip));
            w.sel[row].bhi = d + 1 < kBins ? total_key(div_by_recip(from_key((d + 1) << 21), recip)) : 0xffffffffu;
            w.sel[row].bon = 1u;
        }
    }
}

// ---- stage 4: p = e / S in place, first radix digit -------------------------

// Rows with a fast threshold (k_smp_sum) also list every key >= fast_key:
// buffered per workgroup in LDS, then placed with one atomic.  A workgroup
// with more than kFastWg of them pushes the row's count past kCap, and the
// row takes the radix path.
__global__ __launch_bounds__(kBlock) void k_smp_div(SmpGeo g, float *logits, SmpWs w)
{
    __shared__ uint32_t s_hist[kBins];
    __shared__ uint64_t s_fbuf[kFastWg];
    __shared__ uint32_t s_fcnt, s_fbase;
    const uint32_t row = blockIdx.x / g.chunks, chunk = blockIdx.x % g.chunks;
    float *x = logits + static_cast<int64_t>(row) * g.ld;
    const RowSel sel = w.sel[row];
    const bool fast = sel.fast_on != 0;
    if (!fast)
        for (uint32_t b = threadIdx.x; b < kBins; b += blockDim.x) s_hist[b] = 0;
    if (threadIdx.x == 0) s_fcnt = 0;
    __syncthreads();
    const uint32_t fkey = sel.fast_key;
    // S >= 1 (the maximal element contributes expf(0) = 1) or NaN: the
    // reciprocal form is the correctly rounded quotient (div_by_recip)
    const double recip = 1.0 / static_cast<double>(sel.total);
    uint64_t c0, c1;
    chunk_range(g, chunk, c0, c1);
    if (!fast) { // uniform
        visit<true, 4>(g, x, c0, c1, [&](float &v, uint64_t) {
            v = div_by_recip(v, recip);
            atomicAdd(&s_hist[total_key(v) >> 21], 1u);
        });
        flush_hist(s_hist, kBins, w.hist + static_cast<uint64_t>(row) * kBins);
        return;
    }
    // a fast row needs no histogram: should its list overflow, k_smp_resolve
    // scans the row for the first digit
    visit<true, 4>(g, x, c0, c1, [&](float &v, uint64_t col) {
        v = div_by_recip(v, recip);
        const uint32_t key = total_key(v);
        if (key >= fkey) {
            const uint32_t i = atomicAdd(&s_fcnt, 1u);
            if (i < kFastWg) s_fbuf[i] = cand_word(key, static_cast<uint32_t>(col));
        }
    });
    __syncthreads();
    const uint32_t n = s_fcnt;
    if (n == 0) return; // uniform
    if (threadIdx.x == 0) s_fbase = atomicAdd(&w.sel[row].fast_count, n <= kFastWg ? n : kCap + 1);
    __syncthreads();
    const uint32_t base = s_fbase;
    uint64_t *list = w.cand + static_cast<uint64_t>(row) * g.cand_ld;
    if (n <= kFastWg)
        for (uint32_t i = threadIdx.x; i < n; i += blockDim.x)
            if (base + i < kCap) list[base + i] = s_fbuf[i];
}

// The bucket path's division: p = e / S in place and the first-digit
// histogram, as k_smp_div, and the lists of the row's bracket: A (keys above
// bhi) into the candidate list, B (keys in [blo, bhi]) into the bucket list.
// Steps of kDivVec float4 per thread (5120 columns per workgroup: config 5's
// chunk in one step).  Per step each thread counts its A and B words, a wave
// prefix sum of the packed counts places them in the workgroup's LDS buffers
// (kListWg words each, one LDS atomic per wave and list); words past a
// buffer take a global atomic of their own.  At the end one 64-bit atomic
// (A low half, B high half) places the buffers.  The counts are exact, the
// lists complete up to their capacities.  Held to 8 waves per SIMD (64
// VGPRs, no spills): 7, the compiler's default, leaves config 5's 1920
// workgroups two rounds (22.5 against 20.2 us).
constexpr uint32_t kDivVec = 5;
constexpr uint32_t kListWg = 512;
__global__ __launch_bounds__(kBlock) __attribute__((amdgpu_waves_per_eu(8, 8))) void k_smp_divlist(SmpGeo g, float *logits, SmpWs w)
{
    __shared__ uint32_t s_hist[kBins];
    __shared__ uint64_t s_lbuf[2][kListWg];
    __shared__ uint32_t s_lcnt[2];
    __shared__ uint64_t s_lbase;
    const uint32_t row = blockIdx.x / g.chunks, chunk = blockIdx.x % g.chunks;
    const uint32_t lane = threadIdx.x % kWave;
    float *x = logits + static_cast<int64_t>(row) * g.ld;
    for (uint32_t b = threadIdx.x; b < kBins; b += blockDim.x) s_hist[b] = 0;
    if (threadIdx.x == 0) s_lcnt[0] = s_lcnt[1] = 0;
    const float total = w.sel[row].total;
    const bool lst = w.sel[row].bon != 0; // uniform; else no list (k_smp_rank scans the row)
    const uint32_t blo = w.sel[row].blo, bhi = w.sel[row].bhi;
    __syncthreads();
    const double recip = 1.0 / static_cast<double>(total); // as k_smp_div
    uint64_t *alist = w.cand + static_cast<uint64_t>(row) * g.cand_ld;
    uint64_t *blist = w.bucket + static_cast<uint64_t>(row) * kBucketCap;
    unsigned long long *fill = reinterpret_cast<unsigned long long *>(&w.sel[row].gfill);
    uint64_t c0, c1;
    chunk_range(g, chunk, c0, c1);
    const uint32_t e1 = static_cast<uint32_t>(c1); // card < 2^31
    for (uint64_t blk = c0; blk < c1; blk += 4ull * kDivVec * kBlock) {
        const uint32_t col0 = static_cast<uint32_t>(blk) + 4u * threadIdx.x; // float4 i at col0 + 4 kBlock i
        float4 q[kDivVec];
#pragma unroll
        for (uint32_t i = 0; i < kDivVec; ++i) {
            const uint32_t c = col0 + 4u * kBlock * i;
            if (g.vec && c + 4 <= e1) {
                q[i] = *reinterpret_cast<const float4 *>(x + c);
            } else {
                q[i].x = c < e1 ? x[c] : 0.0f;
                q[i].y = c + 1 < e1 ? x[c + 1] : 0.0f;
                q[i].z = c + 2 < e1 ? x[c + 2] : 0.0f;
                q[i].w = c + 3 < e1 ? x[c + 3] : 0.0f;
            }
        }
        uint32_t key[4 * kDivVec];
        uint32_t na = 0, nb = 0;
#pragma unroll
        for (uint32_t i = 0; i < kDivVec; ++i) {
            float *f = reinterpret_cast<float *>(&q[i]);
#pragma unroll
            for (uint32_t j = 0; j < 4; ++j) {
                const bool in = col0 + 4u * kBlock * i + j < e1;
                f[j] = div_by_recip(f[j], recip);
                const uint32_t k = total_key(f[j]);
                key[4 * i + j] = k;
                if (in) atomicAdd(&s_hist[k >> 21], 1u);
                na += (lst && in && k > bhi) ? 1u : 0u;
                nb += (lst && in && k >= blo && k <= bhi) ? 1u : 0u;
            }
            const uint32_t c = col0 + 4u * kBlock * i;
            if (g.vec && c + 4 <= e1) {
                *reinterpret_cast<float4 *>(x + c) = q[i];
            } else {
#pragma unroll
                for (uint32_t j = 0; j < 4; ++j)
                    if (c + j < e1) x[c + j] = f[j];
            }
        }
        // per wave: the A and B words of this step (at most 16 each per lane)
        const uint32_t incl = wave_incl_scan(na | (nb << 16));
        const uint32_t wtot = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(incl), kWave - 1));
        if (wtot == 0) continue; // uniform over the wave
        uint32_t ba = 0, bb = 0;
        if (lane == kWave - 1) {
            if (wtot & 0xffffu) ba = atomicAdd(&s_lcnt[0], wtot & 0xffffu);
            if (wtot >> 16) bb = atomicAdd(&s_lcnt[1], wtot >> 16);
        }
        uint32_t sa = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(ba), kWave - 1)) + (incl & 0xffffu) - na;
        uint32_t sb = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(bb), kWave - 1)) + (incl >> 16) - nb;
#pragma unroll
        for (uint32_t j = 0; j < 4 * kDivVec; ++j) {
            const uint32_t col = col0 + 4u * kBlock * (j / 4) + j % 4;
            const uint32_t k = key[j];
            const bool in = lst && col < e1;
            if (in && k > bhi) {
                if (sa < kListWg) {
                    s_lbuf[0][sa] = cand_word(k, col);
                } else { // past the buffer
                    const uint32_t at = static_cast<uint32_t>(atomicAdd(fill, 1ull));
                    if (at < g.cand_ld) alist[at] = cand_word(k, col);
                }
                ++sa;
            } else if (in && k >= blo) {
                if (sb < kListWg) {
                    s_lbuf[1][sb] = cand_word(k, col);
                } else {
                    const uint32_t at = static_cast<uint32_t>(atomicAdd(fill, 1ull << 32) >> 32);
                    if (at < kBucketCap) blist[at] = cand_word(k, col);
                }
                ++sb;
            }
        }
    }
    flush_hist(s_hist, kBins, w.hist + static_cast<uint64_t>(row) * kBins); // its barrier orders the buffers
    const uint32_t na = s_lcnt[0] < kListWg ? s_lcnt[0] : kListWg, nb = s_lcnt[1] < kListWg ? s_lcnt[1] : kListWg;
    if (na + nb == 0) return; // uniform
    if (threadIdx.x == 0)
        s_lbase = atomicAdd(fill, static_cast<unsigned long long>(na) | (static_cast<unsigned long long>(nb) << 32));
    __syncthreads();
    const uint32_t ba = static_cast<uint32_t>(s_lbase), bb = static_cast<uint32_t>(s_lbase >> 32);
    for (uint32_t i = threadIdx.x; i < na; i += blockDim.x)
        if (ba + i < g.cand_ld) alist[ba + i] = s_lbuf[0][i];
    for (uint32_t i = threadIdx.x; i < nb; i += blockDim.x)
        if (bb + i < kBucketCap) blist[bb + i] = s_lbuf[1][i];
}

// Inclusive prefix sum over a 256-thread workgroup (uses s_tmp[4]).
__device__ __forceinline__ uint32_t block_incl_scan256(uint32_t v, uint32_t *s_tmp, uint32_t &total)
{
    const uint32_t lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
#pragma unroll
    for (int off = 1; off < kWave; off <<= 1) {
        const uint32_t o = __shfl_up(v, off, kWave);
        if (lane >= static_cast<uint32_t>(off)) v += o;
    }
    if (lane == kWave - 1) s_tmp[wave] = v;
    __syncthreads();
    uint32_t before = 0;
    total = 0;
#pragma unroll
    for (uint32_t w = 0; w < kBlock / kWave; ++w) {
        before += w < wave ? s_tmp[w] : 0u;
        total += s_tmp[w];
    }
    return v + before;
}

// ---- stages 5-7: the threshold, one workgroup per row ----------------------
//
// Digits of the total-order key, 11, 11 and 10 bits from the top.  A pick
// finds the digit b holding the need-th largest key of the row's open
// prefix region -- greater(b) < need <= greater(b) + count(b), greater(b)
// counting the higher digits -- and extends the prefix by it.  The row is
// resolved as soon as every key at or above the prefix fits the kCap
// candidates one workgroup sorts (mode 1); at 32 bits the threshold key T
// is exact (mode 2) and the ties at T are counted per chunk, for the
// collect step to take the lowest-index ones.  The first digit's histogram
// comes from k_smp_div; the later ones (rows that need them) from scans of
// the row here, so rows resolved by the first digit cost one short launch.

constexpr uint32_t kResolveThreads = 1024;

// Inclusive prefix sum over a kResolveThreads workgroup (s_tmp: one word
// per wave).
__device__ __forceinline__ uint32_t block_incl_scan1024(uint32_t v, uint32_t *s_tmp, uint32_t &total)
{
    const uint32_t lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    v = wave_incl_scan(v);
    if (lane == kWave - 1) s_tmp[wave] = v;
    __syncthreads();
    uint32_t before = 0;
    total = 0;
#pragma unroll
    for (uint32_t w = 0; w < kResolveThreads / kWave; ++w) {
        const uint32_t x = s_tmp[w];
        before += w < wave ? x : 0u;
        total += x;
    }
    __syncthreads(); // s_tmp may be rewritten after this
    return v + before;
}

// The pick over hist[0, 2^bits), bins in increasing key order; returns the
// advanced selection (the same in every thread).
__device__ __forceinline__ RowSel pick_digit(const RowSel &sel, const uint32_t *hist, uint32_t bits, uint32_t *s_tmp,
                             uint32_t *s_pick)
{
    const uint32_t per = (1u << bits) / kResolveThreads; // 2 or 1 bins per thread
    uint32_t mine[kBins / kResolveThreads] = {};
    uint32_t local = 0;
    for (uint32_t i = 0; i < per; ++i) {
        mine[i] = hist[threadIdx.x * per + i];
        local += mine[i];
    }
    if (threadIdx.x == 0) s_pick[0] = s_pick[1] = s_pick[2] = 0;
    uint32_t total;
    const uint32_t incl = block_incl_scan1024(local, s_tmp, total); // its barriers order s_pick's reset
    uint32_t cum = total - incl; // elements in higher threads' (higher) digits
    for (int i = static_cast<int>(per) - 1; i >= 0; --i) {
        if (cum < sel.need && sel.need <= cum + mine[i]) {
            s_pick[0] = threadIdx.x * per + static_cast<uint32_t>(i);
            s_pick[1] = cum;
            s_pick[2] = mine[i];
        }
        cum += mine[i];
    }
    __syncthreads();
    RowSel n = sel;
    n.prefix = (sel.prefix << bits) | s_pick[0];
    n.depth = sel.depth + bits;
    n.above = sel.above + s_pick[1];
    n.need = sel.need - s_pick[1];
    if (n.above + s_pick[2] <= kCap) {
        n.mode = 1; // every key whose top `depth` bits are >= prefix
        n.count = n.above + s_pick[2];
    } else if (n.depth == 32) {
        n.mode = 2; // keys > T, then the lowest-index `need` keys == T
        n.count = n.above + n.need;
    }
    __syncthreads(); // s_pick is read by every thread before the next pick
    return n;
}

// The radix selection of one row (mode 0, not resolved by the fast list) by
// one 1024-thread workgroup: the first digit from k_smp_div's histogram (or
// from a scan, for a fast row whose list overflowed), later digits from
// scans of the row, and at an exact threshold the ties per chunk (w.ties).
// Returns the row's selection (mode 1 or 2).
__device__ RowSel resolve_row(const SmpGeo &g, float *logits, const SmpWs &w, uint32_t row, RowSel sel,
                              uint32_t *s_hist, uint32_t *s_tmp, uint32_t *s_pick)
{
    float *x = logits + static_cast<int64_t>(row) * g.ld;
    if (!sel.fast_on) {
        sel = pick_digit(sel, w.hist + static_cast<uint64_t>(row) * kBins, 11, s_tmp, s_pick);
    } else { // a fast row whose list overflowed: k_smp_div left no histogram
        for (uint32_t b = threadIdx.x; b < kBins; b += blockDim.x) s_hist[b] = 0;
        __syncthreads();
        visit<false>(g, x, 0, g.card, [&](float &v, uint64_t) { atomicAdd(&s_hist[total_key(v) >> 21], 1u); });
        __syncthreads();
        sel = pick_digit(sel, s_hist, 11, s_tmp, s_pick);
    }
    for (uint32_t pass = 1; pass <= 2 && sel.mode == 0; ++pass) {
        const uint32_t bits = pass == 2 ? 10u : 11u;
        const uint32_t nbins = 1u << bits;
        const uint32_t dshift = 32u - sel.depth; // depth is 11 or 22 here
        const uint32_t shift = dshift - bits;
        const uint32_t prefix = sel.prefix;
        for (uint32_t b = threadIdx.x; b < nbins; b += blockDim.x) s_hist[b] = 0;
        __syncthreads();
        visit<false>(g, x, 0, g.card, [&](float &v, uint64_t) {
            const uint32_t key = total_key(v);
            if ((key >> dshift) == prefix) atomicAdd(&s_hist[(key >> shift) & (nbins - 1)], 1u);
        });
        __syncthreads();
        sel = pick_digit(sel, s_hist, bits, s_tmp, s_pick);
    }
    if (sel.mode == 2) {
        // chunks <= kBins (launch_sampler checks it)
        for (uint32_t c = threadIdx.x; c < g.chunks; c += blockDim.x) s_hist[c] = 0;
        __syncthreads();
        const uint32_t t_key = sel.prefix;
        const uint32_t cc = static_cast<uint32_t>(g.chunk_cols);
        visit<false>(g, x, 0, g.card, [&](float &v, uint64_t col) {
            if (total_key(v) == t_key) atomicAdd(&s_hist[static_cast<uint32_t>(col) / cc], 1u);
        });
        __syncthreads();
        for (uint32_t c = threadIdx.x; c < g.chunks; c += blockDim.x)
            w.ties[static_cast<uint64_t>(row) * g.chunks + c] = s_hist[c];
    }
    return sel;
}

// Rows of a top_k above kCap (the merge path): k_smp_resolve, k_smp_collect
// and the merge kernels.
__global__ __launch_bounds__(kResolveThreads) void k_smp_resolve(SmpGeo g, float *logits, SmpWs w)
{
    __shared__ uint32_t s_hist[kBins]; // digit histogram; later the per-chunk tie counts
    __shared__ uint32_t s_tmp[kResolveThreads / kWave];
    __shared__ uint32_t s_pick[3];
    const uint32_t row = blockIdx.x;
    const RowSel sel = w.sel[row];
    if (sel.mode != 0) return; // uniform
    if (sel.fast_on && sel.fast_count <= kCap) { // uniform: k_smp_div listed the candidates
        if (threadIdx.x == 0) {
            w.sel[row].count = sel.fast_count; // >= top_k: the maxima behind the threshold
            w.sel[row].mode = 3;
        }
        return;
    }
    const RowSel r = resolve_row(g, logits, w, row, sel, s_hist, s_tmp, s_pick);
    if (threadIdx.x == 0) w.sel[row] = r; // for k_smp_collect
}

// ---- stage 8: candidates ------------------------------------------------------
//
// Steps of 4 consecutive columns per thread (1024 per workgroup): each step
// counts its candidates, one workgroup prefix sum places them, and one atomic
// per step that has any reserves their slots in the row's list.  The order
// of the list is irrelevant (it is sorted next); the count is exact.

__global__ __launch_bounds__(kBlock) void k_smp_collect(SmpGeo g, float *logits, SmpWs w)
{
    __shared__ uint32_t s_tmp[2][kBlock / kWave];
    __shared__ uint32_t s_base;
    const uint32_t row = blockIdx.x / g.chunks, chunk = blockIdx.x % g.chunks;
    const RowSel sel = w.sel[row];
    if (sel.mode == 3) return; // uniform: listed by k_smp_div
    float *x = logits + static_cast<int64_t>(row) * g.ld;
    uint64_t *list = w.cand + static_cast<uint64_t>(row) * g.cand_ld;
    uint64_t c0, c1;
    chunk_range(g, chunk, c0, c1);
    const bool exact = sel.mode == 2;
    const uint32_t T = sel.prefix;
    const uint32_t dshift = 32u - sel.depth;
    // mode 2: ties at T in the chunks before this one
    uint32_t tie_base = 0;
    if (exact) {
        uint32_t mine = 0;
        for (uint32_t c = threadIdx.x; c < chunk; c += blockDim.x) mine += w.ties[static_cast<uint64_t>(row) * g.chunks + c];
        (void)block_incl_scan256(mine, s_tmp[0], tie_base);
        __syncthreads();
    }
    uint32_t par = 1;
    for (uint64_t blk = c0; blk < c1; blk += 4 * kBlock) {
        const uint64_t col0 = blk + 4 * static_cast<uint64_t>(threadIdx.x);
        uint32_t key[4];
        bool in[4];
        if (g.vec && col0 + 4 <= c1) {
            const float4 q = *reinterpret_cast<const float4 *>(x + col0);
            key[0] = total_key(q.x);
            key[1] = total_key(q.y);
            key[2] = total_key(q.z);
            key[3] = total_key(q.w);
#pragma unroll
            for (int j = 0; j < 4; ++j) in[j] = true;
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                in[j] = col0 + j < c1;
                key[j] = in[j] ? total_key(x[col0 + j]) : 0u;
            }
        }
        bool take[4];
        if (!exact) {
#pragma unroll
            for (int j = 0; j < 4; ++j) take[j] = in[j] && (key[j] >> dshift) >= T;
        } else {
            // ties at T are taken in column order while fewer than `need` precede them
            uint32_t nt = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) nt += (in[j] && key[j] == T) ? 1u : 0u;
            uint32_t step_ties;
            const uint32_t incl = block_incl_scan256(nt, s_tmp[par], step_ties);
            par ^= 1u;
            uint32_t rank = tie_base + incl - nt;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const bool tie = in[j] && key[j] == T;
                take[j] = (in[j] && key[j] > T) || (tie && rank < sel.need);
                rank += tie ? 1u : 0u;
            }
            tie_base += step_ties;
        }
        uint32_t nc = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) nc += take[j] ? 1u : 0u;
        uint32_t step_total;
        const uint32_t cincl = block_incl_scan256(nc, s_tmp[par], step_total);
        par ^= 1u;
        if (step_total == 0) continue; // uniform
        if (threadIdx.x == 0) s_base = atomicAdd(&w.sel[row].written, step_total);
        __syncthreads();
        uint32_t slot = s_base + cincl - nc;
        __syncthreads(); // s_base is rewritten by the next step
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            // the selection counted exactly `count` <= cand_ld candidates; the
            // bound only keeps a miscount from writing outside the row's list
            if (take[j] && slot < g.cand_ld) list[slot] = cand_word(key[j], static_cast<uint32_t>(col0 + j));
            slot += take[j] ? 1u : 0u;
        }
    }
}


// ---- stage 9: ranking and selection -----------------------------------------

struct SmpOut {
    int32_t *sorted;
    float *top_p;
    int32_t *top_i;
    int64_t sorted_ld, top_ld;
    int32_t *selected;
    float *score;
    int32_t *status; // may be null
};

constexpr uint32_t kStatesInline = 512;
struct SmpStates {
    uint32_t v[kStatesInline]; // start states of rows [row0, row0 + kStatesInline)
};

// Synchronises the T threads that run a ranking step: the whole workgroup
// (T == kRankThreads), or wave 0 alone (T == kWave; the other waves have
// left), whose LDS writes a fence and a wave barrier order.
template <uint32_t T>
__device__ __forceinline__ void group_sync()
{
    if constexpr (T == kWave) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    } else {
        __syncthreads();
    }
}

// Race selection over the ranked slots j < top_k (sampler/sm.rs:821-847):
// slot j draws state_j = s0 * 16807^(j+1) mod (2^31 - 1), u_j = state_j as
// f32 / 2^31 (2147483647 as f32 is 2^31), race_j = p_j / -ln(u_j); the
// first slot with the greatest race (strict >, starting from -inf) wins.
//
// The race word of a slot orders slots as that rule does: total_key(race)
// above ~slot, so the greatest word holds the greatest race and, among equal
// races, the first slot.  Races are >= +0 (p >= +0 over -ln(u) >= 0) when
// they are not -inf or NaN, so the key order is the float order; 0 stands
// for no slot.
__device__ __forceinline__ uint64_t race_word(float race, uint32_t slot)
{
    return (static_cast<uint64_t>(total_key(race)) << 32) | static_cast<uint32_t>(~slot);
}

// The greatest race word over slots slot0 + j, j < n, whose draws start from
// s0j = s0 16807^slot0 (slot0 + j draws s0j 16807^(j+1)); prob(j) is the
// probability of slot slot0 + j.  T threads take part (see group_sync); the
// result is thread 0's.
// logf's table in LDS, read per lane (staged by threads 0-15; the caller
// synchronises before use).
struct LogfTab {
    double invc[16], logc[16];
};
__device__ __forceinline__ void stage_logf(LogfTab *t)
{
    if (threadIdx.x < 16) {
        t->invc[threadIdx.x] = kLogfInvc[threadIdx.x];
        t->logc[threadIdx.x] = kLogfLogc[threadIdx.x];
    }
}

template <uint32_t T, class P>
__device__ uint64_t race_best(uint32_t n, uint32_t s0j, uint32_t slot0, P prob, const LogfTab *tab, uint32_t pw)
{
    __shared__ uint64_t s_w[kRankThreads / kWave];
    const double *s_invc = tab->invc, *s_logc = tab->logc;
    uint64_t best = 0;
    // pw = 16807^(t+1) (kPmPowers.v[t]); slot t + m T multiplies by (16807^T)^m
    for (uint32_t j = threadIdx.x; j < n; j += T) {
        const uint32_t state = mulmod(s0j, pw);
        const float uniform = static_cast<float>(state) * 0x1p-31f;
        const float race = prob(j) / -emel_logf(uniform, s_invc, s_logc);
        const uint64_t wd = race > -__builtin_inff() ? race_word(race, slot0 + j) : 0ull;
        best = wd > best ? wd : best;
        pw = mulmod(pw, kPmPowers.v[T - 1]);
    }
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) {
        const uint64_t ob = static_cast<uint64_t>(__shfl_xor(static_cast<unsigned long long>(best), off, kWave));
        best = ob > best ? ob : best;
    }
    if constexpr (T > kWave) {
        if (threadIdx.x % kWave == 0) s_w[threadIdx.x / kWave] = best;
        __syncthreads();
        if (threadIdx.x == 0)
            for (uint32_t v = 1; v < T / kWave; ++v) best = s_w[v] > best ? s_w[v] : best;
    }
    return best;
}

// The row's outputs from the winning race word (0: no slot); index(j) is
// the token of ranked slot j.
template <class I>
__device__ __forceinline__ void write_selection(const SmpGeo &g, const SmpOut &o, uint32_t row, uint64_t best, I index)
{
    const int32_t selected = best ? index(~static_cast<uint32_t>(best)) : -1;
    const float score = best ? from_key(static_cast<uint32_t>(best >> 32)) : -__builtin_inff();
    o.selected[row] = selected;
    o.score[row] = score;
    const bool valid = selected >= 0 && static_cast<uint64_t>(selected) < g.card && __builtin_isfinite(score);
    if (o.status) o.status[row] = valid ? 0 : kInvalidRequest;
}

// The race over slots j < top_k, decided in one workgroup.
template <uint32_t T, class P, class I>
__device__ void select_slots(const SmpGeo &g, uint32_t row, uint32_t s0, P prob, I index, const SmpOut &o)
{
    __shared__ LogfTab s_tab;
    const uint32_t pw = kPmPowers.v[threadIdx.x];
    stage_logf(&s_tab);
    group_sync<T>();
    const uint64_t best = race_best<T>(g.top_k, s0, 0, prob, &s_tab, pw);
    if (threadIdx.x == 0) write_selection(g, o, row, best, index);
}

__device__ __forceinline__ void write_ranked(const SmpGeo &g, const SmpOut &o, uint32_t row, uint32_t j, uint64_t word)
{
    const uint32_t idx = ~static_cast<uint32_t>(word);
    const float p = from_key(static_cast<uint32_t>(word >> 32));
    o.top_p[static_cast<int64_t>(row) * o.top_ld + j] = p;
    o.top_i[static_cast<int64_t>(row) * o.top_ld + j] = static_cast<int32_t>(idx);
    o.sorted[static_cast<int64_t>(row) * o.sorted_ld + j] = static_cast<int32_t>(idx);
}

// Sort, descending, of the elements [0, n) held in s at slot(e), for n a
// power of two with kSortPer <= n <= kSortPer * blockDim.x.  Thread t sorts
// the run [t kSortPer, (t + 1) kSortPer) in registers (a bitonic network), then
// sorted runs of length L merge pairwise into runs of 2 L, log2(n /
// kSortPer) rounds: thread t produces kSortPer consecutive outputs of its
// pair's merged run, finds where they start in the two runs with a
// merge-path binary search, merges them in registers, and writes them back
// once every thread has read.  Words are distinct except the zero padding,
// whose copies are interchangeable; an exhausted run reads as 0.
constexpr uint32_t kSortPer = 8;
static_assert(kCap == kSortPer * kRankThreads, "one workgroup sorts kCap words");

// LDS slot of sort element e: one pad word after every 32 (256 bytes), so
// that lanes touching elements 8 or 4 apart (each lane's run, the merge
// fronts) spread over the banks instead of sharing a few.
__device__ __forceinline__ uint32_t slot(uint32_t e) { return e + (e >> 5); }
constexpr uint32_t kCapSlots = kCap + kCap / 32;

__device__ __forceinline__ void sort_regs_desc(uint64_t (&v)[kSortPer])
{
#pragma unroll
    for (uint32_t size = 2; size <= kSortPer; size <<= 1) {
#pragma unroll
        for (uint32_t stride = size >> 1; stride > 0; stride >>= 1) {
#pragma unroll
            for (uint32_t i = 0; i < kSortPer; ++i) {
                const uint32_t j = i ^ stride;
                if (j > i) {
                    const bool swap = (v[i] < v[j]) == ((i & size) == 0);
                    const uint64_t a = v[i], b = v[j];
                    v[i] = swap ? b : a;
                    v[j] = swap ? a : b;
                }
            }
        }
    }
}

template <uint32_t T>
__device__ void lds_sort_desc(uint64_t *s, uint32_t n)
{
    const uint32_t t = threadIdx.x;
    const bool act = t * kSortPer < n;
    uint64_t v[kSortPer];
    if (act) {
#pragma unroll
        for (uint32_t r = 0; r < kSortPer; ++r) v[r] = s[slot(t * kSortPer + r)];
        sort_regs_desc(v);
    }
    for (uint32_t len = kSortPer; len < n; len <<= 1) {
        if (act) {
#pragma unroll
            for (uint32_t r = 0; r < kSortPer; ++r) s[slot(t * kSortPer + r)] = v[r];
        }
        group_sync<T>();
        if (act) {
            const uint32_t per_pair = 2 * len / kSortPer; // threads per merged run
            const uint32_t a0 = (t / per_pair) * 2 * len, b0 = a0 + len; // the two runs
            const uint32_t d = (t % per_pair) * kSortPer; // outputs before this thread's
            // i = how many of the first d outputs come from run A
            uint32_t lo = d > len ? d - len : 0, hi = d < len ? d : len;
            while (lo < hi) {
                const uint32_t mid = (lo + hi) >> 1;
                if (s[slot(a0 + mid)] > s[slot(b0 + d - 1 - mid)]) lo = mid + 1;
                else hi = mid;
            }
            uint32_t i = lo, j = d - lo;
            uint64_t a = s[slot(a0 + (i < len ? i : len - 1))], b = s[slot(b0 + (j < len ? j : len - 1))];
            a = i < len ? a : 0ull;
            b = j < len ? b : 0ull;
#pragma unroll
            for (uint32_t r = 0; r < kSortPer; ++r) {
                const bool take_a = a > b;
                v[r] = take_a ? a : b;
                i += take_a ? 1u : 0u;
                j += take_a ? 0u : 1u;
                const uint64_t na = s[slot(a0 + (i < len ? i : len - 1))];
                const uint64_t nb = s[slot(b0 + (j < len ? j : len - 1))];
                a = i < len ? na : 0ull;
                b = j < len ? nb : 0ull;
            }
        }
        group_sync<T>(); // every read of this round precedes the next writes
    }
    if (act) {
#pragma unroll
        for (uint32_t r = 0; r < kSortPer; ++r) s[slot(t * kSortPer + r)] = v[r];
    }
    group_sync<T>();
}

// Stages the words c[0, n) into sort elements [0, np) of s (np <= kCap,
// zeros after n), all of a thread's kSortPer global loads issued before its
// first LDS store.
template <uint32_t T>
__device__ __forceinline__ void stage_words(uint64_t *s, const uint64_t *c, uint32_t n, uint32_t np)
{
    uint64_t q[kSortPer];
#pragma unroll
    for (uint32_t r = 0; r < kSortPer; ++r) {
        const uint32_t i = threadIdx.x + r * T;
        q[r] = i < n ? c[i] : 0ull; // short lists (the fast path's) load only their words
    }
#pragma unroll
    for (uint32_t r = 0; r < kSortPer; ++r) {
        const uint32_t i = threadIdx.x + r * T;
        if (i < np) s[slot(i)] = i < n ? q[r] : 0ull;
    }
    group_sync<T>();
}

// Candidate lists of at most kCap: one workgroup sorts a row in LDS.
// The ranking of one row's candidate list (count words in w.cand) by one
// 1024-thread workgroup: the LDS sort, the ranked outputs and the race
// (random state s0).
__device__ void rank_row(const SmpGeo &g, const SmpWs &w, const SmpOut &o, uint32_t s0, uint32_t row, uint32_t count,
                         uint64_t *s_c)
{
    const uint32_t n = count < kCap ? count : kCap; // top_k <= count <= kCap here
    uint32_t np = kSortPer;
    while (np < n || np < g.top_k) np <<= 1;
    const uint64_t *list = w.cand + static_cast<uint64_t>(row) * g.cand_ld;
    if (np <= kWave * kSortPer && g.top_k <= kWave) { // uniform: a short list (the fast path's) by wave 0 alone
        if (threadIdx.x >= kWave) return;
        stage_words<kWave>(s_c, list, n, np);
        lds_sort_desc<kWave>(s_c, np);
        if (threadIdx.x < g.top_k) write_ranked(g, o, row, threadIdx.x, s_c[slot(threadIdx.x)]);
        select_slots<kWave>(
            g, row, s0, [&](uint32_t j) { return from_key(static_cast<uint32_t>(s_c[slot(j)] >> 32)); },
            [&](uint32_t j) { return static_cast<int32_t>(~static_cast<uint32_t>(s_c[slot(j)])); }, o);
        return;
    }
    stage_words<kRankThreads>(s_c, list, n, np);
    lds_sort_desc<kRankThreads>(s_c, np);
    for (uint32_t j = threadIdx.x; j < g.top_k; j += blockDim.x) write_ranked(g, o, row, j, s_c[slot(j)]);
    select_slots<kRankThreads>(
        g, row, s0, [&](uint32_t j) { return from_key(static_cast<uint32_t>(s_c[slot(j)] >> 32)); },
        [&](uint32_t j) { return static_cast<int32_t>(~static_cast<uint32_t>(s_c[slot(j)])); }, o);
}

// The candidate list of one row (mode 1 or 2) by one 1024-thread workgroup,
// in column order: the selection of k_smp_collect, the ties at T taken while
// fewer than `need` precede them.  Each thread takes 16 consecutive columns
// per step (their four float4 loads in flight together); one workgroup
// prefix sum per step places the candidates (and one more counts the ties).
constexpr uint32_t kTailPer = 16;
__device__ void collect_row(const SmpGeo &g, const float *x, uint64_t *list, const RowSel &sel, uint32_t *s_tmp)
{
    const bool exact = sel.mode == 2;
    const uint32_t T = sel.prefix;
    const uint32_t dshift = 32u - sel.depth;
    uint32_t written = 0, ties = 0;
    for (uint64_t blk = 0; blk < g.card; blk += kTailPer * kRankThreads) {
        const uint64_t col0 = blk + kTailPer * static_cast<uint64_t>(threadIdx.x);
        uint32_t key[kTailPer];
        bool in[kTailPer];
        if (g.vec && col0 + kTailPer <= g.card) {
            float4 q[kTailPer / 4];
#pragma unroll
            for (uint32_t j = 0; j < kTailPer / 4; ++j) q[j] = *reinterpret_cast<const float4 *>(x + col0 + 4 * j);
#pragma unroll
            for (uint32_t j = 0; j < kTailPer / 4; ++j) {
                key[4 * j] = total_key(q[j].x);
                key[4 * j + 1] = total_key(q[j].y);
                key[4 * j + 2] = total_key(q[j].z);
                key[4 * j + 3] = total_key(q[j].w);
            }
#pragma unroll
            for (uint32_t j = 0; j < kTailPer; ++j) in[j] = true;
        } else {
#pragma unroll
            for (uint32_t j = 0; j < kTailPer; ++j) {
                in[j] = col0 + j < g.card;
                key[j] = in[j] ? total_key(x[col0 + j]) : 0u;
            }
        }
        bool take[kTailPer];
        if (!exact) {
#pragma unroll
            for (uint32_t j = 0; j < kTailPer; ++j) take[j] = in[j] && (key[j] >> dshift) >= T;
        } else {
            uint32_t nt = 0;
#pragma unroll
            for (uint32_t j = 0; j < kTailPer; ++j) nt += (in[j] && key[j] == T) ? 1u : 0u;
            uint32_t step_ties;
            const uint32_t incl = block_incl_scan1024(nt, s_tmp, step_ties);
            uint32_t rank = ties + incl - nt;
#pragma unroll
            for (uint32_t j = 0; j < kTailPer; ++j) {
                const bool tie = in[j] && key[j] == T;
                take[j] = (in[j] && key[j] > T) || (tie && rank < sel.need);
                rank += tie ? 1u : 0u;
            }
            ties += step_ties;
        }
        uint32_t nc = 0;
#pragma unroll
        for (uint32_t j = 0; j < kTailPer; ++j) nc += take[j] ? 1u : 0u;
        uint32_t step_total;
        const uint32_t cincl = block_incl_scan1024(nc, s_tmp, step_total);
        uint32_t slot = written + cincl - nc;
#pragma unroll
        for (uint32_t j = 0; j < kTailPer; ++j) {
            // the selection counts exactly `count` <= cand_ld candidates; the
            // bound only keeps a miscount from writing outside the row's list
            if (take[j] && slot < g.cand_ld) list[slot] = cand_word(key[j], static_cast<uint32_t>(col0 + j));
            slot += take[j] ? 1u : 0u;
        }
        written += step_total;
    }
}

// The bucket path's ranking: `groups` workgroups per row.  Groups q <
// groups - 1 take A's first digits (those >= the digit d of bhi: above it
// every key is in A, at d some), digit b to group floor((cb(b) + a(b) / 2)
// (groups - 1) / |A|), cb(b) the keys of the higher digits (the division's
// histogram) and a(b) the digit's A keys: a group holds whole digits of A, at
// most |A| < kCap keys, and its slots start at the least cb of its digits.  The last group takes B from the bucket list,
// cut by digits of B's own histograms (pick_digit from the top) while it is
// longer than the top_k - |A| words it needs plus kSortDirect, and ranks
// those words after A.  A row whose lists do not select, or whose ties at an
// exact threshold exceed kCap, is selected by the last group alone from
// scans of the row (resolve_row, collect_row, in the bucket list's place)
// and ranked whole, the A groups leaving at once.  Every workgroup races its
// own slots; the last one of the row to finish (a count per row) writes the
// selection from the greatest race word.
constexpr uint32_t kSortDirect = 1024;

// Sort, descending, of the n <= kCap distinct words of s (at slot(e)) by
// fine key bins, for one kRankThreads workgroup: the bin of a word is
// (kmax - key) >> sh, sh the least shift that maps the words' key range onto
// kFineBins bins, so bins run in descending key order.  An LDS atomic per
// word counts its bin and returns the word's place among the bin's; a
// prefix sum of the counts gives each bin's first position; the words are
// scattered by bin into d; and a word's final position is its bin's first
// plus the number of greater words in its bin.  Returns false, s untouched,
// when a bin holds more than kFineMax words (many equal keys, or a key range
// dense at this resolution): the merge sort takes those.
constexpr uint32_t kFineBins = 4096, kFineMax = 64;
static_assert(kFineBins == 4 * kRankThreads, "four fine bins per thread");
__device__ __forceinline__ uint32_t block_reduce1024(uint32_t v, bool take_max, uint32_t *s_red)
{
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) {
        const uint32_t o = __shfl_xor(v, off, kWave);
        v = take_max ? (o > v ? o : v) : (o < v ? o : v);
    }
    if (threadIdx.x % kWave == 0) s_red[threadIdx.x / kWave] = v;
    __syncthreads();
    v = s_red[0];
#pragma unroll
    for (uint32_t w = 1; w < kRankThreads / kWave; ++w) {
        const uint32_t o = s_red[w];
        v = take_max ? (o > v ? o : v) : (o < v ? o : v);
    }
    __syncthreads(); // s_red may be rewritten after this
    return v;
}

__device__ bool bin_sort_desc(uint64_t *s, uint32_t n, uint64_t *d, uint32_t *cnt, uint32_t *s_tmp)
{
    constexpr uint32_t T = kRankThreads;
    // per word of this thread only a packed (bin, place) is kept across the
    // barriers; the words are read again from LDS where needed
    uint32_t kmin = 0xffffffffu, kmax = 0;
#pragma unroll
    for (uint32_t r = 0; r < kSortPer; ++r) {
        const uint32_t e = threadIdx.x + r * T;
        if (e < n) {
            const uint32_t k = static_cast<uint32_t>(s[slot(e)] >> 32);
            kmin = k < kmin ? k : kmin;
            kmax = k > kmax ? k : kmax;
        }
    }
    reinterpret_cast<uint4 *>(cnt)[threadIdx.x] = uint4{0u, 0u, 0u, 0u};
    kmin = block_reduce1024(kmin, false, s_tmp); // its barriers order the zeroing
    kmax = block_reduce1024(kmax, true, s_tmp);
    uint32_t sh = 0;
    while (((kmax - kmin) >> sh) >= kFineBins) ++sh;
    uint32_t pk[kSortPer]; // bin | place in the bin << 12
#pragma unroll
    for (uint32_t r = 0; r < kSortPer; ++r) {
        const uint32_t e = threadIdx.x + r * T;
        pk[r] = kNone;
        if (e < n) {
            const uint32_t b = (kmax - static_cast<uint32_t>(s[slot(e)] >> 32)) >> sh;
            pk[r] = b | (atomicAdd(&cnt[b], 1u) << 12);
        }
    }
    __syncthreads();
    const uint4 c = reinterpret_cast<const uint4 *>(cnt)[threadIdx.x];
    uint32_t big = c.x > c.y ? c.x : c.y;
    big = c.z > big ? c.z : big;
    big = c.w > big ? c.w : big;
    if (block_reduce1024(big, true, s_tmp) > kFineMax) return false; // uniform
    const uint32_t mine = c.x + c.y + c.z + c.w;
    uint32_t total;
    const uint32_t first = block_incl_scan1024(mine, s_tmp, total) - mine;
    reinterpret_cast<uint4 *>(cnt)[threadIdx.x] = uint4{first, first + c.x, first + c.x + c.y, first + c.x + c.y + c.z};
    __syncthreads();
#pragma unroll
    for (uint32_t r = 0; r < kSortPer; ++r) {
        if (pk[r] == kNone) continue;
        const uint32_t b = pk[r] & (kFineBins - 1), at = cnt[b] + (pk[r] >> 12); // < n
        d[at] = s[slot(threadIdx.x + r * T)];
        pk[r] = b | (at << 12);
    }
    __syncthreads();
#pragma unroll
    for (uint32_t r = 0; r < kSortPer; ++r) {
        if (pk[r] == kNone) continue;
        const uint32_t b = pk[r] & (kFineBins - 1);
        const uint32_t b0 = cnt[b], b1 = b + 1 < kFineBins ? cnt[b + 1] : n; // at most kFineMax words
        const uint64_t word = d[pk[r] >> 12];
        uint32_t above = 0;
        for (uint32_t i = b0; i < b1; ++i) above += d[i] > word ? 1u : 0u;
        s[slot(b0 + above)] = word;
    }
    __syncthreads();
    return true;
}

// Sorts the n words of s_c (by fine bins when the workgroup ranks and they
// allow, else by merges), ranks the first `out` at slots slot0 + j and
// returns their greatest race word (thread 0's).
template <uint32_t T>
__device__ uint64_t rank_words(const SmpGeo &g, const SmpOut &o, uint32_t row, uint32_t s0, uint64_t *s_c, uint32_t n,
                               uint32_t out, uint32_t slot0, uint64_t *s_d, uint32_t *s_cnt, uint32_t *s_tmp,
                               const LogfTab *tab, uint32_t pw)
{
    if (T == kWave || !bin_sort_desc(s_c, n, s_d, s_cnt, s_tmp)) {
        uint32_t np = kSortPer;
        while (np < n) np <<= 1;
        for (uint32_t i = n + threadIdx.x; i < np; i += T) s_c[slot(i)] = 0ull;
        group_sync<T>();
        lds_sort_desc<T>(s_c, np);
    }
    for (uint32_t j = threadIdx.x; j < out; j += T) write_ranked(g, o, row, slot0 + j, s_c[slot(j)]);
    return race_best<T>(
        out, mulmod(s0, pm_power(slot0)), slot0,
        [&](uint32_t j) { return from_key(static_cast<uint32_t>(s_c[slot(j)] >> 32)); }, tab, pw);
}

// A workgroup's end (thread 0, holding `best`, the greatest race word of
// the slots from slot0 ranked in s_c): its word and the token of that slot
// go to the row's entry q, released by the count of finished workgroups;
// the last workgroup of the row acquires the entries and writes the
// selection from the greatest word.  Only thread 0 publishes, so one
// device-scope release per workgroup (an L2 write-back) suffices.
__device__ void group_finish(const SmpGeo &g, const SmpOut &o, const SmpWs &w, uint32_t row, uint32_t q,
                             uint64_t best, const uint64_t *s_c, uint32_t slot0, uint32_t groups)
{
    if (threadIdx.x != 0) return;
    GroupBest *gb = w.gbest + static_cast<uint64_t>(row) * kMaxGroups;
    const uint64_t idx = best ? ~static_cast<uint32_t>(s_c[slot(~static_cast<uint32_t>(best) - slot0)]) : 0u;
    __hip_atomic_store(&gb[q].word, best, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&gb[q].idx, idx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (__hip_atomic_fetch_add(&w.sel[row].gdone, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT) != groups - 1) return;
    uint64_t b = 0, bi = 0;
    for (uint32_t k = 0; k < groups; ++k) {
        const uint64_t wk = __hip_atomic_load(&gb[k].word, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (wk > b) {
            b = wk;
            bi = __hip_atomic_load(&gb[k].idx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
    write_selection(g, o, row, b, [&](uint32_t) { return static_cast<int32_t>(bi); });
}

// Appends v to s (at slot(*s_n + k)) for the lanes where take holds, one LDS
// atomic per wave; every lane of the wave calls it.
__device__ __forceinline__ void wave_append(bool take, uint64_t v, uint32_t *s_n, uint64_t *s)
{
    const uint64_t m = __ballot(take);
    if (m == 0) return; // uniform over the wave
    const uint32_t lane = threadIdx.x % kWave, leader = static_cast<uint32_t>(__builtin_ctzll(m));
    uint32_t base = 0;
    if (lane == leader) base = atomicAdd(s_n, static_cast<uint32_t>(__builtin_popcountll(m)));
    base = __shfl(base, static_cast<int>(leader), kWave);
    const uint32_t e = base + static_cast<uint32_t>(__builtin_popcountll(m & ((1ull << lane) - 1)));
    if (take && e < kCap) s[slot(e)] = v;
}

// Ranks the n <= kCap words staged in s_c, on wave 0 alone when they are few.
__device__ __forceinline__ void rank_group(const SmpGeo &g, const SmpOut &o, const SmpWs &w, uint32_t row, uint32_t q,
                                           uint32_t s0,
                           uint64_t *s_c, uint32_t n, uint32_t out, uint32_t slot0, uint32_t groups, uint64_t *s_d,
                           uint32_t *s_cnt, uint32_t *s_tmp, const LogfTab *tab, uint32_t pw)
{
    if (n <= kWave * kSortPer) { // uniform
        if (threadIdx.x >= kWave) return;
        const uint64_t best = rank_words<kWave>(g, o, row, s0, s_c, n, out, slot0, s_d, s_cnt, s_tmp, tab, pw);
        group_finish(g, o, w, row, q, best, s_c, slot0, groups);
        return;
    }
    const uint64_t best = rank_words<kRankThreads>(g, o, row, s0, s_c, n, out, slot0, s_d, s_cnt, s_tmp, tab, pw);
    group_finish(g, o, w, row, q, best, s_c, slot0, groups);
}

static_assert(kBins == 2 * kRankThreads, "two first digits per thread");
__global__ __launch_bounds__(kRankThreads) void k_smp_rank(SmpGeo g, float *logits, SmpWs w, SmpOut o, SmpStates st,
                                                           uint32_t row0, uint32_t groups)
{
    __shared__ uint64_t s_c[kCapSlots];
    __shared__ uint64_t s_d[kCap];          // bin_sort_desc's scatter
    __shared__ uint32_t s_hist[kFineBins];  // A: the group of each first digit; B: digit histograms; fine bins
    __shared__ uint32_t s_tmp[kRankThreads / kWave];
    __shared__ uint32_t s_pick[3];
    __shared__ uint32_t s_off, s_n;
    __shared__ LogfTab s_tab;
    stage_logf(&s_tab); // ordered by the barriers before the race
    const uint32_t pw = kPmPowers.v[threadIdx.x];
    const uint32_t r = blockIdx.x / groups, q = blockIdx.x % groups, ga = groups - 1;
    const uint32_t row = row0 + r, s0 = st.v[r];
    const uint32_t b0 = 2 * threadIdx.x, b1 = b0 + 1;
    const uint2 h = reinterpret_cast<const uint2 *>(w.hist + static_cast<uint64_t>(row) * kBins)[threadIdx.x];
    if (threadIdx.x == 0) {
        s_off = kNone;
        s_n = 0;
        s_pick[0] = kNone;
    }
    const uint32_t bon = w.sel[row].bon, bhi = w.sel[row].bhi;
    const uint64_t gfill = w.sel[row].gfill;
    uint32_t n = 0, out = 0, slot0 = 0; // the words staged in s_c, how many to rank, from which slot
    uint32_t total;
    const uint32_t incl = block_incl_scan1024(h.x + h.y, s_tmp, total); // its barriers order the resets
    const uint32_t cb1 = total - incl, cb0 = cb1 + h.y; // keys in the digits above b1, above b0
    // k_smp_div's lists hold every key above bhi (A) and in [blo, bhi] (B);
    // they select exactly when |A| < top_k <= |A| + |B| and B fits its list
    const uint32_t above = static_cast<uint32_t>(gfill), inb = static_cast<uint32_t>(gfill >> 32);
    const bool listed = bon && above < g.top_k && g.top_k - above <= inb && inb <= kBucketCap; // uniform
    if (q < ga) { // A
        if (!listed) { // uniform: the last group selects from scans
            group_finish(g, o, w, row, q, 0ull, s_c, 0, groups);
            return;
        }
        // digits above bhi's hold A keys only; bhi's digit d may hold some.  A
        // digit goes to the group of its A keys' middle (cb plus half of them),
        // which stays monotone in the digit and balances the groups better
        // than the digit's start
        // (shifted by |A| / (6 ga): the top group spans the widest key range,
        // whose fine bins are the densest, so it takes a smaller share)
        const uint32_t d = bhi >> 21;
        auto group_of = [&](uint32_t b, uint32_t hb, uint32_t cb) {
            if (b < d || hb == 0 || cb >= above) return kNone;
            const uint32_t ha = b == d ? above - cb : hb; // A keys of digit b
            const uint32_t gq = (cb + ha / 2 + above / (6 * ga)) * ga / above;
            return gq < ga ? gq : ga - 1;
        };
        const uint32_t g0 = group_of(b0, h.x, cb0), g1 = group_of(b1, h.y, cb1);
        s_hist[b0] = g0;
        s_hist[b1] = g1;
        if (g0 == q) atomicMin(&s_off, cb0);
        if (g1 == q) atomicMin(&s_off, cb1);
        __syncthreads();
        const uint32_t off = s_off;
        if (off == kNone) { // uniform: no digit
            group_finish(g, o, w, row, q, 0ull, s_c, 0, groups);
            return;
        }
        const uint32_t na = above; // < top_k <= kCap
        const uint64_t *alist = w.cand + static_cast<uint64_t>(row) * g.cand_ld;
        uint64_t v[kSortPer];
#pragma unroll
        for (uint32_t k = 0; k < kSortPer; ++k) {
            const uint32_t i = threadIdx.x + k * kRankThreads;
            v[k] = i < na ? alist[i] : 0ull;
        }
#pragma unroll
        for (uint32_t k = 0; k < kSortPer; ++k) {
            const uint32_t i = threadIdx.x + k * kRankThreads;
            wave_append(i < na && s_hist[static_cast<uint32_t>(v[k] >> 53)] == q, v[k], &s_n, s_c);
        }
        __syncthreads();
        n = s_n < kCap ? s_n : kCap;
        out = n;
        slot0 = off;
    } else {
        // B: its largest need words after A's slots.  Its first digit comes from
        // the row's histogram: digits strictly inside [blo, bhi]'s hold B keys
        // only, bhi's digit also the A keys not above it, blo's the rest of B.
        // Later digits, while B is long, from histograms of the list.
        const uint32_t need = g.top_k - above;
        uint64_t *blist = w.bucket + static_cast<uint64_t>(row) * kBucketCap;
        bool scan = true;
        if (listed) { // uniform
            const uint32_t nb = inb;
            const uint32_t dlo = w.sel[row].blo >> 21, dhi = bhi >> 21;
            auto b_digit = [&](uint32_t b, uint32_t hb, uint32_t cb) {
                if (b < dlo || b > dhi) return;
                const uint32_t higher = b == dhi ? 0u : cb - above; // B keys in the digits above b
                const uint32_t here = dlo == dhi ? nb : b == dhi ? hb - (above - cb) : b == dlo ? nb - higher : hb;
                if (higher < need && need <= higher + here) {
                    s_pick[0] = b;
                    s_pick[1] = higher;
                    s_pick[2] = here;
                }
            };
            b_digit(b0, h.x, cb0);
            b_digit(b1, h.y, cb1);
            __syncthreads();
            RowSel bs{};
            if (s_pick[0] == kNone) bs.mode = 2; // uniform; cannot happen with consistent counts: scans
            bs.prefix = s_pick[0];
            bs.depth = 11;
            bs.above = s_pick[1];
            bs.need = need - s_pick[1];
            bs.count = s_pick[1] + s_pick[2];
            if (bs.mode != 2) bs.mode = bs.count <= kCap ? 1u : 0u;
            const uint32_t enough = need + kSortDirect < kCap ? need + kSortDirect : kCap; // words worth one sort
            for (uint32_t pass = 1; pass < 3 && bs.mode != 2 && bs.count > enough; ++pass) {
                const uint32_t bits = pass == 2 ? 10u : 11u, nbins = 1u << bits;
                const uint32_t shift = 32u - bs.depth - bits;
                bs.mode = 0;
                for (uint32_t b = threadIdx.x; b < nbins; b += kRankThreads) s_hist[b] = 0;
                __syncthreads();
                for (uint32_t i0 = 0; i0 < nb; i0 += kSortPer * kRankThreads) {
                    uint32_t key[kSortPer];
#pragma unroll
                    for (uint32_t k = 0; k < kSortPer; ++k) {
                        const uint32_t i = i0 + threadIdx.x + k * kRankThreads;
                        key[k] = i < nb ? static_cast<uint32_t>(blist[i] >> 32) : 0u;
                    }
#pragma unroll
                    for (uint32_t k = 0; k < kSortPer; ++k) {
                        const uint32_t i = i0 + threadIdx.x + k * kRankThreads;
                        const bool match = bs.depth == 0 || (key[k] >> (32u - bs.depth)) == bs.prefix;
                        if (i < nb && match) atomicAdd(&s_hist[(key[k] >> shift) & (nbins - 1)], 1u);
                    }
                }
                __syncthreads();
                bs = pick_digit(bs, s_hist, bits, s_tmp, s_pick);
                if (bs.mode == 0) bs.count = nb; // still more than kCap: refine further
            }
            if (bs.mode == 1) { // uniform; else the ties at T exceed kCap
                for (uint32_t i0 = 0; i0 < nb; i0 += kSortPer * kRankThreads) {
                    uint64_t v[kSortPer];
#pragma unroll
                    for (uint32_t k = 0; k < kSortPer; ++k) {
                        const uint32_t i = i0 + threadIdx.x + k * kRankThreads;
                        v[k] = i < nb ? blist[i] : 0ull;
                    }
#pragma unroll
                    for (uint32_t k = 0; k < kSortPer; ++k) {
                        const uint32_t i = i0 + threadIdx.x + k * kRankThreads;
                        const uint32_t key = static_cast<uint32_t>(v[k] >> 32);
                        wave_append(i < nb && (bs.depth == 0 || (key >> (32u - bs.depth)) >= bs.prefix), v[k], &s_n, s_c);
                    }
                }
                __syncthreads();
                n = s_n; // bs.count <= kCap
                if (n <= kCap) { // uniform
                    out = need < n ? need : n;
                    slot0 = above;
                    scan = false;
                }
            }
        }
        if (scan) { // uniform: the whole row from scans
            __syncthreads(); // every thread has read s_pick, which resolve_row rewrites
            RowSel rs{};
            rs.need = g.top_k;
            rs = resolve_row(g, logits, w, row, rs, s_hist, s_tmp, s_pick);
            collect_row(g, logits + static_cast<int64_t>(row) * g.ld, blist, rs, s_tmp);
            __syncthreads(); // the list, written by the whole workgroup, is staged next
            n = rs.count < kCap ? rs.count : kCap;
            stage_words<kRankThreads>(s_c, blist, n, n);
            out = g.top_k;
            slot0 = 0;
        }
    }
    // one call site: rank_group inlines, so its LDS buffers keep their address space
    rank_group(g, o, w, row, q, s0, s_c, n, out, slot0, groups, s_d, s_hist, s_tmp, &s_tab, pw);
}

// A launch whose rows can take the fast list: one workgroup per row
// resolves, collects and ranks it in one launch.  A row the fast list resolved (k_smp_div listed it) goes
// straight to the ranking; the others take the radix selection, then the
// candidate list in column order.
static_assert(kRankThreads == kResolveThreads, "one workgroup shape for the whole tail");
__global__ __launch_bounds__(kRankThreads) void k_smp_tail(SmpGeo g, float *logits, SmpWs w, SmpOut o, SmpStates st,
                                                           uint32_t row0)
{
    __shared__ uint64_t s_c[kCapSlots];
    __shared__ uint32_t s_hist[kBins];
    __shared__ uint32_t s_tmp[kRankThreads / kWave];
    __shared__ uint32_t s_pick[3];
    const uint32_t row = row0 + blockIdx.x;
    const RowSel sel0 = w.sel[row];
    uint32_t count;
    if (sel0.fast_on && sel0.fast_count <= kCap) { // uniform: k_smp_div listed the candidates
        count = sel0.fast_count; // >= top_k: the maxima behind the threshold
    } else {
        const RowSel sel = resolve_row(g, logits, w, row, sel0, s_hist, s_tmp, s_pick);
        collect_row(g, logits + static_cast<int64_t>(row) * g.ld, w.cand + static_cast<uint64_t>(row) * g.cand_ld, sel,
                    s_tmp);
        count = sel.count;
        __syncthreads(); // the list, written by the whole workgroup, is read by the ranking
    }
    rank_row(g, w, o, st.v[blockIdx.x], row, count, s_c);
}

// Longer lists (top_k > kCap, so count == top_k): sorted kCap tiles ...
__global__ __launch_bounds__(kRankThreads) void k_smp_tile_sort(SmpGeo g, SmpWs w, uint32_t tiles)
{
    __shared__ uint64_t s_c[kCapSlots];
    const uint32_t row = blockIdx.x / tiles, tile = blockIdx.x % tiles;
    const uint32_t n = w.sel[row].count;
    const uint32_t b0 = tile * kCap;
    if (b0 >= n) return;
    const uint32_t len = n - b0 < kCap ? n - b0 : kCap;
    uint32_t np = kSortPer;
    while (np < len) np <<= 1;
    uint64_t *c = w.cand + static_cast<uint64_t>(row) * g.cand_ld + b0;
    stage_words<kRankThreads>(s_c, c, len, np);
    lds_sort_desc<kRankThreads>(s_c, np);
    for (uint32_t i = threadIdx.x; i < len; i += blockDim.x) c[i] = s_c[slot(i)];
}

// ... merged pairwise (runs of `width` into runs of 2 width), kMergePer
// outputs per thread located by a merge-path search ...
constexpr uint32_t kMergePer = 8;
__global__ __launch_bounds__(kBlock) void k_smp_merge(SmpGeo g, SmpWs w, const uint64_t *src, uint64_t *dst,
                                                      uint32_t width, uint32_t blocks_per_row)
{
    const uint32_t row = blockIdx.x / blocks_per_row;
    const uint32_t n = w.sel[row].count;
    const uint64_t o = (static_cast<uint64_t>(blockIdx.x % blocks_per_row) * kBlock + threadIdx.x) * kMergePer;
    if (o >= n) return;
    const uint64_t *s = src + static_cast<uint64_t>(row) * g.cand_ld;
    uint64_t *d = dst + static_cast<uint64_t>(row) * g.cand_ld;
    const uint64_t a0 = o / (2ull * width) * (2ull * width);
    const uint64_t la = n - a0 < width ? n - a0 : width;
    const uint64_t b0 = a0 + la;
    const uint64_t lb = n - b0 < width ? n - b0 : (b0 >= n ? 0 : width);
    const uint64_t *A = s + a0, *B = s + b0;
    const uint64_t diag = o - a0;
    uint64_t lo = diag > lb ? diag - lb : 0, hi = diag < la ? diag : la;
    while (lo < hi) {
        const uint64_t mid = (lo + hi) / 2;
        if (A[mid] > B[diag - mid - 1]) lo = mid + 1;
        else hi = mid;
    }
    uint64_t i = lo, j = diag - lo;
    const uint64_t end = o + kMergePer < a0 + la + lb ? o + kMergePer : a0 + la + lb;
    for (uint64_t k = o; k < end; ++k) {
        const bool takeA = j >= lb || (i < la && A[i] > B[j]);
        d[k] = takeA ? A[i++] : B[j++];
    }
}

// ... and finished from the sorted list.
__global__ __launch_bounds__(kRankThreads) void k_smp_finish(SmpGeo g, const uint64_t *sorted, SmpOut o,
                                                             SmpStates st, uint32_t row0)
{
    const uint32_t row = row0 + blockIdx.x;
    const uint64_t *c = sorted + static_cast<uint64_t>(row) * g.cand_ld;
    // kSortPer loads in flight per thread before the ranked stores
    for (uint32_t j0 = 0; j0 < g.top_k; j0 += kSortPer * kRankThreads) {
        uint64_t q[kSortPer];
#pragma unroll
        for (uint32_t r = 0; r < kSortPer; ++r) {
            const uint32_t j = j0 + threadIdx.x + r * kRankThreads;
            q[r] = c[j < g.top_k ? j : 0];
        }
#pragma unroll
        for (uint32_t r = 0; r < kSortPer; ++r) {
            const uint32_t j = j0 + threadIdx.x + r * kRankThreads;
            if (j < g.top_k) write_ranked(g, o, row, j, q[r]);
        }
    }
    select_slots<kRankThreads>(
        g, row, st.v[blockIdx.x], [&](uint32_t j) { return from_key(static_cast<uint32_t>(c[j] >> 32)); },
        [&](uint32_t j) { return static_cast<int32_t>(~static_cast<uint32_t>(c[j])); }, o);
}

// ---- validator: candidate ids and logits - max -------------------------------

struct ValArgs {
    const float *logits;
    int32_t *ids;
    float *scores;
    uint64_t n;
    uint64_t chunk_cols;
    uint32_t chunks;
    uint32_t vec;
};

// Chunk (value, lowest index) maxima, NaN never a candidate (argmax_merge).
__global__ __launch_bounds__(kBlock) void k_val_max(ValArgs a, uint64_t *part)
{
    __shared__ float s_v[kBlock / kWave];
    __shared__ uint32_t s_i[kBlock / kWave];
    const uint64_t c0 = static_cast<uint64_t>(blockIdx.x) * a.chunk_cols;
    const uint64_t c1 = c0 + a.chunk_cols < a.n ? c0 + a.chunk_cols : a.n;
    float bv = -__builtin_inff();
    uint32_t bi = kNone;
    for (uint64_t k = c0 + threadIdx.x; k < c1; k += blockDim.x) argmax_merge(bv, bi, a.logits[k], static_cast<uint32_t>(k));
    wave_argmax(bv, bi);
    if (threadIdx.x % kWave == 0) {
        s_v[threadIdx.x / kWave] = bv;
        s_i[threadIdx.x / kWave] = bi;
    }
    __syncthreads();
    if (threadIdx.x != 0) return;
    for (int v = 1; v < kBlock / kWave; ++v) argmax_merge(s_v[0], s_i[0], s_v[v], s_i[v]);
    part[blockIdx.x] = (static_cast<uint64_t>(s_i[0]) << 32) | f32_to_bits(s_v[0]);
}

// execute_build (validator/sm.rs): maximum starts at logits[0] and moves on
// strictly greater values, so it is the first maximal element (== compares
// -0 and +0 equal), or logits[0] itself when that is NaN.
__global__ __launch_bounds__(kBlock) void k_val_write(ValArgs a, const uint64_t *part)
{
    __shared__ float s_m;
    if (threadIdx.x < kWave) {
        float bv = -__builtin_inff();
        uint32_t bi = kNone;
        for (uint32_t c = threadIdx.x; c < a.chunks; c += kWave) {
            const uint64_t q = part[c];
            argmax_merge(bv, bi, bits_to_f32(static_cast<uint32_t>(q)), static_cast<uint32_t>(q >> 32));
        }
        wave_argmax(bv, bi);
        if (threadIdx.x == 0) {
            const float first = a.logits[0];
            s_m = first != first ? first : bv;
        }
    }
    __syncthreads();
    const float m = s_m;
    const uint64_t c0 = static_cast<uint64_t>(blockIdx.x) * a.chunk_cols;
    const uint64_t c1 = c0 + a.chunk_cols < a.n ? c0 + a.chunk_cols : a.n;
    for (uint64_t k = c0 + threadIdx.x; k < c1; k += blockDim.x) {
        a.ids[k] = static_cast<int32_t>(k);
        a.scores[k] = a.logits[k] - m;
    }
}

constexpr uint32_t kTargetBlocks = 2048;
constexpr uint64_t kMinChunkCols = 4 * kBlock;

void plan_chunks(uint32_t rows, uint64_t card, uint64_t &chunk_cols, uint32_t &chunks)
{
    const uint64_t want = (kTargetBlocks + rows - 1) / rows;
    uint64_t c = (card + want - 1) / want;
    if (c < kMinChunkCols) c = kMinChunkCols;
    // whole float4 steps of a workgroup: every thread of a chunk visits the
    // same number of float4 (the last chunk of a row excepted)
    c = (c + kMinChunkCols - 1) / kMinChunkCols * kMinChunkCols;
    chunk_cols = c;
    chunks = static_cast<uint32_t>((card + c - 1) / c);
}

uint64_t align256(uint64_t b) { return (b + 255) & ~uint64_t{255}; }

struct WsLayout {
    uint64_t part, psum, sub, seg, sel, hist, ehist, ties, cand, cand2, bucket, gbest, total;
};

// Geometry of a launch (what launch_sampler derives from its arguments).
SmpGeo plan_geo(uint32_t rows, uint64_t card, uint32_t top_k)
{
    SmpGeo g{};
    g.rows = rows;
    g.card = card;
    plan_chunks(rows, card, g.chunk_cols, g.chunks);
    g.top_k = top_k;
    g.cand_ld = top_k > kCap ? top_k : kCap;
    return g;
}

// k_smp_rank's workgroups per row: A groups of about 1024 keys (at most
// kMaxGroups - 1, and at most kRankWgs workgroups in all while there are
// rows to spare), then B.
constexpr uint32_t kRankWgs = 256;
uint32_t rank_groups(uint32_t top_k, uint32_t rows)
{
    uint32_t ga = (top_k + 1023) / 1024;
    if (ga > kMaxGroups - 1) ga = kMaxGroups - 1;
    const uint32_t fit = rows < kRankWgs ? kRankWgs / rows : 1u; // groups that keep one wave of workgroups
    if (ga + 1 > fit) ga = fit > 1 ? fit - 1 : 1u;
    return ga + 1;
}

WsLayout layout(uint32_t rows, uint32_t chunks, uint64_t chunk_cols, uint64_t cand_ld, bool merge, bool bucket)
{
    const uint64_t spc = (chunk_cols + kSub - 1) / kSub;
    WsLayout l{};
    l.part = 0;
    l.psum = l.part + align256(uint64_t{rows} * chunks * sizeof(float));
    l.sub = l.psum + align256(uint64_t{rows} * chunks * sizeof(double));
    l.seg = l.sub + align256(uint64_t{rows} * chunks * spc * sizeof(SubSum));
    l.sel = l.seg + align256(uint64_t{rows} * chunks * spc * sizeof(SegInfo));
    l.hist = l.sel + align256(uint64_t{rows} * sizeof(RowSel));
    l.ehist = l.hist + align256(uint64_t{rows} * kBins * sizeof(uint32_t));
    l.ties = l.ehist + align256(uint64_t{rows} * kBins * sizeof(uint32_t));
    l.cand = l.ties + align256(uint64_t{rows} * chunks * sizeof(uint32_t));
    l.cand2 = l.cand + align256(uint64_t{rows} * cand_ld * sizeof(uint64_t));
    l.bucket = merge ? l.cand2 + align256(uint64_t{rows} * cand_ld * sizeof(uint64_t)) : l.cand2;
    l.gbest = bucket ? l.bucket + align256(uint64_t{rows} * kBucketCap * sizeof(uint64_t)) : l.bucket;
    l.total = bucket ? l.gbest + align256(uint64_t{rows} * kMaxGroups * sizeof(GroupBest)) : l.gbest;
    return l;
}

} // namespace

uint64_t sampler_workspace_bytes(uint32_t rows, uint64_t card, uint32_t top_k)
{
    const SmpGeo g = plan_geo(rows, card, top_k);
    return layout(rows, g.chunks, g.chunk_cols, g.cand_ld, top_k > kCap, bucket_path(g)).total;
}

hipError_t launch_sampler(const SamplerArgs &a, hipStream_t s)
{
    if (a.rows == 0 || a.card == 0 || a.top_k == 0 || a.top_k > a.card || a.card > 0x7fffffffull || !a.workspace)
        return hipErrorInvalidValue;
    SmpGeo g = plan_geo(a.rows, a.card, a.top_k);
    if (g.chunks > kBins) return hipErrorInvalidValue; // resolve_row counts ties per chunk in kBins words
    g.ld = a.logits_ld;
    g.vec = (reinterpret_cast<uintptr_t>(a.logits) % 16 == 0) && (a.rows == 1 || a.logits_ld % 4 == 0);
    g.scale = a.scale;
    const bool merge = a.top_k > kCap, bucket = bucket_path(g);
    const WsLayout l = layout(a.rows, g.chunks, g.chunk_cols, g.cand_ld, merge, bucket);
    char *base = static_cast<char *>(a.workspace);
    SmpWs w{};
    w.part = reinterpret_cast<float *>(base + l.part);
    w.psum = reinterpret_cast<double *>(base + l.psum);
    w.sub = reinterpret_cast<SubSum *>(base + l.sub);
    w.seg = reinterpret_cast<SegInfo *>(base + l.seg);
    w.sel = reinterpret_cast<RowSel *>(base + l.sel);
    w.hist = reinterpret_cast<uint32_t *>(base + l.hist);
    w.ehist = reinterpret_cast<uint32_t *>(base + l.ehist);
    w.ties = reinterpret_cast<uint32_t *>(base + l.ties);
    w.cand = reinterpret_cast<uint64_t *>(base + l.cand);
    w.cand2 = reinterpret_cast<uint64_t *>(base + l.cand2);
    w.bucket = reinterpret_cast<uint64_t *>(base + l.bucket);
    w.gbest = reinterpret_cast<GroupBest *>(base + l.gbest);

    const dim3 grid(a.rows * g.chunks);
    if (g.chunk_cols <= kFuseCols) {
        k_smp_max<true><<<grid, kBlock, 0, s>>>(g, a.logits, w);
        if (bucket) k_smp_expseg<true><<<dim3(a.rows + a.rows * g.chunks), kBlock, 0, s>>>(g, a.logits, w);
        else k_smp_expseg<false><<<dim3(a.rows + a.rows * g.chunks), kBlock, 0, s>>>(g, a.logits, w);
    } else {
        k_smp_max<false><<<grid, kBlock, 0, s>>>(g, a.logits, w);
        if (bucket) k_smp_exp<true><<<grid, kBlock, 0, s>>>(g, a.logits, w);
        else k_smp_exp<false><<<grid, kBlock, 0, s>>>(g, a.logits, w);
        k_smp_seg<<<grid, kBlock, 0, s>>>(g, a.logits, w);
    }
    k_smp_sum<<<a.rows, bucket ? kSumThreads : 2 * kWave, 0, s>>>(g, a.logits, w);
    if (bucket) k_smp_divlist<<<grid, kBlock, 0, s>>>(g, a.logits, w);
    else k_smp_div<<<grid, kBlock, 0, s>>>(g, a.logits, w);
    // Rows resolved by the fast list need no selection: when the fast list
    // applies, k_smp_tail selects (in one workgroup per row, for the rows it
    // left) and ranks in one launch.  Otherwise, up to kCap, k_smp_div has
    // listed the candidates around the bracket and k_smp_rank selects and
    // ranks in groups; above kCap the selection kernels spread the
    // candidate list over (row, chunk) workgroups for the merge sort.
    const bool tail = !merge && !bucket;
    if (merge) {
        k_smp_resolve<<<a.rows, kResolveThreads, 0, s>>>(g, a.logits, w);
        k_smp_collect<<<grid, kBlock, 0, s>>>(g, a.logits, w);
    }

    SmpOut o{};
    o.sorted = a.sorted;
    o.sorted_ld = a.sorted_ld;
    o.top_p = a.top_p;
    o.top_i = a.top_i;
    o.top_ld = a.top_ld;
    o.selected = a.selected;
    o.score = a.score;
    o.status = a.status;

    const uint32_t groups = rank_groups(a.top_k, a.rows);
    const uint64_t *sorted = w.cand;
    if (merge) {
        const uint32_t tiles = (a.top_k + kCap - 1) / kCap;
        k_smp_tile_sort<<<a.rows * tiles, kRankThreads, 0, s>>>(g, w, tiles);
        const uint32_t per_block = kBlock * kMergePer;
        const uint32_t bpr = (a.top_k + per_block - 1) / per_block;
        uint64_t *src = w.cand, *dst = w.cand2;
        for (uint32_t width = kCap; width < a.top_k; width *= 2) {
            k_smp_merge<<<a.rows * bpr, kBlock, 0, s>>>(g, w, src, dst, width, bpr);
            uint64_t *t = src;
            src = dst;
            dst = t;
        }
        sorted = src;
    }
    for (uint32_t r0 = 0; r0 < a.rows; r0 += kStatesInline) {
        const uint32_t nr = a.rows - r0 < kStatesInline ? a.rows - r0 : kStatesInline;
        SmpStates st{};
        for (uint32_t i = 0; i < nr; ++i) st.v[i] = a.states[r0 + i];
        if (merge) k_smp_finish<<<nr, kRankThreads, 0, s>>>(g, sorted, o, st, r0);
        else if (tail) k_smp_tail<<<nr, kRankThreads, 0, s>>>(g, a.logits, w, o, st, r0);
        else k_smp_rank<<<nr * groups, kRankThreads, 0, s>>>(g, a.logits, w, o, st, r0, groups);
    }
    return hipGetLastError();
}

uint64_t validator_workspace_bytes(uint64_t n)
{
    uint64_t chunk_cols;
    uint32_t chunks;
    plan_chunks(1, n, chunk_cols, chunks);
    return uint64_t{chunks} * sizeof(uint64_t);
}

hipError_t launch_validator(const float *logits, uint64_t n, int32_t *ids, float *scores, void *workspace,
                            hipStream_t s)
{
    if (n == 0 || n > 0x7fffffffull || !workspace) return hipErrorInvalidValue;
    ValArgs a{};
    a.logits = logits;
    a.ids = ids;
    a.scores = scores;
    a.n = n;
    plan_chunks(1, n, a.chunk_cols, a.chunks);
    uint64_t *part = static_cast<uint64_t *>(workspace);
    k_val_max<<<a.chunks, kBlock, 0, s>>>(a, part);
    k_val_write<<<a.chunks, kBlock, 0, s>>>(a, part);
    return hipGetLastError();
}

} // namespace emel
