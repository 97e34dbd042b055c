// seqsum.hpp -- the pieces of an exact, parallel evaluation of a
// sequential f32 sum of non-negative addends:
//
//     s_0 = +0,  s_k = RN(s_{k-1} + e_k)   (k = 1..n, round to nearest even)
//
// emel-logits' sampler normalises its softmax by exactly this sum
// (`total += *value` over f32, crates/emel-logits/src/sampler/sm.rs:786-790),
// so the GPU must reproduce its rounding, not just approximate the sum.
//
// Every finite s >= 0 is m * 2^u with an integer m < 2^24 and u >= -149,
// where 2^u is the spacing of f32 values around s (seq_state).  While the
// running sum stays below 2^24 units of 2^u, RN(s + e) is s plus e rounded
// to a whole number of units: the f32 grid is exactly the multiples of 2^u
// there.  So over a run of addends in one binade
//
//     s_k = (m + R_1 + ... + R_k) * 2^u,   R_i = round(e_i / 2^u),
//
// an integer prefix sum, which a workgroup evaluates in parallel.  The
// identity needs three things, and an addend that breaks one of them is an
// "event" that the caller performs with one real f32 addition instead:
//   - the sum stays below 2^24 units (otherwise it enters the next binade,
//     whose spacing is 2^(u+1));
//   - e_i / 2^u is not an odd multiple of 1/2 (a tie: round-to-even then
//     depends on the parity of the running m);
//   - e_i is not NaN (seq_units reports NaN as 2^24 units, an event).
// After an event the running sum restarts from the new s (seq_state).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.hpp"
#include "libm_replica.hpp"

namespace emel {

constexpr uint32_t kSeqLimit = 1u << 24; // units per binade

struct SeqState {
    uint32_t m; // s / 2^u, below 2^24
    int32_t u;  // exponent of the spacing around s, >= -149
};

// State of a finite s >= +0.  Zero and subnormal s share the spacing 2^-149
// with the lowest normal binade, so they take u = -149 and m < 2^23.
__host__ __device__ __forceinline__ SeqState seq_state(float s)
{
    const uint32_t b = f32_to_bits(s);
    const uint32_t e = b >> 23;
    if (e == 0) return SeqState{b & 0x7fffffu, -149};
    return SeqState{(b & 0x7fffffu) | 0x800000u, static_cast<int32_t>(e) - 150};
}

// m * 2^u as an f32 (exact for m < 2^24).
__host__ __device__ __forceinline__ float seq_value(uint32_t m, int32_t u)
{
    return __builtin_ldexpf(static_cast<float>(m), u);
}

// Units of 2^u that RN(s + e) adds to s (valid unless `tie` is set or the
// running sum reaches 2^24 units): e / 2^u rounded to the nearest integer.
// e is >= +0 or NaN.  e / 2^u is a power-of-two scaling, exact except when
// it would overflow (clamped below: such an addend is an event anyway) or
// when it is far below 1/2 (any inexactness then still rounds to 0).  NaN
// and values of 2^24 units or more report 2^24.
__host__ __device__ __forceinline__ uint32_t seq_units(float e, int32_t u, bool &tie)
{
    float t = __builtin_ldexpf(e, -u);
    t = __builtin_fminf(t, 16777216.0f); // IEEE minNum: also NaN -> 2^24
#if defined(__HIP_DEVICE_COMPILE__)
    tie = __builtin_amdgcn_fractf(t) == 0.5f; // t - floor(t), exact for 0 <= t <= 2^24
#else
    tie = (t - __builtin_floorf(t)) == 0.5f;
#endif
    return static_cast<uint32_t>(__builtin_rintf(t));
}


// Inclusive prefix sum over the 64 lanes of a wave (DPP: row shifts within
// rows of 16 lanes, then the row broadcasts of lanes 15 and 31).
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v)
{
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x111, 0xf, 0xf, true)); // row_shr:1
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x112, 0xf, 0xf, true)); // row_shr:2
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x114, 0xf, 0xf, true)); // row_shr:4
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x118, 0xf, 0xf, true)); // row_shr:8
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x142, 0xa, 0xf, false)); // row_bcast:15
    v += static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x143, 0xc, 0xf, false)); // row_bcast:31
    return v;
}

// The same scan over doubles (each DPP step moves both halves).
template <int CTRL, int ROW_MASK, bool BOUND>
__device__ __forceinline__ double dpp_shift_f64(double v)
{
    const uint64_t b = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = static_cast<uint32_t>(
        __builtin_amdgcn_update_dpp(0, static_cast<int>(static_cast<uint32_t>(b)), CTRL, ROW_MASK, 0xf, BOUND));
    const uint32_t hi = static_cast<uint32_t>(
        __builtin_amdgcn_update_dpp(0, static_cast<int>(static_cast<uint32_t>(b >> 32)), CTRL, ROW_MASK, 0xf, BOUND));
    return __builtin_bit_cast(double, (static_cast<uint64_t>(hi) << 32) | lo);
}

__device__ __forceinline__ double wave_incl_scan_f64(double v)
{
    v += dpp_shift_f64<0x111, 0xf, true>(v);
    v += dpp_shift_f64<0x112, 0xf, true>(v);
    v += dpp_shift_f64<0x114, 0xf, true>(v);
    v += dpp_shift_f64<0x118, 0xf, true>(v);
    v += dpp_shift_f64<0x142, 0xa, false>(v);
    v += dpp_shift_f64<0x143, 0xc, false>(v);
    return v;
}

// Relative distance, either way, between a running f32 sum after `a`
// roundings of non-negative addends (starting from an exact value) and the
// exact sum: each rounding scales by (1 + d) with |d| < 2^-24, so the ratio
// lies in [(1 - 2^-24)^a, (1 + 2^-24)^a], inside [1 - a 2^-24, 1 + a 2^-24 +
// (a 2^-24)^2] (Bernoulli's inequality; e^x <= 1 + x + x^2 for x <= 1).
// 2^-30 covers the f64 rounding of the predicted sums (up to 2^22 terms).
// Past 2^22 roundings it returns 1, which makes every prediction fail.
__host__ __device__ __forceinline__ double seq_rel_bound(double a)
{
    const double au = a * 0x1p-24;
    return au <= 0.25 ? au * (1.0 + au) + 0x1p-30 : 1.0;
}

// ---- one wave walks a tile of its addends ----------------------------------

// The running sum of a walk: m units of 2^u while finite.
struct SumState {
    uint32_t m;
    int32_t u;
    bool finite;
    float special; // NaN or +inf once the running sum leaves the finite range
};

// The rounds over one tile of PER * 64 elements (this lane's PER consecutive
// ones in e).  A round counts the uncommitted elements' units at the current
// binade and scans the lane totals.  Without an event it commits them all.
// Otherwise the first event lies in the first lane that holds a tie or whose
// running units reach 2^24; that lane's elements are then read one by one on
// the scalar unit up to the event, which is added with one f32 addition, and
// the next round starts after it.  A single wave issues these instructions
// one at a time, so every round is kept to few of them: committed elements
// are zeroed once per event (a zero adds no units and is no tie), and a tie
// is found from t - rint(t), which is exactly +-1/2 for a tie and smaller
// otherwise, one maximum per lane.
template <uint32_t PER>
__device__ __forceinline__ void sum_tile(const float (&e)[PER], SumState &s)
{
    const uint32_t lane = threadIdx.x % kWave;
    if (!s.finite) {
        // +inf stays +inf unless a NaN follows; NaN stays NaN
        bool nan = false;
#pragma unroll
        for (uint32_t j = 0; j < PER; ++j) nan |= e[j] != e[j];
        if (__ballot(nan)) s.special = __builtin_nanf("");
        return;
    }
    float x[PER]; // e, with the committed elements zeroed
#pragma unroll
    for (uint32_t j = 0; j < PER; ++j) x[j] = e[j];
    while (true) {
        // this round's units at the current binade (seq_units: the clamp
        // also takes NaN to 2^24 units, an event), kept with t - rint(t)
        // for the event search below
        uint32_t r[PER], lsum = 0;
        float d[PER], dmax = 0.0f;
#pragma unroll
        for (uint32_t j = 0; j < PER; ++j) {
            float t = __builtin_ldexpf(x[j], -s.u);
            t = __builtin_fminf(t, 16777216.0f); // IEEE minNum: also NaN -> 2^24
            const float rt = __builtin_rintf(t);
            d[j] = t - rt; // exact: t and rint(t) are within 1/2
            r[j] = static_cast<uint32_t>(rt);
            lsum += r[j];
            dmax = __builtin_fmaxf(dmax, __builtin_fabsf(d[j]));
        }
        // lsum <= PER * 2^24; saturated at 2^24 the scan cannot overflow (a
        // saturated value already marks a crossing)
        const uint32_t x_in = lsum < kSeqLimit ? lsum : kSeqLimit;
        const uint32_t incl = wave_incl_scan(x_in);
        // lanes before the first event lane neither tie nor reach 2^24, so
        // its running units before it are s.m plus its exclusive prefix
        const uint64_t emask = __ballot(dmax == 0.5f || s.m + incl >= kSeqLimit);
        if (emask == 0) { // no event: the tile is committed
            s.m += static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(incl), kWave - 1));
            return;
        }
        const int fl = __builtin_ctzll(emask);
        uint32_t run = s.m + static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(incl - x_in), fl));
        // lane fl's elements in order, on the scalar unit: the first tie
        // (|t - rint(t)| = 1/2), or the first element whose units reach 2^24
        // (zeroed elements add 0 units and hold no tie)
        uint32_t k = PER * kWave, run_k = 0;
        float e_k = 0.0f;
#pragma unroll
        for (uint32_t j = 0; j < PER; ++j) {
            if (k == PER * kWave) {
                const uint32_t rj = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(r[j]), fl));
                const uint32_t dj = static_cast<uint32_t>(__builtin_amdgcn_readlane(__builtin_bit_cast(int, d[j]), fl));
                if ((dj & 0x7fffffffu) == 0x3f000000u || run + rj >= kSeqLimit) {
                    k = PER * static_cast<uint32_t>(fl) + j;
                    run_k = run;
                    e_k = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x[j]), fl));
                } else {
                    run += rj;
                }
            }
        }
        if (k == PER * kWave) return; // unreachable: the lane holds an event
        const float sn = seq_value(run_k, s.u) + e_k; // the event element: one f32 addition
        if (!(sn < __builtin_inff())) { // NaN or +inf
            s.special = sn;
            s.finite = false;
            bool nan = false;
#pragma unroll
            for (uint32_t j = 0; j < PER; ++j) nan |= (PER * lane + j > k) && e[j] != e[j];
            if (__ballot(nan)) s.special = __builtin_nanf("");
            return;
        }
        const SeqState st = seq_state(sn);
        s.m = st.m;
        s.u = st.u;
        if (k + 1 >= PER * kWave) return;
        // elements up to k are committed
        const int32_t kk = static_cast<int32_t>(k) - static_cast<int32_t>(PER * lane);
#pragma unroll
        for (uint32_t j = 0; j < PER; ++j) x[j] = static_cast<int32_t>(j) <= kk ? 0.0f : x[j];
    }
}

} // namespace emel
