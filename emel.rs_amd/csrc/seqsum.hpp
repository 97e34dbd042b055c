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

} // namespace emel
