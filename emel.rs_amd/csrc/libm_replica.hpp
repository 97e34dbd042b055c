// libm_replica.hpp -- scalar math with the exact bits the reference's CPU
// path produces.
//
// The reference calls Rust std f32::exp / f32::tanh (unary.rs:538, :598;
// reductions.rs:584), which on x86_64-linux-gnu are glibc expf / tanhf.
// A correctly rounded GPU exp/tanh differs from glibc on ~6e-5 (expf) and
// ~5% (tanhf) of inputs, so these functions restate glibc's published
// algorithms instead:
//
//   emel_expf    ARM optimized-routines expf (math/expf.c, the
//                implementation in glibc since 2.28): x*N/ln2 = k + r with
//                N = 32, exp(x) = 2^(k/N) * p(r) evaluated in double, with
//                the range reduction and polynomial contracted to fused
//                multiply-adds as the x86_64 FMA build of glibc computes it.
//   emel_expm1f  fdlibm s_expm1f.c (Sun Microsystems, 1993; glibc's
//                sysdeps/ieee754/flt-32): reduction by ln2 split into hi/lo,
//                a degree-5 rational correction term, no contraction.
//   emel_tanhf   fdlibm s_tanhf.c: tanh(x) = 1 - 2/(expm1(2|x|)+2) for
//                |x| >= 1, -t/(t+2) with t = expm1(-2|x|) below.
//   emel_logf    ARM optimized-routines logf (math/logf.c, in glibc since
//                2.28): a 16-entry (1/c, log c) table and a cubic in
//                r = z/c - 1, in double (emel-logits' sampler, f32::ln).
//   emel_sinf, emel_cosf
//                ARM optimized-routines sinf / cosf (math/sinf.c, cosf.c,
//                sincosf.h, sincosf_data.c): reduction by pi/2 in double,
//                Payne-Hanek for large inputs, even/odd polynomials.
//   emel_log1pf  fdlibm s_log1pf.c (softplus).
//
// The table holds the correctly rounded doubles of 2^(i/32).  glibc stores
// them with i << 47 subtracted and forms 2^(k/32) as tab[k % 32] + (k << 47)
// on the bit patterns; here 2^(k/32) = ldexp(tab[k % 32], floor(k / 32)),
// the same double whenever it is normal (always, on the main path).
//
// Every function is __host__ __device__: tests build them for the CPU and
// compare them with the host glibc over all 2^32 float inputs.  Compile
// with -ffp-contract=off: the only fused operations are the explicit fma().
//
// The constants, tables and steps of the functions above are those of the
// two published implementations named, restated in this file's own code;
// their licences ask for these notices:
//
// ---- fdlibm (emel_expm1f, emel_tanhf, emel_log1pf) --------------------------
// Copyright (C) 1993 by Sun Microsystems, Inc. All rights reserved.
//
// Developed at SunPro, a Sun Microsystems, Inc. business.
// Permission to use, copy, modify, and distribute this
// software is freely granted, provided that this notice
// is preserved.
//
// (The float versions s_expm1f.c, s_tanhf.c and s_log1pf.c are the
// conversion to float by Ian Lance Taylor, Cygnus Support.)
//
// ---- ARM optimized-routines (emel_expf, emel_logf, emel_sinf, emel_cosf) ---
// Copyright (c) 2017-2018 Arm Limited.
// SPDX-License-Identifier: MIT (the project is MIT OR Apache-2.0 WITH
// LLVM-exception; the MIT terms are taken here):
//
// Permission is hereby granted, free of charge, to any person obtaining a
// copy of this software and associated documentation files (the
// "Software"), to deal in the Software without restriction, including
// without limitation the rights to use, copy, modify, merge, publish,
// distribute, sublicense, and/or sell copies of the Software, and to permit
// persons to whom the Software is furnished to do so, subject to the
// following conditions:
//
// The above copyright notice and this permission notice shall be included
// in all copies or substantial portions of the Software.
//
// THE SOFTWARE IS PROVIDED "AS IS", WITHOUT WARRANTY OF ANY KIND, EXPRESS
// OR IMPLIED, INCLUDING BUT NOT LIMITED TO THE WARRANTIES OF
// MERCHANTABILITY, FITNESS FOR A PARTICULAR PURPOSE AND NONINFRINGEMENT. IN
// NO EVENT SHALL THE AUTHORS OR COPYRIGHT HOLDERS BE LIABLE FOR ANY CLAIM,
// DAMAGES OR OTHER LIABILITY, WHETHER IN AN ACTION OF CONTRACT, TORT OR
// OTHERWISE, ARISING FROM, OUT OF OR IN CONNECTION WITH THE SOFTWARE OR THE
// USE OR OTHER DEALINGS IN THE SOFTWARE.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace emel {

// tab[i] = bits(2^(i/32)) - (i << 47): the double nearest 2^(i/32) with
// i/32 taken back out of its exponent field, i = 0..31, so that adding
// k << 47 to tab[k % 32] (the exponent field gains k / 32 and the i/32
// cancels) gives bits(2^(k/32)) without a separate scaling.
static constexpr uint64_t kExp2Table[32] = {
    0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full, 0x3fef9301d0125b51ull,
    0x3fef72b83c7d517bull, 0x3fef54873168b9aaull, 0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull,
    0x3fef06fe0a31b715ull, 0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,
    0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull, 0x3feea47eb03a5585ull,
    0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull, 0x3feea11473eb0187ull, 0x3feea589994cce13ull,
    0x3feeace5422aa0dbull, 0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,
    0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull, 0x3fef3720dcef9069ull,
    0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full, 0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull,
};

__host__ __device__ __forceinline__ float bits_to_f32(uint32_t u) { return __builtin_bit_cast(float, u); }
__host__ __device__ __forceinline__ uint32_t f32_to_bits(float f) { return __builtin_bit_cast(uint32_t, f); }
__host__ __device__ __forceinline__ double bits_to_f64(uint64_t u) { return __builtin_bit_cast(double, u); }
__host__ __device__ __forceinline__ uint64_t f64_to_bits(double d) { return __builtin_bit_cast(uint64_t, d); }

// Constants of the expf main path: N/ln2 with N = 32, the rounding shift
// 1.5*2^52, and the cubic coefficients of 2^(r/N) - 1 pre-scaled by N^-1,
// N^-2, N^-3.
struct ExpfConsts {
    double inv_ln2n = 0x1.71547652b82fep+0 * 32.0;
    double shift = 0x1.8p+52;
    double c0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
    double c1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
    double c2 = 0x1.62e42ff0c52d6p-1 / 32.0;
};

// The constants held in vector registers for a whole kernel.  gfx950's
// three-operand double instructions take no literals and one scalar
// operand, so fma(c, r, c') would otherwise rebuild a constant in vector
// registers for every element.
__host__ __device__ __forceinline__ ExpfConsts expf_consts_in_vgprs()
{
    ExpfConsts c;
#if defined(__HIP_DEVICE_COMPILE__)
    asm volatile("" : "+v"(c.inv_ln2n), "+v"(c.shift), "+v"(c.c0), "+v"(c.c1), "+v"(c.c2));
#endif
    return c;
}

// Marks y as computed on every path: the compiler may not sink its
// computation into the branch of a later select (a divergent branch per
// element costs more than the arithmetic it would skip).
__host__ __device__ __forceinline__ float keep_unconditional(float y)
{
#if defined(__HIP_DEVICE_COMPILE__)
    asm volatile("" : "+v"(y));
#endif
    return y;
}

// The main path of expf: x*N/ln2 = k + r, 2^(k/N) from the table, the
// cubic in r, all in double.  Defined (and in range for the table index)
// for every x; the result is expf(x) whenever -0x1.9fe368p6 <= x <=
// 0x1.62e42ep6, the range in which glibc takes this path.
__host__ __device__ __forceinline__ float expf_main_path(float x, const uint64_t *tab,
                                                         const ExpfConsts &c = ExpfConsts{})
{
    const double xd = static_cast<double>(x);
    double kd = __builtin_fma(c.inv_ln2n, xd, c.shift);
    const uint64_t ki = f64_to_bits(kd);
    kd -= c.shift;
    const double r = __builtin_fma(c.inv_ln2n, xd, -kd);
    // k is the low word of kd's bits.  2^(k/N) = tab[k mod N] + (k << 47) as
    // 64-bit integers: the addend has no low word, so only the high word
    // changes (by k << 15).  Exact while k / N stays inside the double
    // exponent range, which it does for every |x| < 700; larger |x| give
    // garbage here that the callers' range selects replace.
    struct Words {
        uint32_t lo, hi;
    };
    const uint32_t k = static_cast<uint32_t>(ki);
    const Words tk = __builtin_bit_cast(Words, tab[k & 31]);
    const double s = __builtin_bit_cast(double, Words{tk.lo, tk.hi + (k << 15)});
    const double z = __builtin_fma(c.c0, r, c.c1);
    const double r2 = r * r;
    double y = __builtin_fma(c.c2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    y = y * s;
    return static_cast<float>(y);
}

// expf.  `tab` is kExp2Table or a copy of it (kernels stage it in LDS).
// glibc branches to its special cases (|x| >= 88, NaN, infinities) before
// the main path; here the main path always runs and the special results
// are selected afterwards, which keeps a wave free of divergent branches:
// overflow (x > 0x1.62e42ep6, +inf) -> +inf, underflow (x < -0x1.9fe368p6,
// -inf) -> 0, NaN -> x + x.
__host__ __device__ __forceinline__ float emel_expf(float x, const uint64_t *tab,
                                                    const ExpfConsts &c = ExpfConsts{})
{
    float y = keep_unconditional(expf_main_path(x, tab, c));
    y = x > 0x1.62e42ep6f ? __builtin_inff() : y;
    y = x < -0x1.9fe368p6f ? 0.0f : y;
    return x != x ? x + x : y;
}

// expf for arguments that are <= 0 or NaN (soft_max's x - max): the same
// bits as emel_expf, with the special cases folded into one select, since
// only the underflow (and -inf) case can occur.
__host__ __device__ __forceinline__ float emel_expf_nonpos(float x, const uint64_t *tab,
                                                           const ExpfConsts &c = ExpfConsts{})
{
    // x < log(2^-150) (including -inf): 0, as emel_expf returns
    const float y = keep_unconditional(expf_main_path(x, tab, c));
    return x < -0x1.9fe368p6f ? 0.0f : y;
}

// Correctly rounded f32 quotient a / b through a double reciprocal:
// RN24(RN53(a * RN53(1/b))) == RN24(a / b) for finite a and normal b >= 1
// (no over/underflow of the intermediate).  Proof: the double product is
// a/b * (1 + e) with |e| < 2^-51.9.  RN24 of it can differ from RN24(a/b)
// only if a rounding midpoint m lies within that distance of a/b.  For
// m = M * 2^k with M an odd 25-bit integer and a, b carrying 24-bit
// significands A, B, a - b*m is a non-zero multiple of 2^(k + exponent of
// b) whenever b is not a power of two (a/b is then never a midpoint), so
// |a/b - m| > 2^-49 * m; for subnormal results the grid is 2^-150 and
// |a/b - m| > 2^-174 while the error is below 2^-177.  If b is a power of
// two the reciprocal and the product are exact.  NaN and infinite b
// propagate as in a / b.  soft_max divides every element of a row by the
// same row sum b >= 1, so one double reciprocal per row replaces the
// iterative f32 division per element.
__host__ __device__ __forceinline__ float div_by_recip(float a, double recip_b)
{
    return static_cast<float>(static_cast<double>(a) * recip_b);
}

// expm1f, fdlibm float version.
__host__ __device__ __forceinline__ float emel_expm1f(float x)
{
    constexpr float kLn2Hi = 6.9313812256e-01f;  // 0x3f317180
    constexpr float kLn2Lo = 9.0580006145e-06f;  // 0x3717f7d1
    constexpr float kInvLn2 = 1.4426950216e+00f; // 0x3fb8aa3b
    constexpr float kQ1 = -3.3333335072e-02f;    // 0xbd088889
    constexpr float kQ2 = 1.5873016091e-03f;     // 0x3ad00d01
    constexpr float kQ3 = -7.9365076090e-05f;    // 0xb8a670cd
    constexpr float kQ4 = 4.0082177293e-06f;     // 0x36867e54
    constexpr float kQ5 = -2.0109921195e-07f;    // 0xb457edbb

    uint32_t hx = f32_to_bits(x);
    const uint32_t negative = hx & 0x80000000u;
    hx &= 0x7fffffffu;
    if (hx >= 0x4195b844u) { // |x| >= 27 ln2
        if (hx >= 0x42b17218u) {
            if (hx > 0x7f800000u) return x + x; // NaN
            if (hx == 0x7f800000u) return negative ? -1.0f : x;
            if (x > 8.8721679688e+01f) return __builtin_inff();
        }
        if (negative) return 1.0e-30f - 1.0f; // -1
    }
    float hi, lo, c = 0.0f, t;
    int32_t k;
    if (hx > 0x3eb17218u) { // |x| > ln2/2
        if (hx < 0x3f851592u) { // |x| < 3 ln2 / 2
            if (!negative) { hi = x - kLn2Hi; lo = kLn2Lo; k = 1; }
            else { hi = x + kLn2Hi; lo = -kLn2Lo; k = -1; }
        } else {
            k = static_cast<int32_t>(kInvLn2 * x + (negative ? -0.5f : 0.5f));
            t = static_cast<float>(k);
            hi = x - t * kLn2Hi;
            lo = t * kLn2Lo;
        }
        x = hi - lo;
        c = (hi - x) - lo;
    } else if (hx < 0x33000000u) { // |x| < 2^-25
        return x;
    } else {
        k = 0;
    }
    const float hfx = 0.5f * x;
    const float hxs = x * hfx;
    const float r1 = 1.0f + hxs * (kQ1 + hxs * (kQ2 + hxs * (kQ3 + hxs * (kQ4 + hxs * kQ5))));
    t = 3.0f - r1 * hfx;
    float e = hxs * ((r1 - t) / (6.0f - x * t));
    if (k == 0) return x - (x * e - hxs);
    e = (x * (e - c) - c);
    e -= hxs;
    if (k == -1) return 0.5f * (x - e) - 0.5f;
    if (k == 1) {
        if (x < -0.25f) return -2.0f * (e - (x + 0.5f));
        return 1.0f + 2.0f * (x - e);
    }
    float y;
    if (k <= -2 || k > 56) {
        y = 1.0f - (e - x);
        y = bits_to_f32(f32_to_bits(y) + (static_cast<uint32_t>(k) << 23));
        return y - 1.0f;
    }
    if (k < 23) {
        t = bits_to_f32(0x3f800000u - (0x1000000u >> k)); // 1 - 2^-k
        y = t - (e - x);
    } else {
        t = bits_to_f32(static_cast<uint32_t>(0x7f - k) << 23); // 2^-k
        y = x - (e + t);
        y += 1.0f;
    }
    return bits_to_f32(f32_to_bits(y) + (static_cast<uint32_t>(k) << 23));
}

// tanhf, fdlibm float version.
__host__ __device__ __forceinline__ float emel_tanhf(float x)
{
    const uint32_t jx = f32_to_bits(x);
    const uint32_t ix = jx & 0x7fffffffu;
    const bool negative = (jx >> 31) != 0;
    float z;
    if (ix >= 0x7f800000u) { // Inf or NaN
        return negative ? 1.0f / x - 1.0f : 1.0f / x + 1.0f;
    }
    if (ix < 0x41b00000u) { // |x| < 22
        if (ix == 0) return x;
        if (ix < 0x24000000u) return x * (1.0f + x); // |x| < 2^-55
        const float ax = bits_to_f32(ix);
        if (ix >= 0x3f800000u) { // |x| >= 1
            const float t = emel_expm1f(2.0f * ax);
            z = 1.0f - 2.0f / (t + 2.0f);
        } else {
            const float t = emel_expm1f(-2.0f * ax);
            z = -t / (t + 2.0f);
        }
    } else {
        z = 1.0f - 1.0e-30f; // 1 with inexact
    }
    return negative ? -z : z;
}

// logf, ARM optimized-routines design (math/logf.c, glibc's logf since
// 2.28).  x = 2^k z with z in [0x1.66p-1, 0x1.66p0) (the offset 0x3f330000
// centres the interval on 1); the top 4 mantissa bits of z pick one of 16
// subintervals with a centre c, stored as invc ~ 1/c (chosen so that
// z * invc - 1 is exact in double) and logc = log(c).  Then
// log(x) = k ln2 + logc + log1p(r), r = z invc - 1, with log1p(r) ~ r + A2 r^2
// + A1 r^3 + A0 r^4 (A0..A2 a minimax fit on the subinterval range),
// evaluated in double and rounded once.  Special inputs: log(1) = 0 exactly,
// log(+-0) = -inf, log(+inf) = +inf, negative or NaN -> NaN, subnormals are
// normalised first.  The reference reaches it through Rust f32::ln
// (emel-logits sampler.rs select step: -uniform.ln()).
static constexpr double kLogfInvc[16] = {
    0x1.661ec79f8f3bep+0, 0x1.571ed4aaf883dp+0, 0x1.49539f0f010bp+0,  0x1.3c995b0b80385p+0,
    0x1.30d190c8864a5p+0, 0x1.25e227b0b8eap+0,  0x1.1bb4a4a1a343fp+0, 0x1.12358f08ae5bap+0,
    0x1.0953f419900a7p+0, 0x1p+0,               0x1.e608cfd9a47acp-1, 0x1.ca4b31f026aap-1,
    0x1.b2036576afce6p-1, 0x1.9c2d163a1aa2dp-1, 0x1.886e6037841edp-1, 0x1.767dcf5534862p-1,
};
static constexpr double kLogfLogc[16] = {
    -0x1.57bf7808caadep-2, -0x1.2bef0a7c06ddbp-2, -0x1.01eae7f513a67p-2, -0x1.b31d8a68224e9p-3,
    -0x1.6574f0ac07758p-3, -0x1.1aa2bc79c81p-3,   -0x1.a4e76ce8c0e5ep-4, -0x1.1973c5a611cccp-4,
    -0x1.252f438e10c1ep-5, 0x0p+0,                0x1.aa5aa5df25984p-5,  0x1.c5e53aa362eb4p-4,
    0x1.526e57720db08p-3,  0x1.bc2860d22477p-3,   0x1.1058bc8a07ee1p-2,  0x1.4043057b6ee09p-2,
};

// `invc` / `logc` are kLogfInvc / kLogfLogc or copies of them (kernels stage
// them in LDS).
__host__ __device__ __forceinline__ float emel_logf(float x, const double *invc = kLogfInvc,
                                                    const double *logc = kLogfLogc)
{
    constexpr double kA0 = -0x1.00ea348b88334p-2;
    constexpr double kA1 = 0x1.5575b0be00b6ap-2;
    constexpr double kA2 = -0x1.ffffef20a4123p-2;
    constexpr double kLn2 = 0x1.62e42fefa39efp-1;
    uint32_t ix = f32_to_bits(x);
    if (ix == 0x3f800000u) return 0.0f;
    if (ix - 0x00800000u >= 0x7f800000u - 0x00800000u) {
        // below the normal range, infinite or NaN
        if (ix * 2u == 0u) return -__builtin_inff();
        if (ix == 0x7f800000u) return x;
        if ((ix & 0x80000000u) || ix * 2u >= 0xff000000u) return (x - x) / (x - x);
        ix = f32_to_bits(x * 0x1p23f); // subnormal: normalise
        ix -= 23u << 23;
    }
    const uint32_t tmp = ix - 0x3f330000u;
    const uint32_t i = (tmp >> (23 - 4)) % 16u;
    const int32_t k = static_cast<int32_t>(tmp) >> 23;
    const uint32_t iz = ix - (tmp & (0x1ffu << 23));
    const double z = static_cast<double>(bits_to_f32(iz));
    const double r = z * invc[i] - 1.0;
    const double y0 = logc[i] + static_cast<double>(k) * kLn2;
    const double r2 = r * r;
    double y = kA1 * r + kA2;
    y = kA0 * r2 + y;
    y = y * r2 + (y0 + r);
    return static_cast<float>(y);
}

// fp32 -> binary16 bits with the reference helper's arithmetic
// (unary.rs:546-570): round to nearest even through a scaled add, NaN -> 0x7e00.
__host__ __device__ __forceinline__ uint16_t emel_fp32_to_fp16(float value)
{
    const float scale_to_inf = bits_to_f32(0x77800000u);  // 2^112
    const float scale_to_zero = bits_to_f32(0x08800000u); // 2^-110
    float base = (__builtin_fabsf(value) * scale_to_inf) * scale_to_zero;
    const uint32_t w = f32_to_bits(value);
    const uint32_t doubled = w + w;
    const uint32_t sign = w & 0x80000000u;
    uint32_t bias = doubled & 0xff000000u;
    if (bias < 0x71000000u) bias = 0x71000000u;
    base += bits_to_f32((bias >> 1) + 0x07800000u);
    const uint32_t bb = f32_to_bits(base);
    const uint32_t nonsign = ((bb >> 13) & 0x7c00u) + (bb & 0x0fffu);
    return static_cast<uint16_t>((sign >> 16) | (doubled > 0xff000000u ? 0x7e00u : nonsign));
}

// binary16 bits -> fp32 (unary.rs:572-586, quant.rs:287-300).
__host__ __device__ __forceinline__ float emel_fp16_to_f32(uint16_t h)
{
    const uint32_t w = static_cast<uint32_t>(h) << 16;
    const uint32_t sign = w & 0x80000000u;
    const uint32_t doubled = w + w;
    const float normalized = bits_to_f32((doubled >> 4) + (0xe0u << 23)) * bits_to_f32(0x07800000u);
    const float denormalized = bits_to_f32((doubled >> 17) | (126u << 23)) - 0.5f;
    return bits_to_f32(sign | f32_to_bits(doubled < (1u << 27) ? denormalized : normalized));
}

// binary16 bits -> fp32 and fp32 -> binary16 bits with the hardware
// conversions (v_cvt_f32_f16 / v_cvt_f16_f32: exact widening and IEEE
// round-to-nearest-even with f16 denormals, the same results as the
// software helpers above over all inputs except NaN payloads; checked
// exhaustively on the GPU by the test suite).
__device__ __forceinline__ float hw_fp16_to_f32(uint16_t h)
{
    return static_cast<float>(__builtin_bit_cast(_Float16, h));
}
__device__ __forceinline__ uint16_t hw_fp32_to_fp16(float x)
{
    return __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
}

// GELU's tanh approximation for an already fp16-rounded input q, rounded
// to fp16 bits (the inner part of GeluFormula, unary.rs:531-539).
__host__ __device__ __forceinline__ uint16_t emel_gelu_core_fp16(float q)
{
    const float inner = 0.7978846f * (q + 0.044715f * q * q * q);
    const float approximation = 0.5f * q * (1.0f + emel_tanhf(inner));
    return emel_fp32_to_fp16(approximation);
}

// SiluFormula (unary.rs:595-600): x / (1 + expf(-x)).  The argument of
// expf is clamped to [-20, 89] and expf's main path evaluated without its
// special-case selects, which gives the same quotient for every x:
//   -x <= 0x1.62e42ep6: the main path is expf (above -20, glibc's main
//   range);
//   -x in (0x1.62e42ep6, 89] and above: the main path's value exceeds
//   FLT_MAX by more than half an ulp and rounds to +inf, expf's overflow
//   result, so x / inf gives -0 (and -inf / inf NaN);
//   -x < -20: expf(-x) < 2^-28, so 1 + expf(-x) rounds to 1 either way;
//   NaN x: the quotient is NaN whatever the clamp returns.
// Checked against glibc over all 2^32 inputs on the host and against the
// select-based expf on the GPU by the test suite.
__host__ __device__ __forceinline__ float silu_exp_arg(float v)
{
#if defined(__HIP_DEVICE_COMPILE__)
    return __builtin_amdgcn_fmed3f(v, -20.0f, 89.0f);
#else
    return __builtin_fminf(__builtin_fmaxf(v, -20.0f), 89.0f);
#endif
}
__host__ __device__ __forceinline__ float emel_silu(float x, const uint64_t *tab, const ExpfConsts &c = ExpfConsts{})
{
    return x / (1.0f + expf_main_path(silu_exp_arg(-x), tab, c));
}

// GeluFormula (unary.rs:522-541): separate products, fp16 round trips on
// the input and the result.
__host__ __device__ __forceinline__ float emel_gelu(float value)
{
    if (value <= -10.0f) return 0.0f;
    if (value >= 10.0f) return value;
    const float q = emel_fp16_to_f32(emel_fp32_to_fp16(value));
    return emel_fp16_to_f32(emel_gelu_core_fp16(q));
}

// ---- GELU by polynomial and table --------------------------------------------
// For |x| < 10 the result depends only on q = fp16(x).  Three ranges of the
// fp16 magnitude m of q, per sign:
//   m below kGeluPolyPos (q >= 0) or kGeluPolyNeg (q < 0), |q| up to about
//   0.26 / 0.30: the result equals fp16(0.5 q (1 + t (1 - t^2/3 + 2 t^4/15)))
//   with t = 0.7978846 (q + 0.044715 q^3), tanh's degree-5 Taylor
//   polynomial, in f32 with the formula's order of operations
//   (gelu_poly).  Each limit is the first magnitude where that fails.
//   saturated: every q >= 3.380859375 (bits 0x42c3) gives exactly q, and
//   every q <= -5.16015625 (bits 0xc529) gives -0.0 (the product underflows
//   fp16);
//   in between: a table of the results, the positive magnitudes from
//   kGeluPolyPos then the negative ones from kGeluPolyNeg, 7918 fp16
//   entries (15.8 KB, small enough for every workgroup to stage in LDS).
// The limits and the whole lookup are checked against emel_gelu over all
// 2^32 inputs by the test suite, which also rescans each polynomial limit.
constexpr uint32_t kGeluPosLimit = 0x42c3u;
constexpr uint32_t kGeluNegLimit = 0x4529u;
constexpr uint32_t kGeluPolyPos = 0x342eu;
constexpr uint32_t kGeluPolyNeg = 0x34d0u;
constexpr uint32_t kGeluPosEntries = kGeluPosLimit - kGeluPolyPos;
constexpr uint32_t kGeluNegEntries = kGeluNegLimit - kGeluPolyNeg;
constexpr uint32_t kGeluEntries = kGeluPosEntries + kGeluNegEntries;
constexpr uint32_t kGeluTableHalfs = (kGeluEntries + 7u) / 8u * 8u; // padded to 16-byte rows

// fp16 bits of the q that table slot `slot` holds the result for.
__host__ __device__ __forceinline__ uint16_t gelu_slot_key(uint32_t slot)
{
    return static_cast<uint16_t>(slot < kGeluPosEntries ? kGeluPolyPos + slot
                                                        : 0x8000u | (kGeluPolyNeg + slot - kGeluPosEntries));
}

// Where the result for fp16 bits h comes from: table slot `slot` (table),
// the polynomial (poly), or else saturation (or NaN).  slot is 0 outside
// the table, so a lookup needs no further select.
struct GeluClass {
    uint32_t slot;
    bool table;
    bool poly;
};
__host__ __device__ __forceinline__ GeluClass gelu_class(uint16_t h)
{
    const uint32_t mag = h & 0x7fffu;
    const bool neg = (h & 0x8000u) != 0;
    const uint32_t lo = neg ? kGeluPolyNeg : kGeluPolyPos;
    const uint32_t rel = mag - lo; // wraps below the table
    const bool table = rel < (neg ? kGeluNegEntries : kGeluPosEntries);
    return GeluClass{table ? rel + (neg ? kGeluPosEntries : 0u) : 0u, table, mag < lo};
}

// The f32 value whose fp16 rounding is GELU(q) for |q| in the polynomial
// range.  On the device the value is passed through an empty asm so that
// the compiler cannot fuse the last product into the fp16 conversion
// (v_fma_mix adds +0.0, which loses the sign of -0 * 1, and rounds the
// product once instead of through f32).
__host__ __device__ __forceinline__ float gelu_poly(float q)
{
    const float t = 0.7978846f * (q + 0.044715f * q * q * q);
    const float t2 = t * t;
    float r = 0.5f * q * (1.0f + t * (1.0f + t2 * (-1.0f / 3.0f + t2 * (2.0f / 15.0f))));
#if defined(__HIP_DEVICE_COMPILE__)
    asm("" : "+v"(r));
#endif
    return r;
}

// GeluFormula from the pieces: x the input, q = fp16(x) widened, c =
// gelu_class of its bits, entry the widened table value at c.slot, poly
// the widened fp16 rounding of gelu_poly(q); each is ignored outside its
// range.
__host__ __device__ __forceinline__ float gelu_finish(float x, float q, GeluClass c, float entry, float poly)
{
    float y = c.table ? entry : (c.poly ? poly : (q < 0.0f ? -0.0f : q));
    if (x <= -10.0f) y = 0.0f;
    if (x >= 10.0f || x != x) y = x;
    return y;
}

// ---- sinf / cosf ---------------------------------------------------------------
//
// ARM optimized-routines sinf / cosf (math/sinf.c, math/cosf.c and
// math/sincosf.h; in glibc since 2.28, whose x86_64 build selects a variant
// compiled with FMA, so every a + b*c of the source is one fused operation
// here).  The argument is widened to double.  |x| < 0x1p-12 returns x (sin)
// or 1 (cos); |x| below 0x1p-1 <= pi/4 (the top-12-bit test) evaluates the
// polynomial directly; |x| < 120 reduces by pi/2 with one fused
// multiply-subtract (the quadrant from a 2^24-scaled 2/pi product and an
// integer shift); larger finite |x| reduce with a 4/pi table of 192 bits and
// a 32x96-bit integer product; infinities and NaN give NaN.  The quadrant
// selects the sine or cosine polynomial and, through a sign table and a
// second coefficient set with the cosine negated, the result's sign.
struct SinCosCoeffs {
    double c0, c1, c2, c3, c4; // cosine: c0 + c1 x^2 + ... (c0 = +1 or -1)
    double s1, s2, s3;         // sine: x + s1 x^3 + s2 x^5 + s3 x^7
};
__host__ __device__ __forceinline__ SinCosCoeffs sincos_coeffs(bool negated_cos)
{
    const double m = negated_cos ? -1.0 : 1.0;
    return SinCosCoeffs{m * 0x1p0, m * -0x1.ffffffd0c621cp-2, m * 0x1.55553e1068f19p-5, m * -0x1.6c087e89a359dp-10,
                        m * 0x1.99343027bf8c3p-16, -0x1.555545995a603p-3, 0x1.1107605230bc4p-7,
                        -0x1.994eb3774cf24p-13};
}

// 4/pi to 192 bits, 8 new bits per entry (entry i holds bits 8i-24 .. 8i+7).
static constexpr uint32_t kInvPio4[24] = {
    0xa2u,       0xa2f9u,     0xa2f983u,   0xa2f9836eu, 0xf9836e4eu, 0x836e4e44u, 0x6e4e4415u, 0x4e441529u,
    0x441529fcu, 0x1529fc27u, 0x29fc2757u, 0xfc2757d1u, 0x2757d1f5u, 0x57d1f534u, 0xd1f534ddu, 0xf534ddc0u,
    0x34ddc0dbu, 0xddc0db62u, 0xc0db6295u, 0xdb629599u, 0x6295993cu, 0x95993c43u, 0x993c4390u, 0x3c439041u,
};

// sinf_poly: the sine polynomial for an even quadrant, the cosine one for an
// odd quadrant; x2 = x*x.
__host__ __device__ __forceinline__ float sincosf_poly(double x, double x2, const SinCosCoeffs &p, int n)
{
    if ((n & 1) == 0) {
        const double x3 = x * x2;
        const double s1 = __builtin_fma(x2, p.s3, p.s2);
        const double x7 = x3 * x2;
        const double s = __builtin_fma(x3, p.s1, x);
        return static_cast<float>(__builtin_fma(x7, s1, s));
    }
    const double x4 = x2 * x2;
    const double c2 = __builtin_fma(x2, p.c4, p.c3);
    const double c1 = __builtin_fma(x2, p.c1, p.c0);
    const double x6 = x4 * x2;
    const double c = __builtin_fma(x4, p.c2, c1);
    return static_cast<float>(__builtin_fma(x6, c2, c));
}

__host__ __device__ __forceinline__ uint32_t abstop12(float x) { return (f32_to_bits(x) >> 20) & 0x7ffu; }

// |x| < 120: x - n*pi/2 with n the nearest quadrant (2/pi prescaled by 2^24).
__host__ __device__ __forceinline__ double sincosf_reduce_fast(double x, int &n)
{
    const double r = x * 0x1.45F306DC9C883p+23;
    n = (static_cast<int32_t>(r) + 0x800000) >> 24;
    return __builtin_fma(-static_cast<double>(n), 0x1.921FB54442D18p0, x);
}

// Finite |x| >= 120 (bits xi, sign ignored): the exact 2.62 fixed-point
// product with 4/pi, rounded to the nearest quadrant.
__host__ __device__ __forceinline__ double sincosf_reduce_large(uint32_t xi, int &np)
{
    const uint32_t *arr = &kInvPio4[(xi >> 26) & 15u];
    const int shift = static_cast<int>((xi >> 23) & 7u);
    xi = (xi & 0xffffffu) | 0x800000u;
    xi <<= shift;
    uint64_t res0 = static_cast<uint32_t>(xi * arr[0]); // low 32 bits only
    const uint64_t res1 = static_cast<uint64_t>(xi) * arr[4];
    const uint64_t res2 = static_cast<uint64_t>(xi) * arr[8];
    res0 = (res2 >> 32) | (res0 << 32);
    res0 += res1;
    const uint64_t n = (res0 + (uint64_t{1} << 61)) >> 62;
    res0 -= n << 62;
    np = static_cast<int>(n);
    return static_cast<double>(static_cast<int64_t>(res0)) * 0x1.921FB54442D18p-62; // 2 pi 2^-64
}

// want_cos selects cosf; sinf otherwise.
__host__ __device__ __forceinline__ float emel_sincosf(float y, bool want_cos)
{
    // the quadrant sign table {1, -1, -1, 1}, without an indexed array
    auto quadrant_sign = [](int q) { return ((q + 1) & 2) ? -1.0 : 1.0; };
    const uint32_t top = abstop12(y);
    double x = static_cast<double>(y);
    if (top < abstop12(0x1.921FB6p-1f)) {
        if (top < abstop12(0x1p-12f)) return want_cos ? 1.0f : y;
        return sincosf_poly(x, x * x, sincos_coeffs(false), want_cos ? 1 : 0);
    }
    if (top < abstop12(120.0f)) {
        int n;
        x = sincosf_reduce_fast(x, n);
        const double s = quadrant_sign(n);
        return sincosf_poly(x * s, x * x, sincos_coeffs((n & 2) != 0), want_cos ? n ^ 1 : n);
    }
    if (top < abstop12(__builtin_inff())) {
        const uint32_t xi = f32_to_bits(y);
        const int sign = static_cast<int>(xi >> 31);
        int n;
        x = sincosf_reduce_large(xi, n);
        const double s = quadrant_sign(n + sign);
        return sincosf_poly(x * s, x * x, sincos_coeffs(((n + sign) & 2) != 0), want_cos ? n ^ 1 : n);
    }
    return (y - y) / (y - y); // NaN for infinities and NaN
}

__host__ __device__ __forceinline__ float emel_sinf(float x) { return emel_sincosf(x, false); }
__host__ __device__ __forceinline__ float emel_cosf(float x) { return emel_sincosf(x, true); }

// ---- log1pf --------------------------------------------------------------------
//
// fdlibm s_log1pf.c (glibc sysdeps/ieee754/flt-32, not contracted): 1 + x =
// 2^k (1 + f) with a correction term c for the rounding of 1 + x, then
// log(1 + f) = f - hfsq + s (hfsq + R(s^2)), s = f / (2 + f), in float.
__host__ __device__ __forceinline__ float emel_log1pf(float x)
{
    constexpr float kLn2Hi = 6.9313812256e-01f; // 0x3f317180
    constexpr float kLn2Lo = 9.0580006145e-06f; // 0x3717f7d1
    constexpr float kTwo25 = 3.355443200e+07f;  // 0x4c000000
    constexpr float kLp1 = 6.6666668653e-01f;   // 0x3f2aaaab
    constexpr float kLp2 = 4.0000000596e-01f;   // 0x3ecccccd
    constexpr float kLp3 = 2.8571429849e-01f;   // 0x3e924925
    constexpr float kLp4 = 2.2222198546e-01f;   // 0x3e638e29
    constexpr float kLp5 = 1.8183572590e-01f;   // 0x3e3a3325
    constexpr float kLp6 = 1.5313838422e-01f;   // 0x3e1cd04f
    constexpr float kLp7 = 1.4798198640e-01f;   // 0x3e178897
    const int32_t hx = static_cast<int32_t>(f32_to_bits(x));
    const int32_t ax = hx & 0x7fffffff;
    int32_t k = 1, hu = 0;
    float f = 0.0f, c = 0.0f;
    if (hx < 0x3ed413d7) {       // x < 0.41422
        if (ax >= 0x3f800000) {  // x <= -1
            if (x == -1.0f) return -kTwo25 / (x - x); // -inf
            return (x - x) / (x - x);                  // NaN
        }
        if (ax < 0x31000000) {   // |x| < 2^-29
            if (ax < 0x24800000) return x;
            return x - x * x * 0.5f;
        }
        if (hx > 0 || hx <= static_cast<int32_t>(0xbe95f61fu)) { // -0.2929 < x < 0.41422
            k = 0;
            f = x;
            hu = 1;
        }
    } else if (hx >= 0x7f800000) {
        return x + x;
    }
    if (k != 0) {
        float u;
        if (hx < 0x5a000000) {
            u = 1.0f + x;
            hu = static_cast<int32_t>(f32_to_bits(u));
            k = (hu >> 23) - 127;
            c = (k > 0) ? 1.0f - (u - x) : x - (u - 1.0f); // correction term
            c /= u;
        } else {
            u = x;
            hu = static_cast<int32_t>(f32_to_bits(u));
            k = (hu >> 23) - 127;
            c = 0.0f;
        }
        hu &= 0x007fffff;
        if (hu < 0x3504f7) {
            u = bits_to_f32(static_cast<uint32_t>(hu) | 0x3f800000u); // normalize u
        } else {
            k += 1;
            u = bits_to_f32(static_cast<uint32_t>(hu) | 0x3f000000u); // normalize u/2
            hu = (0x00800000 - hu) >> 2;
        }
        f = u - 1.0f;
    }
    const float hfsq = 0.5f * f * f;
    const float fk = static_cast<float>(k);
    if (hu == 0) { // |f| < 2^-20
        if (f == 0.0f) {
            if (k == 0) return 0.0f;
            c += fk * kLn2Lo;
            return fk * kLn2Hi + c;
        }
        const float R = hfsq * (1.0f - 0.66666666666666666f * f);
        if (k == 0) return f - R;
        return fk * kLn2Hi - ((R - (fk * kLn2Lo + c)) - f);
    }
    const float s = f / (2.0f + f);
    const float z = s * s;
    const float R = z * (kLp1 + z * (kLp2 + z * (kLp3 + z * (kLp4 + z * (kLp5 + z * (kLp6 + z * kLp7))))));
    if (k == 0) return f - (hfsq - s * (hfsq + R));
    return fk * kLn2Hi - ((hfsq - (s * (hfsq + R) + (fk * kLn2Lo + c))) - f);
}

} // namespace emel
