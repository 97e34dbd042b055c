// libm_replica_check.cpp -- test helper (built by __graft_entry__.build()).
//
// Compiles the product's device math (emel.rs_amd/csrc/libm_replica.hpp) for
// the host CPU and counts, over a range of f32 bit patterns, the inputs on
// which it differs from an independent checker:
//   expf / expm1f / tanhf  -> the host glibc (what Rust std calls, and so
//                             what the reference's CPU path computes);
//   fp32 -> fp16           -> the compiler's _Float16 conversion (IEEE
//                             round-to-nearest-even);
//   fp16 -> fp32           -> the compiler's _Float16 widening (exact).
// NaN results count as equal when both are NaN.  Ranges are split over
// `threads` threads.
#include "libm_replica.hpp"

#include <cmath>
#include <cstdint>
#include <thread>
#include <vector>

namespace {

template <class F>
uint64_t count_range(uint64_t lo, uint64_t hi, int threads, F mismatch)
{
    if (threads < 1) threads = 1;
    std::vector<uint64_t> bad(threads, 0);
    std::vector<std::thread> pool;
    for (int t = 0; t < threads; ++t) {
        pool.emplace_back([=, &bad] {
            uint64_t local = 0;
            for (uint64_t u = lo + t; u < hi; u += threads) local += mismatch(static_cast<uint32_t>(u)) ? 1 : 0;
            bad[t] = local;
        });
    }
    for (auto &th : pool) th.join();
    uint64_t total = 0;
    for (uint64_t b : bad) total += b;
    return total;
}

bool differ(float a, float b)
{
    if (std::isnan(a) && std::isnan(b)) return false;
    return emel::f32_to_bits(a) != emel::f32_to_bits(b);
}

} // namespace

extern "C" {

uint64_t check_expf(uint64_t lo, uint64_t hi, int threads)
{
    return count_range(lo, hi, threads, [](uint32_t u) {
        const float x = emel::bits_to_f32(u);
        return differ(emel::emel_expf(x, emel::kExp2Table), expf(x));
    });
}

uint64_t check_expm1f(uint64_t lo, uint64_t hi, int threads)
{
    return count_range(lo, hi, threads, [](uint32_t u) {
        const float x = emel::bits_to_f32(u);
        return differ(emel::emel_expm1f(x), expm1f(x));
    });
}

uint64_t check_tanhf(uint64_t lo, uint64_t hi, int threads)
{
    return count_range(lo, hi, threads, [](uint32_t u) {
        const float x = emel::bits_to_f32(u);
        return differ(emel::emel_tanhf(x), tanhf(x));
    });
}

uint64_t check_fp32_to_fp16(uint64_t lo, uint64_t hi, int threads)
{
    return count_range(lo, hi, threads, [](uint32_t u) {
        const float x = emel::bits_to_f32(u);
        const uint16_t got = emel::emel_fp32_to_fp16(x);
        if (std::isnan(x)) return got != static_cast<uint16_t>(((u >> 16) & 0x8000u) | 0x7e00u);
        const _Float16 h = static_cast<_Float16>(x);
        return got != __builtin_bit_cast(uint16_t, h);
    });
}

uint64_t check_fp16_to_f32(void)
{
    return count_range(0, 65536, 1, [](uint32_t u) {
        const uint16_t h = static_cast<uint16_t>(u);
        const float want = static_cast<float>(__builtin_bit_cast(_Float16, h));
        return differ(emel::emel_fp16_to_f32(h), want);
    });
}

// div_by_recip(a, 1/b) against IEEE a / b: every a bit pattern in [lo, hi)
// for each of the nb divisors bs[] (normal, >= 1).
uint64_t check_div_recip(const float *bs, int nb, uint64_t lo, uint64_t hi, int threads)
{
    uint64_t total = 0;
    for (int i = 0; i < nb; ++i) {
        const float b = bs[i];
        const double r = 1.0 / static_cast<double>(b);
        total += count_range(lo, hi, threads, [b, r](uint32_t u) {
            const float a = emel::bits_to_f32(u);
            return differ(emel::div_by_recip(a, r), a / b);
        });
    }
    return total;
}

// Random pairs: a any f32 bit pattern, b any f32 in [1, 2^64).
uint64_t check_div_recip_random(uint64_t seed, uint64_t n, int threads)
{
    return count_range(0, n, threads, [seed](uint32_t i) {
        uint64_t z = seed + 0x9e3779b97f4a7c15ull * (static_cast<uint64_t>(i) + 1);
        z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
        z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
        z ^= z >> 31;
        const float a = emel::bits_to_f32(static_cast<uint32_t>(z));
        const float b = emel::bits_to_f32(0x3f800000u + static_cast<uint32_t>((z >> 32) % (64u << 23)));
        return differ(emel::div_by_recip(a, 1.0 / static_cast<double>(b)), a / b);
    });
}

// The table-driven GELU of the kernels (gelu_slot / gelu_finish over a
// table filled like k_gelu_table) against emel_gelu for every input in
// [lo, hi).  Also counts table slots whose key maps back to another slot.
uint64_t check_gelu_table(uint64_t lo, uint64_t hi, int threads)
{
    std::vector<uint16_t> tab(emel::kGeluTableHalfs, 0);
    uint64_t bad = 0;
    for (uint32_t slot = 0; slot < emel::kGeluEntries; ++slot) {
        const uint16_t key = emel::gelu_slot_key(slot);
        if (emel::gelu_slot(key) != slot) ++bad;
        tab[slot] = emel::emel_gelu_core_fp16(emel::emel_fp16_to_f32(key));
    }
    const uint16_t *t = tab.data();
    return bad + count_range(lo, hi, threads, [t](uint32_t u) {
        const float x = emel::bits_to_f32(u);
        const uint16_t h = emel::emel_fp32_to_fp16(x);
        const uint32_t slot = emel::gelu_slot(h);
        const float entry = emel::emel_fp16_to_f32(t[slot < emel::kGeluEntries ? slot : 0u]);
        return differ(emel::gelu_finish(x, emel::emel_fp16_to_f32(h), slot, entry), emel::emel_gelu(x));
    });
}

// Scalar values for the golden-vector tests (unary manifest inputs).
float replica_silu(float x) { return emel::emel_silu(x, emel::kExp2Table); }
float replica_gelu(float x) { return emel::emel_gelu(x); }
float replica_expf(float x) { return emel::emel_expf(x, emel::kExp2Table); }
float replica_tanhf(float x) { return emel::emel_tanhf(x); }

} // extern "C"
