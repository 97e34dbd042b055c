// libm_replica_check.cpp -- test helper (built by __graft_entry__.build()).
//
// Compiles the product's device math (emel.rs_amd/csrc/libm_replica.hpp) for
// the host CPU and counts, over a range of f32 bit patterns, the inputs on
// which it differs from an independent checker:
//   expf / expm1f / tanhf / logf
//                          -> the host glibc (what Rust std calls, and so
//                             what the reference's CPU path computes);
//   fp32 -> fp16           -> the compiler's _Float16 conversion (IEEE
//                             round-to-nearest-even);
//   fp16 -> fp32           -> the compiler's _Float16 widening (exact);
//   seqsum.hpp             -> a plain sequential f32 loop: the host
//                             emulation of k_smp_sum's rounds (units per
//                             binade, events, restarts) must give its bits.
// NaN results count as equal when both are NaN.  Ranges are split over
// `threads` threads.
#include "libm_replica.hpp"
#include "seqsum.hpp"

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

// The round structure of k_smp_sum (sampler.hip) on the host: tiles of
// threads * per elements; a round commits the rest of the tile when no
// element is an event, else commits up to the first event and adds that
// element with one f32 addition.  Exact (unsaturated) prefix sums.
// per == 0 selects k_smp_sum's schedule: tiles of threads * {1, 2, 4, 8}
// elements, then threads * 16 to the end.
float seqsum_blocked(const float *e, uint64_t n, uint32_t threads, uint32_t per)
{
    uint32_t m = 0;
    int32_t u = -149;
    bool finite = true;
    float special = 0.0f;
    const uint64_t max_tile = static_cast<uint64_t>(threads) * (per ? per : 16);
    std::vector<float> ev(max_tile);
    std::vector<uint32_t> r(max_tile);
    std::vector<uint8_t> tie(max_tile);
    uint32_t warm = 0;
    for (uint64_t base = 0, tile = 0; base < n; base += tile) {
        tile = static_cast<uint64_t>(threads) * (per ? per : (warm < 4 ? (1u << warm) : 16u));
        ++warm;
        for (uint64_t i = 0; i < tile; ++i) ev[i] = base + i < n ? e[base + i] : 0.0f;
        if (!finite) {
            for (uint64_t i = 0; i < tile; ++i)
                if (std::isnan(ev[i])) special = std::nanf("");
            continue;
        }
        uint64_t start = 0;
        while (true) {
            uint64_t total = 0;
            bool anytie = false;
            for (uint64_t i = 0; i < tile; ++i) {
                bool t;
                const uint32_t q = emel::seq_units(ev[i], u, t);
                r[i] = i >= start ? q : 0u;
                tie[i] = i >= start && t;
                total += r[i];
                anytie |= tie[i] != 0;
            }
            if (!anytie && m + total < emel::kSeqLimit) {
                m += static_cast<uint32_t>(total);
                break;
            }
            uint64_t run = m, k = tile;
            for (uint64_t i = start; i < tile; ++i) {
                if (tie[i] || run + r[i] >= emel::kSeqLimit) {
                    k = i;
                    break;
                }
                run += r[i];
            }
            if (k == tile) return std::nanf("0x7e57"); // cannot happen: flag it
            const float sn = emel::seq_value(static_cast<uint32_t>(run), u) + ev[k];
            if (!(sn < INFINITY)) {
                special = sn;
                finite = false;
                for (uint64_t i = k + 1; i < tile; ++i)
                    if (std::isnan(ev[i])) special = std::nanf("");
                break;
            }
            const emel::SeqState st = emel::seq_state(sn);
            m = st.m;
            u = st.u;
            start = k + 1;
            if (start >= tile) break;
        }
    }
    return finite ? emel::seq_value(m, u) : special;
}

static uint64_t splitmix(uint64_t &z)
{
    uint64_t x = (z += 0x9e3779b97f4a7c15ull);
    x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ull;
    x = (x ^ (x >> 27)) * 0x94d049bb133111ebull;
    return x ^ (x >> 31);
}

// Addend families: 0 softmax-like (expf of N(0,2) - 8, mostly < 1),
// 1 dyadic values k * 2^j (many exact ties), 2 tiny and subnormal values
// with zeros, 3 values of every magnitude up to 2^30, 4 family 0 with one
// NaN or +inf planted.
static void fill_case(uint64_t &z, int family, std::vector<float> &e)
{
    for (float &v : e) {
        const uint64_t x = splitmix(z);
        switch (family) {
        case 0:
        case 4: {
            const double u1 = ((x >> 11) + 0.5) * 0x1p-53, u2 = (splitmix(z) >> 11) * 0x1p-53;
            const double g = std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
            v = expf(static_cast<float>(2.0 * g - 8.0));
            break;
        }
        case 1: v = std::ldexp(static_cast<float>(x % 17), -static_cast<int>((x >> 8) % 40)); break;
        case 2: v = (x & 3) == 0 ? 0.0f : emel::bits_to_f32(static_cast<uint32_t>((x >> 8) % 0x01000000u)); break;
        default: v = std::ldexp(static_cast<float>((x >> 40) | 1), static_cast<int>((x >> 8) % 60) - 54); break;
        }
    }
    if (family == 4 && !e.empty()) {
        const uint64_t x = splitmix(z);
        e[x % e.size()] = (x >> 63) ? std::nanf("") : INFINITY;
    }
}

extern "C" float seqsum_blocked_f(const float *e, uint64_t n, uint32_t threads, uint32_t per)
{
    return seqsum_blocked(e, n, threads, per);
}

// Random cases of each family and length up to max_n; tile shapes
// (threads, per) of the kernel (1024, 16) and small ones that force many
// rounds.  Counts results whose bits differ from the sequential loop.
extern "C" uint64_t check_seqsum(uint64_t seed, int cases, uint64_t max_n)
{
    uint64_t z = seed, bad = 0;
    const uint32_t shapes[4][2] = {{1024, 0}, {1024, 16}, {4, 2}, {64, 1}};
    for (int c = 0; c < cases; ++c) {
        const int family = c % 5;
        const uint64_t n = 1 + splitmix(z) % max_n;
        std::vector<float> e(n);
        fill_case(z, family, e);
        float want = 0.0f;
        for (float v : e) want += v;
        for (const auto &sh : shapes) {
            const float got = seqsum_blocked(e.data(), n, sh[0], sh[1]);
            if (differ(got, want)) ++bad;
        }
    }
    return bad;
}

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

uint64_t check_logf(uint64_t lo, uint64_t hi, int threads)
{
    return count_range(lo, hi, threads, [](uint32_t u) {
        const float x = emel::bits_to_f32(u);
        return differ(emel::emel_logf(x), logf(x));
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
