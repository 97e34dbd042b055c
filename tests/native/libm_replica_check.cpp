// libm_replica_check.cpp -- test helper (built by __graft_entry__.build()).
//
// Compiles the product's device math (emel.rs_amd/csrc/libm_replica.hpp) for
// the host CPU and counts, over a range of f32 bit patterns, the inputs on
// which it differs from an independent checker:
//   expf / expm1f / tanhf / logf / sinf / cosf / log1pf
//                          -> the host glibc (what Rust std calls, and so
//                             what the reference's CPU path computes);
//   fp32 -> fp16           -> the compiler's _Float16 conversion (IEEE
//                             round-to-nearest-even);
//   fp16 -> fp32           -> the compiler's _Float16 widening (exact);
//   silu                   -> x / (1 + glibc expf(-x)) (the kernels' form
//                             clamps expf's argument instead of selecting
//                             its special cases);
//   GELU by polynomial and table -> the scalar formula, and each
//                             polynomial limit rescanned;
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

// The sampler's exact sum (sampler.hip: k_smp_seg + k_smp_sum) on the host.
struct EmuState {
    uint32_t m = 0;
    int32_t u = -149;
    bool finite = true;
    float special = 0.0f;
};

// One tile of `tile` elements through k_smp_sum's rounds: a round commits the
// rest of the tile when no element is an event, else commits up to the
// first event and adds that element with one f32 addition.  Exact
// (unsaturated) prefix sums.
static void emu_tile(const float *ev, uint64_t tile, EmuState &s, std::vector<uint32_t> &r,
                     std::vector<uint8_t> &tie)
{
    if (!s.finite) {
        for (uint64_t i = 0; i < tile; ++i)
            if (std::isnan(ev[i])) s.special = std::nanf("");
        return;
    }
    uint64_t start = 0;
    while (true) {
        uint64_t total = 0;
        bool anytie = false;
        for (uint64_t i = 0; i < tile; ++i) {
            bool t;
            const uint32_t q = emel::seq_units(ev[i], s.u, t);
            r[i] = i >= start ? q : 0u;
            tie[i] = i >= start && t;
            total += r[i];
            anytie |= tie[i] != 0;
        }
        if (!anytie && s.m + total < emel::kSeqLimit) {
            s.m += static_cast<uint32_t>(total);
            return;
        }
        uint64_t run = s.m, k = tile;
        for (uint64_t i = start; i < tile; ++i) {
            if (tie[i] || run + r[i] >= emel::kSeqLimit) {
                k = i;
                break;
            }
            run += r[i];
        }
        if (k == tile) { // cannot happen: flag it
            s.finite = false;
            s.special = std::nanf("0x7e57");
            return;
        }
        const float sn = emel::seq_value(static_cast<uint32_t>(run), s.u) + ev[k];
        if (!(sn < INFINITY)) {
            s.special = sn;
            s.finite = false;
            for (uint64_t i = k + 1; i < tile; ++i)
                if (std::isnan(ev[i])) s.special = std::nanf("");
            return;
        }
        const emel::SeqState st = emel::seq_state(sn);
        s.m = st.m;
        s.u = st.u;
        start = k + 1;
        if (start >= tile) return;
    }
}

// Walks [c0, c1) in tiles of lanes * 16 elements (k_smp_sum: 64 lanes).
// At the start of a row the first `head` elements are added one by one.
static void emu_walk(const float *e, uint64_t c0, uint64_t c1, uint32_t lanes, EmuState &s, uint64_t head = 512)
{
    const uint64_t tile = 16ull * lanes;
    std::vector<float> ev(tile);
    std::vector<uint32_t> r(tile);
    std::vector<uint8_t> tie(tile);
    uint64_t skip = 0;
    if (c0 == 0 && s.finite && s.m == 0) {
        skip = std::min(head, c1 - c0);
        float acc = emel::seq_value(s.m, s.u);
        for (uint64_t i = 0; i < skip; ++i) acc += e[c0 + i];
        if (!(acc < INFINITY)) {
            s.finite = false;
            s.special = acc;
        } else {
            const emel::SeqState h = emel::seq_state(acc);
            s.m = h.m;
            s.u = h.u;
        }
    }
    for (uint64_t base = c0; base < c1; base += tile) {
        for (uint64_t i = 0; i < tile; ++i) ev[i] = base + i < c1 && base + i >= c0 + skip ? e[base + i] : 0.0f;
        emu_tile(ev.data(), tile, s, r, tie);
    }
}

static uint64_t splitmix(uint64_t &z);

// chunk == 0: the whole range is walked (no predictions).  Otherwise
// chunks of `chunk` elements split into sub-chunks of `sub`: k_smp_seg's
// prediction per sub-chunk (f64 prefix of chunk and sub-chunk sums, the
// rounding bound, units at the predicted binade or at both of two adjacent
// ones, one tie resolved by
// parity) and k_smp_sum's checks on the exact state; a sub-chunk that is
// not taken is walked alone.  *jumped counts sub-chunks taken in one step.
// perturb > 0 stands in for k_smp_expseg's approximate sums: the prefix and
// the sub-chunk's sum each scaled by a random factor in [1 - perturb,
// 1 + perturb], the bounds widened by `widen` (the kernel's kApproxRel).
float seqsum_chunked(const float *e, uint64_t n, uint32_t lanes, uint64_t chunk, uint64_t sub, uint64_t *jumped,
                     double perturb = 0.0, double widen = 0.0, uint64_t seed = 0)
{
    uint64_t z = seed;
    auto jitter = [&]() {
        return perturb > 0.0 ? 1.0 + perturb * (2.0 * static_cast<double>(splitmix(z) >> 11) * 0x1p-53 - 1.0) : 1.0;
    };
    EmuState s;
    if (jumped) *jumped = 0;
    if (chunk == 0) {
        emu_walk(e, 0, n, lanes, s);
        return s.finite ? emel::seq_value(s.m, s.u) : s.special;
    }
    double pre = 0.0;
    for (uint64_t c0 = 0; c0 < n; c0 += chunk) {
        const uint64_t c1 = std::min(n, c0 + chunk);
        double Pk = pre;
        for (uint64_t a0 = c0; a0 < c1; a0 += sub) {
            const uint64_t a1 = std::min(c1, a0 + sub);
            double ssum = 0.0;
            for (uint64_t i = a0; i < a1; ++i) ssum += static_cast<double>(e[i]);
            const double pe = Pk * jitter(), se = ssum * jitter();
            const double lo = pe * (1.0 - widen) * (1.0 - (static_cast<double>(a0) * 0x1p-24 + 0x1p-30));
            const double hi = (pe + se) * (1.0 + widen) * (1.0 + (static_cast<double>(a1) * 0x1p-24 + 0x1p-30));
            Pk += ssum;
            int elo = 0, ehi = 0;
            std::frexp(lo, &elo);
            std::frexp(hi, &ehi);
            // one binade, or two adjacent ones: a count at each
            const bool usable = lo >= 0x1p-126 && hi < 0x1p127 && lo <= hi && ehi - elo <= 1;
            // the count at the state's binade, when it is one of them
            const int32_t u = s.u == elo - 24 + 1 && ehi != elo ? elo - 24 + 1 : elo - 24;
            bool ok = usable;
            uint64_t units = 0;
            int ties = 0;
            uint32_t par = 0;
            if (ok) {
                for (uint64_t i = a0; i < a1; ++i) {
                    bool t;
                    uint32_t q = emel::seq_units(e[i], u, t);
                    if (t) {
                        q = static_cast<uint32_t>(std::floor(std::ldexp(e[i], -u)));
                        if (ties == 0) par = static_cast<uint32_t>((units + q) & 1u);
                        ++ties;
                    }
                    units += q;
                }
                if (ties > 1) ok = false;
            }
            const uint64_t add = units + (ties == 1 ? ((s.m + par) & 1u) : 0u);
            if (s.finite && ok && u == s.u && s.m + add < emel::kSeqLimit) {
                s.m += static_cast<uint32_t>(add);
                if (jumped) ++*jumped;
                continue;
            }
            if (!s.finite && std::isnan(s.special)) break;
            emu_walk(e, a0, a1, lanes, s);
        }
        pre = Pk;
    }
    return s.finite ? emel::seq_value(s.m, s.u) : s.special;
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

extern "C" float seqsum_chunked_f(const float *e, uint64_t n, uint32_t lanes, uint64_t chunk, uint64_t sub,
                                  uint64_t *jumped)
{
    return seqsum_chunked(e, n, lanes, chunk, sub, jumped);
}

extern "C" float seqsum_approx_f(const float *e, uint64_t n, uint32_t lanes, uint64_t chunk, uint64_t sub,
                                 double perturb, double widen, uint64_t seed, uint64_t *jumped)
{
    return seqsum_chunked(e, n, lanes, chunk, sub, jumped, perturb, widen, seed);
}

// check_seqsum's families through the predictions with perturbed prefixes
// (config 5's chunk shapes): counts results whose bits differ from the
// sequential loop.
extern "C" uint64_t check_seqsum_approx(uint64_t seed, int cases, uint64_t max_n, double perturb, double widen)
{
    uint64_t z = seed, bad = 0;
    for (int c = 0; c < cases; ++c) {
        const int family = c % 5;
        const uint64_t n = 1 + splitmix(z) % max_n;
        std::vector<float> e(n);
        fill_case(z, family, e);
        float want = 0.0f;
        for (float v : e) want += v;
        for (const uint64_t chunk : {5120ull, 1024ull})
            if (differ(seqsum_chunked(e.data(), n, 32, chunk, 512, nullptr, perturb, widen, splitmix(z)), want)) ++bad;
    }
    return bad;
}

// Random cases of each family and length up to max_n, through the walk
// alone (tiles of 64 x 16 and 4 x 16 elements) and through sub-chunk
// predictions (config 5's 5120-element chunks of 512-element sub-chunks,
// walked in tiles of 512 as the kernel does, 4748-element chunks of
// 1024-element sub-chunks, and small shapes).  Counts results whose bits differ from the sequential
// loop.
extern "C" uint64_t check_seqsum(uint64_t seed, int cases, uint64_t max_n)
{
    uint64_t z = seed, bad = 0;
    const uint64_t shapes[7][3] = {{64, 0, 0}, {4, 0, 0}, {64, 4748, 1024}, {4, 100, 64}, {64, 1024, 1024},
                                   {4, 300, 300}, {32, 5120, 512}};
    for (int c = 0; c < cases; ++c) {
        const int family = c % 5;
        const uint64_t n = 1 + splitmix(z) % max_n;
        std::vector<float> e(n);
        fill_case(z, family, e);
        float want = 0.0f;
        for (float v : e) want += v;
        for (const auto &sh : shapes) {
            const float got = seqsum_chunked(e.data(), n, static_cast<uint32_t>(sh[0]), sh[1], sh[2], nullptr);
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

uint64_t check_sinf(uint64_t lo, uint64_t hi, int threads)
{
    return count_range(lo, hi, threads, [](uint32_t u) {
        const float x = emel::bits_to_f32(u);
        return differ(emel::emel_sinf(x), sinf(x));
    });
}

uint64_t check_cosf(uint64_t lo, uint64_t hi, int threads)
{
    return count_range(lo, hi, threads, [](uint32_t u) {
        const float x = emel::bits_to_f32(u);
        return differ(emel::emel_cosf(x), cosf(x));
    });
}

uint64_t check_log1pf(uint64_t lo, uint64_t hi, int threads)
{
    return count_range(lo, hi, threads, [](uint32_t u) {
        const float x = emel::bits_to_f32(u);
        return differ(emel::emel_log1pf(x), log1pf(x));
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

// The table-driven GELU of the kernels (gelu_class / gelu_finish over a
// table filled like k_gelu_table) against emel_gelu for every input in
// [lo, hi).  Also counts table slots whose key maps back to another slot.
uint64_t check_gelu_table(uint64_t lo, uint64_t hi, int threads)
{
    std::vector<uint16_t> tab(emel::kGeluTableHalfs, 0);
    uint64_t bad = 0;
    for (uint32_t slot = 0; slot < emel::kGeluEntries; ++slot) {
        const uint16_t key = emel::gelu_slot_key(slot);
        const emel::GeluClass c = emel::gelu_class(key);
        if (!c.table || c.poly || c.slot != slot) ++bad;
        tab[slot] = emel::emel_gelu_core_fp16(emel::emel_fp16_to_f32(key));
    }
    const uint16_t *t = tab.data();
    return bad + count_range(lo, hi, threads, [t](uint32_t u) {
        const float x = emel::bits_to_f32(u);
        const uint16_t h = emel::emel_fp32_to_fp16(x);
        const float q = emel::emel_fp16_to_f32(h);
        const emel::GeluClass c = emel::gelu_class(h);
        const float entry = emel::emel_fp16_to_f32(t[c.slot]);
        const float poly = emel::emel_fp16_to_f32(emel::emel_fp32_to_fp16(emel::gelu_poly(q)));
        return differ(emel::gelu_finish(x, q, c, entry, poly), emel::emel_gelu(x));
    });
}

// The first fp16 magnitude (of sign `negative`) at which fp16(gelu_poly(q))
// differs from GeluFormula's core, scanning up from 0: the polynomial's
// range ends exactly there (kGeluPolyPos / kGeluPolyNeg).
uint32_t gelu_poly_first_miss(int negative)
{
    for (uint32_t mag = 0; mag < 0x7c00u; ++mag) {
        const uint16_t h = static_cast<uint16_t>((negative ? 0x8000u : 0u) | mag);
        const float q = emel::emel_fp16_to_f32(h);
        if (emel::emel_fp32_to_fp16(emel::gelu_poly(q)) != emel::emel_gelu_core_fp16(q)) return mag;
    }
    return 0x7c00u;
}
uint32_t gelu_poly_limit(int negative) { return negative ? emel::kGeluPolyNeg : emel::kGeluPolyPos; }

// emel_silu (clamped argument, expf's main path without its special-case
// selects) against SiluFormula on the host glibc, x / (1 + expf(-x)).
uint64_t check_silu(uint64_t lo, uint64_t hi, int threads)
{
    return count_range(lo, hi, threads, [](uint32_t u) {
        const float x = emel::bits_to_f32(u);
        return differ(emel::emel_silu(x, emel::kExp2Table), x / (1.0f + expf(-x)));
    });
}

// Scalar values for the golden-vector tests (unary manifest inputs).
float replica_silu(float x) { return emel::emel_silu(x, emel::kExp2Table); }
float replica_gelu(float x) { return emel::emel_gelu(x); }
float replica_expf(float x) { return emel::emel_expf(x, emel::kExp2Table); }
float replica_tanhf(float x) { return emel::emel_tanhf(x); }

} // extern "C"
