// gpu_checks.hip -- test helper (built by __graft_entry__.build()).
//
// Exhaustive GPU checks of the device-side shortcuts the kernels take,
// against the reference-restating code they replace:
//   hw_fp32_to_fp16 vs emel_fp32_to_fp16  (all 2^32 f32 inputs)
//   hw_fp16_to_f32  vs emel_fp16_to_f32   (all 65536 f16 inputs)
//   emel_expf_nonpos vs emel_expf         (all f32 <= 0, and NaNs)
//   emel_silu vs x / (1 + emel_expf(-x))  (all 2^32 f32 inputs)
//   the kernels' GELU lookup vs emel_gelu (all 2^32 f32 inputs)
//   __builtin_sqrtf (the power.rs kernels) correctly rounded: for every
//   positive finite x the exact squares of the two rounding midpoints
//   around the result bracket x (exact in double: <= 52 significant bits);
//   sqrt(+-0) = +-0, sqrt(+inf) = +inf, negatives and NaN give NaN
// NaN results match NaN results.  Each entry point launches a grid-stride
// kernel over the range on the null stream, waits, and returns the number
// of mismatching inputs (or UINT64_MAX on a HIP error).
#include <hip/hip_runtime.h>

#include <cstdint>

#include "libm_replica.hpp"

namespace {

__device__ unsigned long long g_bad;

__device__ __forceinline__ bool nan16(uint16_t h) { return (h & 0x7c00u) == 0x7c00u && (h & 0x03ffu) != 0; }

__global__ void k_f32_to_f16(uint64_t lo, uint64_t hi)
{
    unsigned long long bad = 0;
    for (uint64_t u = lo + blockIdx.x * 256ull + threadIdx.x; u < hi; u += 256ull * gridDim.x) {
        const float x = emel::bits_to_f32(static_cast<uint32_t>(u));
        const uint16_t a = emel::hw_fp32_to_fp16(x);
        const uint16_t b = emel::emel_fp32_to_fp16(x);
        if (a != b && !(nan16(a) && nan16(b))) ++bad;
    }
    if (bad) atomicAdd(&g_bad, bad);
}

__global__ void k_f16_to_f32()
{
    const uint32_t h = blockIdx.x * 256u + threadIdx.x;
    if (h >= 65536u) return;
    const float a = emel::hw_fp16_to_f32(static_cast<uint16_t>(h));
    const float b = emel::emel_fp16_to_f32(static_cast<uint16_t>(h));
    if (emel::f32_to_bits(a) != emel::f32_to_bits(b) && !(a != a && b != b)) atomicAdd(&g_bad, 1ull);
}

__global__ void k_expf_nonpos(uint64_t lo, uint64_t hi)
{
    __shared__ uint64_t tab[32];
    if (threadIdx.x < 32) tab[threadIdx.x] = emel::kExp2Table[threadIdx.x];
    __syncthreads();
    unsigned long long bad = 0;
    for (uint64_t u = lo + blockIdx.x * 256ull + threadIdx.x; u < hi; u += 256ull * gridDim.x) {
        const float x = emel::bits_to_f32(static_cast<uint32_t>(u));
        if (!(x <= 0.0f) && x == x) continue; // positive inputs are outside the contract
        const float a = emel::emel_expf_nonpos(x, tab);
        const float b = emel::emel_expf(x, tab);
        if (emel::f32_to_bits(a) != emel::f32_to_bits(b) && !(a != a && b != b)) ++bad;
    }
    if (bad) atomicAdd(&g_bad, bad);
}

// emel_silu (clamped argument, no special-case selects) against the
// SiluFormula with the select-based emel_expf.
__global__ void k_silu(uint64_t lo, uint64_t hi)
{
    __shared__ uint64_t tab[32];
    if (threadIdx.x < 32) tab[threadIdx.x] = emel::kExp2Table[threadIdx.x];
    __syncthreads();
    unsigned long long bad = 0;
    for (uint64_t u = lo + blockIdx.x * 256ull + threadIdx.x; u < hi; u += 256ull * gridDim.x) {
        const float x = emel::bits_to_f32(static_cast<uint32_t>(u));
        const float a = emel::emel_silu(x, tab);
        const float b = x / (1.0f + emel::emel_expf(-x, tab));
        if (emel::f32_to_bits(a) != emel::f32_to_bits(b) && !(a != a && b != b)) ++bad;
    }
    if (bad) atomicAdd(&g_bad, bad);
}

// The GELU lookup of the kernels (hardware fp16 conversions, polynomial,
// table, saturation) against the scalar GeluFormula replica.
__device__ __align__(16) uint16_t g_gelu[emel::kGeluTableHalfs];

__global__ void k_gelu_fill()
{
    const uint32_t slot = blockIdx.x * 256u + threadIdx.x;
    if (slot < emel::kGeluTableHalfs)
        g_gelu[slot] = slot < emel::kGeluEntries
                           ? emel::emel_gelu_core_fp16(emel::emel_fp16_to_f32(emel::gelu_slot_key(slot)))
                           : 0;
}

__global__ void k_gelu(uint64_t lo, uint64_t hi)
{
    unsigned long long bad = 0;
    for (uint64_t u = lo + blockIdx.x * 256ull + threadIdx.x; u < hi; u += 256ull * gridDim.x) {
        const float x = emel::bits_to_f32(static_cast<uint32_t>(u));
        const uint16_t h = emel::hw_fp32_to_fp16(x);
        const float q = emel::hw_fp16_to_f32(h);
        const emel::GeluClass c = emel::gelu_class(h);
        const float entry = emel::hw_fp16_to_f32(g_gelu[c.slot]);
        const float poly = emel::hw_fp16_to_f32(emel::hw_fp32_to_fp16(emel::gelu_poly(q)));
        const float a = emel::gelu_finish(x, q, c, entry, poly);
        const float b = emel::emel_gelu(x);
        if (emel::f32_to_bits(a) != emel::f32_to_bits(b) && !(a != a && b != b)) ++bad;
    }
    if (bad) atomicAdd(&g_bad, bad);
}

__global__ void k_sqrtf(uint64_t lo, uint64_t hi)
{
    unsigned long long bad = 0;
    for (uint64_t u = lo + blockIdx.x * 256ull + threadIdx.x; u < hi; u += 256ull * gridDim.x) {
        const float x = emel::bits_to_f32(static_cast<uint32_t>(u));
        const float y = __builtin_sqrtf(x);
        const uint32_t yb = emel::f32_to_bits(y);
        bool ok;
        if (x != x || x < 0.0f) {
            ok = y != y;
        } else if (x == 0.0f || x == __builtin_inff()) {
            ok = yb == emel::f32_to_bits(x);
        } else {
            const uint32_t e = (yb >> 23) & 0xffu;
            if (e == 0u || e == 0xffu || (yb >> 31) != 0u) {
                ok = false;
            } else {
                const double ulp = __builtin_ldexp(1.0, static_cast<int>(e) - 150);
                const double below = (yb & 0x7fffffu) == 0u ? ulp / 4 : ulp / 2; // next value down has half the ulp
                const double d = static_cast<double>(y), xd = static_cast<double>(x);
                const double l = d - below, h = d + ulp / 2;
                ok = l * l < xd && xd < h * h;
            }
        }
        if (!ok) ++bad;
    }
    if (bad) atomicAdd(&g_bad, bad);
}

// f64 square root and quotient as the generic norms compute them
// (__builtin_sqrt, operator /); the host compares with IEEE results.
__global__ void k_f64_ops(const double *x, const double *y, double *sq, double *dv, uint64_t n)
{
    for (uint64_t i = blockIdx.x * 256ull + threadIdx.x; i < n; i += 256ull * gridDim.x) {
        sq[i] = __builtin_sqrt(x[i]);
        dv[i] = x[i] / y[i];
    }
}

template <class Launch>
uint64_t run(Launch launch)
{
    const unsigned long long zero = 0;
    if (hipMemcpyToSymbol(HIP_SYMBOL(g_bad), &zero, sizeof zero) != hipSuccess) return UINT64_MAX;
    launch();
    if (hipGetLastError() != hipSuccess || hipDeviceSynchronize() != hipSuccess) return UINT64_MAX;
    unsigned long long bad = 0;
    if (hipMemcpyFromSymbol(&bad, HIP_SYMBOL(g_bad), sizeof bad) != hipSuccess) return UINT64_MAX;
    return bad;
}

} // namespace

extern "C" {

uint64_t gpu_check_fp32_to_fp16(void)
{
    return run([] { k_f32_to_f16<<<8192, 256>>>(0, 1ull << 32); });
}

uint64_t gpu_check_fp16_to_f32(void)
{
    return run([] { k_f16_to_f32<<<256, 256>>>(); });
}

uint64_t gpu_check_expf_nonpos(void)
{
    return run([] { k_expf_nonpos<<<8192, 256>>>(0, 1ull << 32); });
}

uint64_t gpu_check_silu(void)
{
    return run([] { k_silu<<<8192, 256>>>(0, 1ull << 32); });
}

uint64_t gpu_check_gelu(void)
{
    return run([] {
        k_gelu_fill<<<(emel::kGeluTableHalfs + 255) / 256, 256>>>();
        k_gelu<<<8192, 256>>>(0, 1ull << 32);
    });
}

uint64_t gpu_check_sqrtf(void)
{
    return run([] { k_sqrtf<<<8192, 256>>>(0, 1ull << 32); });
}

// sq[i] = sqrt(x[i]), dv[i] = x[i] / y[i] on the device, n doubles of host
// memory in and out.  Returns 0, or UINT64_MAX on a HIP error.
uint64_t gpu_f64_ops(const double *x, const double *y, double *sq, double *dv, uint64_t n)
{
    double *d = nullptr;
    const uint64_t bytes = n * sizeof(double);
    if (hipMalloc(&d, 4 * bytes) != hipSuccess) return UINT64_MAX;
    uint64_t rc = 0;
    if (hipMemcpy(d, x, bytes, hipMemcpyHostToDevice) != hipSuccess ||
        hipMemcpy(d + n, y, bytes, hipMemcpyHostToDevice) != hipSuccess) {
        rc = UINT64_MAX;
    } else {
        k_f64_ops<<<1024, 256>>>(d, d + n, d + 2 * n, d + 3 * n, n);
        if (hipGetLastError() != hipSuccess || hipDeviceSynchronize() != hipSuccess ||
            hipMemcpy(sq, d + 2 * n, bytes, hipMemcpyDeviceToHost) != hipSuccess ||
            hipMemcpy(dv, d + 3 * n, bytes, hipMemcpyDeviceToHost) != hipSuccess)
            rc = UINT64_MAX;
    }
    (void)hipFree(d);
    return rc;
}

} // extern "C"
