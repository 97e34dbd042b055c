// elementwise.hip -- gfx950 kernels for the elementwise family:
// equal-count binary add/sub/mul/div (binary.rs:383-424), row broadcast
// (broadcast.rs:352-390), 4-D modulo broadcast (OpRepeat + binary,
// generic.rs:1641-1665), the 21 typed unary events (unary.rs:472-610),
// log / sin / cos (reductions.rs:640-668), scale (activation.rs:366-377),
// fused SwiGLU, the six
// OpGlu gates (glu.rs:103-141, :258-270), copy (event.rs:133-165) and square
// / square root (power.rs:315-360).
//
// All of them are HBM-bound streams (<= 1 flop per byte except the
// transcendental ones, which stay under the memory time).  Three kernel
// shapes cover every accepted layout:
//   k_dense    all operands dense and paired by linear index: 128-bit
//              non-temporal loads/stores, VPT float4 per thread, a scalar
//              tail;
//   k_rowbcast dense [rows, ne0] op dense row [ne0]: 128-bit loads, the
//              row operand re-read from L2;
//   k_rows     any strides with a contiguous dim 0 (permuted views, modulo
//              broadcast): 128-bit accesses along dim 0, rows decoded with
//              multiply-high division;
//   k_ordinal  anything else: one element per thread, the reference's
//              per-element ordinal decode.
#include <cstdlib>
#include <map>
#include <mutex>
#include <type_traits>

#include "common.hpp"
#include "launch.hpp"
#include "libm_replica.hpp"

namespace emel {
namespace {

// GELU's result depends only on the fp16 rounding q of its input when
// |x| < 10 (GeluFormula, unary.rs:522-541).  Small |q| take a polynomial,
// large |q| saturate, and the 7918 values of q in between are looked up
// (libm_replica.hpp, gelu_class / gelu_poly / gelu_finish).  The table is
// computed once per device by the same replica code and read from this
// global copy by the strided kernels, from a copy in LDS by k_gelu_lds.
__device__ __align__(16) uint16_t g_gelu_tab[kGeluTableHalfs];

constexpr uint32_t kGeluBlock = 1024; // threads per k_gelu_lds workgroup
constexpr int kGeluPerCu = 2;         // two workgroups fill a CU (2048 threads)
constexpr int kGeluU = 2;             // float4 per thread per step (measured best of 1, 2, 3, 4, 8)

__global__ __launch_bounds__(kBlock) void k_gelu_table()
{
    const uint32_t slot = blockIdx.x * kBlock + threadIdx.x;
    if (slot < kGeluEntries)
        g_gelu_tab[slot] = emel_gelu_core_fp16(emel_fp16_to_f32(gelu_slot_key(slot)));
    else if (slot < kGeluTableHalfs)
        g_gelu_tab[slot] = 0;
}

__device__ __forceinline__ float gelu_lookup(float a, const uint16_t *tab)
{
    const uint16_t h = hw_fp32_to_fp16(a);
    const float q = hw_fp16_to_f32(h);
    const GeluClass c = gelu_class(h);
    const float entry = hw_fp16_to_f32(tab[c.slot]);
    const float poly = hw_fp16_to_f32(hw_fp32_to_fp16(gelu_poly(q)));
    return gelu_finish(a, q, c, entry, poly);
}

struct DeviceInfo {
    bool gelu_ready = false;
    int cus = 0;
};

// Per-device facts the launchers need: the GELU table (built the first time
// a GELU runs on the device) and the compute-unit count.
hipError_t device_info(hipStream_t stream, bool need_gelu, DeviceInfo &out)
{
    static std::mutex mu;
    static std::map<int, DeviceInfo> known;
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    std::lock_guard<std::mutex> lock(mu);
    DeviceInfo &d = known[dev];
    if (d.cus == 0) {
        e = hipDeviceGetAttribute(&d.cus, hipDeviceAttributeMultiprocessorCount, dev);
        if (e != hipSuccess) return e;
        if (d.cus <= 0) d.cus = 1;
    }
    if (need_gelu && !d.gelu_ready) {
        // Building the table ends with a wait, which a stream under capture
        // cannot do: the first GELU on a device must run eagerly.
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        e = hipStreamIsCapturing(stream, &cs);
        if (e != hipSuccess) return e;
        if (cs != hipStreamCaptureStatusNone) return hipErrorStreamCaptureUnsupported;
        k_gelu_table<<<dim3((kGeluTableHalfs + kBlock - 1) / kBlock), kBlock, 0, stream>>>();
        e = hipGetLastError();
        if (e == hipSuccess) e = hipStreamSynchronize(stream); // visible to every stream from now on
        if (e != hipSuccess) return e;
        d.gelu_ready = true;
    }
    out = d;
    return hipSuccess;
}

// ---- per-element formulas ------------------------------------------------

// What the exp-based formulas read: the 2^(i/32) table (in LDS) and the
// expf constants (in vector registers).
struct ExpCtx {
    const uint64_t *tab;
    ExpfConsts c;
};

template <Ew OP> struct Fn;

#define EMEL_FN(OPV, TABLE, BINARY, EXPR)                                                          \
    template <> struct Fn<Ew::OPV> {                                                                \
        static constexpr bool kTable = TABLE;                                                       \
        static constexpr bool kBinary = BINARY;                                                     \
        __device__ __forceinline__ static float apply(float a, float b, Scal sc, const ExpCtx &t)  \
        {                                                                                           \
            const float s = sc.x, s2 = sc.y;                                                        \
            (void)b; (void)s; (void)s2; (void)t;                                                    \
            return EXPR;                                                                            \
        }                                                                                           \
    };

EMEL_FN(Add, false, true, a + b)
EMEL_FN(Sub, false, true, a - b)
EMEL_FN(Mul, false, true, a * b)
EMEL_FN(Div, false, true, a / b)
EMEL_FN(Abs, false, false, __builtin_fabsf(a))
EMEL_FN(Neg, false, false, -a)
EMEL_FN(Tanh, false, false, emel_tanhf(a))
EMEL_FN(Elu, false, false, a >= 0.0f ? a : emel_expm1f(a))
// f32::max(x, 0.0) with glibc fmaxf's results: x when x > 0, otherwise +0
// (NaN -> +0, and -0 -> +0).
EMEL_FN(Relu, false, false, a > 0.0f ? a : 0.0f)
EMEL_FN(Sigmoid, true, false, 1.0f / (1.0f + emel_expf(-a, t.tab, t.c)))
EMEL_FN(Gelu, false, false, gelu_lookup(a, g_gelu_tab))
EMEL_FN(Silu, true, false, emel_silu(a, t.tab, t.c))
EMEL_FN(Exp, true, false, emel_expf(a, t.tab, t.c))
EMEL_FN(Scale, false, false, a * s)
// silu(gate) rounded to f32, then times up: the OpSilu -> OpMul chain.
EMEL_FN(Swiglu, true, true, emel_silu(a, t.tab, t.c) * b)
// OpGlu (glu.rs:103-141, :258-270): values (a) times a gate function of
// gates (b), every product and sum rounded separately.
__device__ __forceinline__ float glu_gelu_erf(float g, const ExpCtx &t)
{
    const float sign = g < 0.0f ? -1.0f : 1.0f;
    const float x = __builtin_fabsf(g) / 1.41421356237309504880f; // core::f32::consts::SQRT_2
    const float u = 1.0f / (1.0f + 0.3275911f * x);
    const float poly = (((((1.0614054f * u - 1.4531521f) * u) + 1.4214138f) * u - 0.28449672f) * u + 0.2548296f) * u;
    const float erf = sign * (1.0f - poly * emel_expf(-x * x, t.tab, t.c));
    return 0.5f * g * (1.0f + erf);
}
// OpDup copies bits; power.rs squares (v * v) and takes the IEEE square
// root (correctly rounded: checked on the GPU over all 2^32 inputs).
EMEL_FN(Copy, false, false, a)
EMEL_FN(Sqr, false, false, a * a)
EMEL_FN(Sqrt, false, false, __builtin_sqrtf(a))
EMEL_FN(GluRe, false, true, a * (b > 0.0f ? b : 0.0f))
EMEL_FN(GluGe, false, true, a * (0.5f * b * (1.0f + emel_tanhf(0.7978846f * b * (1.0f + 0.044715f * b * b)))))
EMEL_FN(GluSwi, true, true, a * emel_silu(b, t.tab, t.c))
EMEL_FN(GluSwiOai, true, true,
        emel_silu(1.702f * __builtin_fminf(b, 7.0f), t.tab, t.c) / 1.702f * (__builtin_fminf(a, 7.0f) + 1.0f))
EMEL_FN(GluGeErf, true, true, a * glu_gelu_erf(b, t))
EMEL_FN(GluGeQuick, true, true, a * (b * (1.0f / (1.0f + emel_expf(-1.702f * b, t.tab, t.c)))))
// Generic-envelope formulas (generic.rs:1307-1350, :1522-1583).
EMEL_FN(Add1, false, false, a + s)
EMEL_FN(LeakyRelu, false, false, a < 0.0f ? a * s : a)
// f32::clamp: below min -> min, then above max -> max; NaN passes through.
EMEL_FN(Clamp, false, false, (a < s ? s : a) > s2 ? s2 : (a < s ? s : a))
// The generic GELU: no fp16 rounding and no saturation, one fused
// multiply-add inside the tanh argument.
EMEL_FN(GeluGeneric, false, false,
        0.5f * a * (1.0f + emel_tanhf(0.7978846f * __builtin_fmaf(0.044715f * a * a, a, a))))
// a = input, b = incoming gradient.
__device__ __forceinline__ float silu_back(float x, float grad, const ExpCtx &t)
{
    const float sg = 1.0f / (1.0f + emel_expf(-x, t.tab, t.c));
    return grad * (sg * (1.0f + x * (1.0f - sg)));
}
EMEL_FN(SiluBack, true, true, silu_back(a, b, t))
// The remaining typed unary events (unary.rs:472-610), every operation
// rounded separately as the reference writes it.
// f32::signum: +-1 with the sign of a (both zeros included); every NaN
// gives f32::NAN, the quiet NaN 0x7fc00000, whatever its sign or payload.
EMEL_FN(Sgn, false, false, a != a ? __builtin_nanf("") : __builtin_copysignf(1.0f, a))
EMEL_FN(Step, false, false, a > 0.0f ? 1.0f : 0.0f)
EMEL_FN(GeluQuick, false, false, 0.5f * a * (1.0f + emel_tanhf(0.7978846f * a * (1.0f + 0.044715f * a * a))))
// (x + 3).clamp(0, 6): NaN passes through
__device__ __forceinline__ float clamp06(float v)
{
    v = v < 0.0f ? 0.0f : v;
    return v > 6.0f ? 6.0f : v;
}
EMEL_FN(Hardswish, false, false, a * clamp06(a + 3.0f) / 6.0f)
EMEL_FN(Hardsigmoid, false, false, clamp06(a + 3.0f) / 6.0f)
EMEL_FN(Expm1, false, false, emel_expm1f(a))
// exp(x).ln_1p(): two glibc calls, each rounded to f32
EMEL_FN(Softplus, true, false, emel_log1pf(emel_expf(a, t.tab, t.c)))
EMEL_FN(GeluErf, true, false, glu_gelu_erf(a, t))
EMEL_FN(Floor, false, false, __builtin_floorf(a))
EMEL_FN(Ceil, false, false, __builtin_ceilf(a))
// f32::round: halfway cases away from zero
EMEL_FN(Round, false, false, __builtin_roundf(a))
EMEL_FN(Trunc, false, false, __builtin_truncf(a))
// reductions.rs:640-668: f32::ln / sin / cos, glibc logf / sinf / cosf
EMEL_FN(Log, false, false, emel_logf(a))
EMEL_FN(Sin, false, false, emel_sinf(a))
EMEL_FN(Cos, false, false, emel_cosf(a))
// OpClamp (activation.rs:403-421): std::clamp's comparisons, min first; NaN
// passes through, and min > max yields min below it
EMEL_FN(ClampStd, false, false, a < s ? s : (a > s2 ? s2 : a))
#undef EMEL_FN

template <Ew OP>
__device__ __forceinline__ float4 apply4(float4 a, float4 b, Scal s, const ExpCtx &t)
{
    float4 r;
    r.x = Fn<OP>::apply(a.x, b.x, s, t);
    r.y = Fn<OP>::apply(a.y, b.y, s, t);
    r.z = Fn<OP>::apply(a.z, b.z, s, t);
    r.w = Fn<OP>::apply(a.w, b.w, s, t);
    return r;
}

// Stages the 2^(i/32) table in LDS for the exp-based formulas and pins the
// expf constants in vector registers.
template <Ew OP>
__device__ __forceinline__ ExpCtx stage_table(uint64_t *lds)
{
    if constexpr (Fn<OP>::kTable) {
        if (threadIdx.x < 32) lds[threadIdx.x] = kExp2Table[threadIdx.x];
        __syncthreads();
        return ExpCtx{lds, expf_consts_in_vgprs()};
    } else {
        return ExpCtx{nullptr, ExpfConsts{}};
    }
}

// ---- dense: every operand contiguous, paired by linear index -------------

// Streaming policy measured on MI355X with cold buffers: non-temporal loads
// and stores, one float4 per thread for the copy (scale), swiglu and the
// formulas.  The one-instruction binaries (add, sub, mul) stream 8 float4
// per lane, each wave over 512 consecutive float4: fewer, fatter waves (mul
// at [11008,512]: 11.85 against 12.5 us).  With 8 float4 per thread swiglu,
// the row broadcast and a 541 MB copy were slower.
template <Ew OP>
struct Stream {
    static constexpr bool kNtLoad = true;
    static constexpr int kVpt = OP == Ew::Add || OP == Ew::Sub || OP == Ew::Mul ? 8 : 1;
};

template <Ew OP, int VPT>
__global__ __launch_bounds__(kBlock) void k_dense(const float *a, const float *b, float *o, uint64_t nvec,
                                                   uint64_t n, Scal s)
{
    __shared__ uint64_t lds[32];
    const ExpCtx tab = stage_table<OP>(lds);
    const float4 *a4 = reinterpret_cast<const float4 *>(a);
    const float4 *b4 = reinterpret_cast<const float4 *>(b);
    float4 *o4 = reinterpret_cast<float4 *>(o);
    // each wave streams VPT * 64 consecutive float4: lane l takes l, l + 64, ...
    const uint64_t base = VPT == 1 ? static_cast<uint64_t>(blockIdx.x) * kBlock + threadIdx.x
                                   : (static_cast<uint64_t>(blockIdx.x) * kBlock + (threadIdx.x & ~(kWave - 1u))) * VPT +
                                         threadIdx.x % kWave;
    float4 va[VPT], vb[VPT];
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const uint64_t i = base + static_cast<uint64_t>(j) * kWave;
        if (i < nvec) {
            va[j] = Stream<OP>::kNtLoad ? ld_nt(a4 + i) : a4[i];
            if constexpr (Fn<OP>::kBinary) vb[j] = Stream<OP>::kNtLoad ? ld_nt(b4 + i) : b4[i];
            else vb[j] = va[j];
        }
    }
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const uint64_t i = base + static_cast<uint64_t>(j) * kWave;
        if (i < nvec) st_nt(o4 + i, apply4<OP>(va[j], vb[j], s, tab));
    }
    const uint64_t gid = static_cast<uint64_t>(blockIdx.x) * kBlock + threadIdx.x;
    const uint64_t idx = nvec * 4 + gid;
    if (idx < n) o[idx] = Fn<OP>::apply(a[idx], Fn<OP>::kBinary ? b[idx] : 0.0f, s, tab);
}

// ---- dense unary formulas built on a libm replica ------------------------
// expf, tanhf, logf, sinf and cosf are evaluated in double (or through
// fdlibm's f32 steps), 20-40 VALU instructions per element: about as long
// as the element's memory traffic.  With one float4 per thread each wave
// loads, waits, computes and stores, and a whole generation of waves
// computes while the memory system idles.  Here the grid holds one
// resident generation (2048 threads per CU) that walks the array
// grid-stride, each thread loading its next float4 before storing the
// current result, so loads stay in flight during the arithmetic.  Measured
// for silu at 5.6 M elements: 9.1 us against 10.3 us with one float4 per
// thread, a copy taking 8.8 us.  Binary formulas move 12 bytes per element
// and stay on k_dense (no gain measured for SwiGLU).
template <Ew OP>
constexpr bool kHeavyUnary = !Fn<OP>::kBinary &&
                             (Fn<OP>::kTable || OP == Ew::Tanh || OP == Ew::Elu || OP == Ew::GeluGeneric ||
                              OP == Ew::GeluQuick || OP == Ew::Expm1 || OP == Ew::Log || OP == Ew::Sin ||
                              OP == Ew::Cos);
constexpr int kResidentPerCu = 2048 / kBlock; // workgroups of one resident generation per CU

template <Ew OP>
__global__ __launch_bounds__(kBlock) void k_dense_walk(const float *a, float *o, uint64_t nvec, uint64_t n, Scal s)
{
    __shared__ uint64_t lds[32];
    const float4 *a4 = reinterpret_cast<const float4 *>(a);
    float4 *o4 = reinterpret_cast<float4 *>(o);
    const uint64_t gid = static_cast<uint64_t>(blockIdx.x) * kBlock + threadIdx.x;
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kBlock;
    float4 v{};
    if (gid < nvec) v = ld_nt(a4 + gid);
    const ExpCtx tab = stage_table<OP>(lds);
    for (uint64_t i = gid; i < nvec; i += stride) {
        const float4 r = apply4<OP>(v, v, s, tab);
        if (i + stride < nvec) v = ld_nt(a4 + i + stride);
        st_nt(o4 + i, r);
    }
    const uint64_t idx = nvec * 4 + gid;
    if (idx < n) o[idx] = Fn<OP>::apply(a[idx], 0.0f, s, tab);
}

// ---- dense GELU with the table in LDS -----------------------------------
// A gather from the global table touches up to 64 cache lines per wave; from
// LDS it costs a few cycles.  Each workgroup stages the 15.8 KB table once
// (its first data is already in flight meanwhile) and then walks the array
// grid-stride, U float4 per thread per step, the next step's loads issued
// before the current step's stores.  The staging is the kernel's overhead
// over a copy: with the earlier whole-range table of 68 KB (34,796 entries,
// no polynomial) the kernel took 10.0 us against 9.0 us now at 5.6 M
// elements, a copy taking 8.8 us.
template <int U>
__global__ __launch_bounds__(kGeluBlock) void k_gelu_lds(const float *a, float *o, uint64_t nvec, uint64_t n)
{
    __shared__ __align__(16) uint16_t tab[kGeluTableHalfs];
    const float4 *a4 = reinterpret_cast<const float4 *>(a);
    float4 *o4 = reinterpret_cast<float4 *>(o);
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * (kGeluBlock * U);
    uint64_t base = static_cast<uint64_t>(blockIdx.x) * (kGeluBlock * U) + threadIdx.x;
    float4 v[U];
#pragma unroll
    for (int j = 0; j < U; ++j) {
        const uint64_t i = base + static_cast<uint64_t>(j) * kGeluBlock;
        if (i < nvec) v[j] = ld_nt(a4 + i);
    }
    {
        const uint4 *src = reinterpret_cast<const uint4 *>(g_gelu_tab);
        uint4 *dst = reinterpret_cast<uint4 *>(tab);
        for (uint32_t k = threadIdx.x; k < kGeluTableHalfs / 8u; k += kGeluBlock) dst[k] = src[k];
    }
    __syncthreads();
    for (; base < nvec; base += stride) {
        float4 r[U];
#pragma unroll
        for (int j = 0; j < U; ++j) {
            r[j].x = gelu_lookup(v[j].x, tab);
            r[j].y = gelu_lookup(v[j].y, tab);
            r[j].z = gelu_lookup(v[j].z, tab);
            r[j].w = gelu_lookup(v[j].w, tab);
        }
        const uint64_t next = base + stride;
#pragma unroll
        for (int j = 0; j < U; ++j) {
            const uint64_t i = next + static_cast<uint64_t>(j) * kGeluBlock;
            if (i < nvec) v[j] = ld_nt(a4 + i);
        }
#pragma unroll
        for (int j = 0; j < U; ++j) {
            const uint64_t i = base + static_cast<uint64_t>(j) * kGeluBlock;
            if (i < nvec) st_nt(o4 + i, r[j]);
        }
    }
    const uint64_t gid = static_cast<uint64_t>(blockIdx.x) * kGeluBlock + threadIdx.x;
    const uint64_t idx = nvec * 4 + gid;
    if (idx < n) o[idx] = gelu_lookup(a[idx], tab);
}

// ---- dense [rows, ne0] op dense row [ne0], ne0 % 4 == 0 --------------------

template <Ew OP, int VPT>
__global__ __launch_bounds__(kBlock) void k_rowbcast(const float *a, const float *b, float *o, uint32_t nvec,
                                                      FastDiv nv0, Scal s)
{
    __shared__ uint64_t lds[32];
    const ExpCtx tab = stage_table<OP>(lds);
    const float4 *a4 = reinterpret_cast<const float4 *>(a);
    const float4 *b4 = reinterpret_cast<const float4 *>(b);
    float4 *o4 = reinterpret_cast<float4 *>(o);
    const uint32_t base = blockIdx.x * (kBlock * VPT) + threadIdx.x;
    float4 va[VPT], vb[VPT];
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const uint32_t i = base + j * kBlock;
        if (i < nvec) {
            va[j] = ld_nt(a4 + i);
            vb[j] = b4[nv0.mod(i)]; // the row operand is re-read by every row: cached
        }
    }
#pragma unroll
    for (int j = 0; j < VPT; ++j) {
        const uint32_t i = base + j * kBlock;
        if (i < nvec) st_nt(o4 + i, apply4<OP>(va[j], vb[j], s, tab));
    }
}

// ---- strided with contiguous dim 0 ---------------------------------------

struct RowsGeo {
    uint32_t nvec;   // float4 work items (< 2^32)
    FastDiv nv0;     // float4 per row
    FastDiv ne1, ne2;
    int64_t a_st[4], b_st[4], o_st[4];
    FastDiv a_mod[3], b_mod[3]; // source extents of dims 1..3
    uint32_t a_modmask, b_modmask; // bit d-1 set: dim d needs a modulo
    uint32_t b_splat;              // b has extent 1 along dim 0
};

__device__ __forceinline__ int64_t rows_offset(const int64_t *st, const FastDiv *md, uint32_t mask, uint32_t i1,
                                               uint32_t i2, uint32_t i3)
{
    if (mask & 1u) i1 = md[0].mod(i1);
    if (mask & 2u) i2 = md[1].mod(i2);
    if (mask & 4u) i3 = md[2].mod(i3);
    return static_cast<int64_t>(i1) * st[1] + static_cast<int64_t>(i2) * st[2] + static_cast<int64_t>(i3) * st[3];
}

template <Ew OP>
__global__ __launch_bounds__(kBlock) void k_rows(RowsGeo g, const float *a, const float *b, float *o, Scal s)
{
    __shared__ uint64_t lds[32];
    const ExpCtx tab = stage_table<OP>(lds);
    const uint32_t i = blockIdx.x * kBlock + threadIdx.x;
    if (i >= g.nvec) return;
    const uint32_t row = g.nv0.div(i);
    const uint32_t v = i - row * g.nv0.d;
    const uint32_t r2 = g.ne1.div(row);
    const uint32_t i1 = row - r2 * g.ne1.d;
    const uint32_t i3 = g.ne2.div(r2);
    const uint32_t i2 = r2 - i3 * g.ne2.d;
    const int64_t col = 4 * static_cast<int64_t>(v);
    const float4 va = ld_nt(reinterpret_cast<const float4 *>(a + rows_offset(g.a_st, g.a_mod, g.a_modmask, i1, i2, i3) + col));
    float4 vb = va;
    if constexpr (Fn<OP>::kBinary) {
        const float *bp = b + rows_offset(g.b_st, g.b_mod, g.b_modmask, i1, i2, i3);
        if (g.b_splat) {
            const float x = *bp;
            vb = make_float4(x, x, x, x);
        } else {
            vb = *reinterpret_cast<const float4 *>(bp + col);
        }
    }
    const int64_t oo = static_cast<int64_t>(i1) * g.o_st[1] + static_cast<int64_t>(i2) * g.o_st[2] +
                       static_cast<int64_t>(i3) * g.o_st[3] + col;
    st_nt(reinterpret_cast<float4 *>(o + oo), apply4<OP>(va, vb, s, tab));
}

// ---- general: one element per thread, per-operand ordinal decode ----------

struct OrdOperand {
    uint64_t ne[4];
    int64_t st[4];
    uint32_t addr; // Addr
};

struct OrdGeo {
    uint64_t count;
    uint64_t ne[4]; // destination extents
    int64_t o_st[4];
    OrdOperand a, b;
};

__device__ __forceinline__ int64_t ord_offset(const OrdOperand &p, uint64_t k, const uint64_t *c)
{
    if (p.addr == static_cast<uint32_t>(Addr::Ordinal)) {
        int64_t off = 0;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            off += static_cast<int64_t>(k % p.ne[d]) * p.st[d];
            k /= p.ne[d];
        }
        return off;
    }
    int64_t off = 0;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        const uint64_t cd = p.addr == static_cast<uint32_t>(Addr::Broadcast) ? c[d] % p.ne[d] : c[d];
        off += static_cast<int64_t>(cd) * p.st[d];
    }
    return off;
}

template <Ew OP>
__global__ __launch_bounds__(kBlock) void k_ordinal(OrdGeo g, const float *a, const float *b, float *o, Scal s)
{
    __shared__ uint64_t lds[32];
    const ExpCtx tab = stage_table<OP>(lds);
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kBlock;
    for (uint64_t k = static_cast<uint64_t>(blockIdx.x) * kBlock + threadIdx.x; k < g.count; k += stride) {
        uint64_t c[4];
        uint64_t rem = k;
        int64_t oo = 0;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            c[d] = rem % g.ne[d];
            rem /= g.ne[d];
            oo += static_cast<int64_t>(c[d]) * g.o_st[d];
        }
        const float va = a[ord_offset(g.a, k, c)];
        const float vb = Fn<OP>::kBinary ? b[ord_offset(g.b, k, c)] : 0.0f;
        o[oo] = Fn<OP>::apply(va, vb, s, tab);
    }
}

// ---- host-side selection ---------------------------------------------------

bool contiguous(const Operand &p)
{
    // Row-major with unit element stride; strides of extent-1 dims do not
    // affect addressing and are ignored.
    int64_t expect = 1;
    for (int d = 0; d < 4; ++d) {
        if (p.ne[d] != 1 && p.st[d] != expect) return false;
        expect *= static_cast<int64_t>(p.ne[d]);
    }
    return true;
}

bool same_ne(const Operand &x, const Operand &y)
{
    for (int d = 0; d < 4; ++d)
        if (x.ne[d] != y.ne[d]) return false;
    return true;
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

template <Ew OP>
hipError_t launch_op(const EwArgs &x, hipStream_t stream)
{
    constexpr bool kBin = Fn<OP>::kBinary;
    const float *a = static_cast<const float *>(x.a.data);
    const float *b = kBin ? static_cast<const float *>(x.b.data) : nullptr;
    float *o = static_cast<float *>(x.o.data);
    const uint64_t n = x.count;
    if (n == 0) return hipSuccess;
    DeviceInfo dev{};
    {
        const hipError_t e = device_info(stream, OP == Ew::Gelu, dev);
        if (e != hipSuccess) return e;
    }

    // Linear pairing holds when each source is dense and either addressed by
    // ordinal or shaped like the destination.
    auto linear = [&](const Operand &p, Addr ad) {
        return contiguous(p) && (ad == Addr::Ordinal || same_ne(p, x.o));
    };
    const bool all_linear = contiguous(x.o) && linear(x.a, x.a_addr) && (!kBin || linear(x.b, x.b_addr));
    const bool vec_ok = aligned16(a) && aligned16(o) && (!kBin || aligned16(b));

    if (all_linear && vec_ok) {
        if constexpr (OP == Ew::Gelu) {
            const uint64_t nvec = n / 4;
            const uint64_t per_block = static_cast<uint64_t>(kGeluBlock) * kGeluU;
            uint64_t blocks = (nvec + per_block - 1) / per_block;
            const uint64_t resident = static_cast<uint64_t>(dev.cus) * kGeluPerCu;
            if (blocks > resident) blocks = resident;
            if (blocks == 0) blocks = 1; // the scalar tail (n < 4)
            k_gelu_lds<kGeluU><<<dim3(static_cast<uint32_t>(blocks)), kGeluBlock, 0, stream>>>(a, o, nvec, n);
            return hipGetLastError();
        }
        if constexpr (kHeavyUnary<OP>) {
            const uint64_t nvec = n / 4;
            uint64_t blocks = (nvec + kBlock - 1) / kBlock;
            const uint64_t resident = static_cast<uint64_t>(dev.cus) * kResidentPerCu;
            if (blocks > resident) blocks = resident;
            if (blocks == 0) blocks = 1; // the scalar tail (n < 4)
            k_dense_walk<OP><<<dim3(static_cast<uint32_t>(blocks)), kBlock, 0, stream>>>(a, o, nvec, n,
                                                                                       Scal{x.scale, x.scale2});
            return hipGetLastError();
        }
        constexpr int vpt = Stream<OP>::kVpt;
        const uint64_t nvec = n / 4;
        const uint64_t per_block = static_cast<uint64_t>(kBlock) * vpt;
        const uint64_t tail = n - nvec * 4;
        uint64_t blocks = (nvec + per_block - 1) / per_block;
        const uint64_t tail_blocks = (tail + kBlock - 1) / kBlock;
        if (blocks < tail_blocks) blocks = tail_blocks;
        if (blocks > 0x7fffffffull) return hipErrorInvalidConfiguration;
        const dim3 grid(static_cast<uint32_t>(blocks));
        k_dense<OP, vpt><<<grid, kBlock, 0, stream>>>(a, b, o, nvec, n, Scal{x.scale, x.scale2});
        return hipGetLastError();
    }

    const uint64_t ne0 = x.o.ne[0];
    const uint64_t rows = n / ne0;

    // dense [rows, ne0] op a dense row of ne0 values
    if (kBin && ne0 % 4 == 0 && vec_ok && contiguous(x.o) && contiguous(x.a) && same_ne(x.a, x.o) &&
        x.a_addr != Addr::Ordinal && x.b.ne[0] == ne0 && x.b.ne[1] == 1 && x.b.ne[2] == 1 && x.b.ne[3] == 1 &&
        x.b.st[0] == 1 && n / 4 < 0xffffffffull && x.b_addr != Addr::Ordinal) {
        constexpr int vpt = 1; // more float4 per thread measured slower here
        const uint32_t nvec = static_cast<uint32_t>(n / 4);
        const uint32_t per_block = kBlock * vpt;
        const dim3 grid((nvec + per_block - 1) / per_block);
        const FastDiv nv0(static_cast<uint32_t>(ne0 / 4));
        k_rowbcast<OP, vpt><<<grid, kBlock, 0, stream>>>(a, b, o, nvec, nv0, Scal{x.scale, x.scale2});
        return hipGetLastError();
    }

    // contiguous dim 0 everywhere, coordinates shared with the destination
    auto coord_addressed = [&](const Operand &p, Addr ad) {
        return ad != Addr::Ordinal || same_ne(p, x.o);
    };
    auto strides4 = [](const Operand &p) {
        for (int d = 1; d < 4; ++d)
            if (p.ne[d] != 1 && p.st[d] % 4 != 0) return false;
        return true;
    };
    const bool b_splat = kBin && x.b.ne[0] == 1;
    const bool rows_ok = ne0 % 4 == 0 && vec_ok && n / 4 < 0xffffffffull && rows < 0xffffffffull &&
                         x.o.ne[1] < 0xffffffffull && x.o.ne[2] < 0xffffffffull && x.o.st[0] == 1 &&
                         strides4(x.o) && (x.a.st[0] == 1 || x.a.ne[0] == 1) && x.a.ne[0] == ne0 &&
                         strides4(x.a) && coord_addressed(x.a, x.a_addr) &&
                         (!kBin || ((b_splat || (x.b.ne[0] == ne0 && x.b.st[0] == 1)) &&
                                    (b_splat || strides4(x.b)) && coord_addressed(x.b, x.b_addr)));
    if (rows_ok) {
        RowsGeo g{};
        g.nvec = static_cast<uint32_t>(n / 4);
        g.nv0 = FastDiv(static_cast<uint32_t>(ne0 / 4));
        g.ne1 = FastDiv(static_cast<uint32_t>(x.o.ne[1]));
        g.ne2 = FastDiv(static_cast<uint32_t>(x.o.ne[2]));
        uint32_t am = 0, bm = 0;
        for (int d = 0; d < 4; ++d) {
            g.a_st[d] = x.a.st[d];
            g.o_st[d] = x.o.st[d];
            g.b_st[d] = kBin ? x.b.st[d] : 0;
        }
        for (int d = 1; d < 4; ++d) {
            g.a_mod[d - 1] = FastDiv(static_cast<uint32_t>(x.a.ne[d]));
            if (x.a.ne[d] != x.o.ne[d]) am |= 1u << (d - 1);
            if (kBin) {
                g.b_mod[d - 1] = FastDiv(static_cast<uint32_t>(x.b.ne[d]));
                if (x.b.ne[d] != x.o.ne[d]) bm |= 1u << (d - 1);
            } else {
                g.b_mod[d - 1] = FastDiv(1);
            }
        }
        g.a_modmask = am;
        g.b_modmask = bm;
        g.b_splat = b_splat ? 1u : 0u;
        const dim3 grid((g.nvec + kBlock - 1) / kBlock);
        k_rows<OP><<<grid, kBlock, 0, stream>>>(g, a, b, o, Scal{x.scale, x.scale2});
        return hipGetLastError();
    }

    OrdGeo g{};
    g.count = n;
    for (int d = 0; d < 4; ++d) {
        g.ne[d] = x.o.ne[d];
        g.o_st[d] = x.o.st[d];
        g.a.ne[d] = x.a.ne[d];
        g.a.st[d] = x.a.st[d];
        g.b.ne[d] = kBin ? x.b.ne[d] : 1;
        g.b.st[d] = kBin ? x.b.st[d] : 0;
    }
    g.a.addr = static_cast<uint32_t>(x.a_addr);
    g.b.addr = static_cast<uint32_t>(kBin ? x.b_addr : Addr::SameCoords);
    uint64_t blocks = (n + kBlock - 1) / kBlock;
    if (blocks > 65536) blocks = 65536;
    k_ordinal<OP><<<dim3(static_cast<uint32_t>(blocks)), kBlock, 0, stream>>>(g, a, b, o, Scal{x.scale, x.scale2});
    return hipGetLastError();
}

} // namespace

hipError_t launch_elementwise(const EwArgs &args, hipStream_t stream)
{
    switch (args.op) {
    case Ew::Add: return launch_op<Ew::Add>(args, stream);
    case Ew::Sub: return launch_op<Ew::Sub>(args, stream);
    case Ew::Mul: return launch_op<Ew::Mul>(args, stream);
    case Ew::Div: return launch_op<Ew::Div>(args, stream);
    case Ew::Abs: return launch_op<Ew::Abs>(args, stream);
    case Ew::Neg: return launch_op<Ew::Neg>(args, stream);
    case Ew::Tanh: return launch_op<Ew::Tanh>(args, stream);
    case Ew::Elu: return launch_op<Ew::Elu>(args, stream);
    case Ew::Relu: return launch_op<Ew::Relu>(args, stream);
    case Ew::Sigmoid: return launch_op<Ew::Sigmoid>(args, stream);
    case Ew::Gelu: return launch_op<Ew::Gelu>(args, stream);
    case Ew::Silu: return launch_op<Ew::Silu>(args, stream);
    case Ew::Exp: return launch_op<Ew::Exp>(args, stream);
    case Ew::Scale: return launch_op<Ew::Scale>(args, stream);
    case Ew::Swiglu: return launch_op<Ew::Swiglu>(args, stream);
    case Ew::Copy: return launch_op<Ew::Copy>(args, stream);
    case Ew::Sqr: return launch_op<Ew::Sqr>(args, stream);
    case Ew::Sqrt: return launch_op<Ew::Sqrt>(args, stream);
    case Ew::GluRe: return launch_op<Ew::GluRe>(args, stream);
    case Ew::GluGe: return launch_op<Ew::GluGe>(args, stream);
    case Ew::GluSwi: return launch_op<Ew::GluSwi>(args, stream);
    case Ew::GluSwiOai: return launch_op<Ew::GluSwiOai>(args, stream);
    case Ew::GluGeErf: return launch_op<Ew::GluGeErf>(args, stream);
    case Ew::GluGeQuick: return launch_op<Ew::GluGeQuick>(args, stream);
    case Ew::Add1: return launch_op<Ew::Add1>(args, stream);
    case Ew::LeakyRelu: return launch_op<Ew::LeakyRelu>(args, stream);
    case Ew::Clamp: return launch_op<Ew::Clamp>(args, stream);
    case Ew::GeluGeneric: return launch_op<Ew::GeluGeneric>(args, stream);
    case Ew::SiluBack: return launch_op<Ew::SiluBack>(args, stream);
    case Ew::ClampStd: return launch_op<Ew::ClampStd>(args, stream);
    case Ew::Sgn: return launch_op<Ew::Sgn>(args, stream);
    case Ew::Step: return launch_op<Ew::Step>(args, stream);
    case Ew::GeluQuick: return launch_op<Ew::GeluQuick>(args, stream);
    case Ew::Hardswish: return launch_op<Ew::Hardswish>(args, stream);
    case Ew::Hardsigmoid: return launch_op<Ew::Hardsigmoid>(args, stream);
    case Ew::Expm1: return launch_op<Ew::Expm1>(args, stream);
    case Ew::Softplus: return launch_op<Ew::Softplus>(args, stream);
    case Ew::GeluErf: return launch_op<Ew::GeluErf>(args, stream);
    case Ew::Floor: return launch_op<Ew::Floor>(args, stream);
    case Ew::Ceil: return launch_op<Ew::Ceil>(args, stream);
    case Ew::Round: return launch_op<Ew::Round>(args, stream);
    case Ew::Trunc: return launch_op<Ew::Trunc>(args, stream);
    case Ew::Log: return launch_op<Ew::Log>(args, stream);
    case Ew::Sin: return launch_op<Ew::Sin>(args, stream);
    case Ew::Cos: return launch_op<Ew::Cos>(args, stream);
    }
    return hipErrorInvalidValue;
}

// ---- OpAcc (elementwise.rs:262-277) -------------------------------------------

namespace {
__global__ __launch_bounds__(kBlock) void k_acc(const float *base, const float *update, float *dst, uint64_t count,
                                                 uint64_t offset, uint64_t n_update)
{
    const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kBlock;
    for (uint64_t k = static_cast<uint64_t>(blockIdx.x) * kBlock + threadIdx.x; k < count; k += stride) {
        float v = base[k];
        if (k >= offset && k - offset < n_update) v = v + update[k - offset]; // no +0.0 outside the update
        dst[k] = v;
    }
}
} // namespace

hipError_t prepare_device_tables(hipStream_t stream)
{
    DeviceInfo d{};
    return device_info(stream, true, d);
}

hipError_t launch_stream_copy(const void *src, void *dst, uint64_t bytes, CopyShape shape, hipStream_t stream)
{
    if (bytes == 0) return hipSuccess;
    const float *a = static_cast<const float *>(src);
    float *o = static_cast<float *>(dst);
    const uint64_t nvec = bytes / 16;
    const uint64_t n = bytes / 4;
    auto dense = [&](auto vpt_tag) {
        constexpr int vpt = decltype(vpt_tag)::value;
        const uint64_t blocks = (nvec + kBlock * vpt - 1) / (kBlock * vpt);
        if (blocks > 0x7fffffffull) return hipErrorInvalidConfiguration;
        k_dense<Ew::Copy, vpt><<<dim3(static_cast<uint32_t>(blocks)), kBlock, 0, stream>>>(a, nullptr, o, nvec, n,
                                                                                            Scal{0.0f, 0.0f});
        return hipGetLastError();
    };
    switch (shape) {
    case CopyShape::Flat: return dense(std::integral_constant<int, 1>{});
    case CopyShape::Wave4: return dense(std::integral_constant<int, 4>{});
    case CopyShape::Wave8: return dense(std::integral_constant<int, 8>{});
    case CopyShape::Walk: {
        DeviceInfo dev{};
        const hipError_t e = device_info(stream, false, dev);
        if (e != hipSuccess) return e;
        uint64_t blocks = (nvec + kBlock - 1) / kBlock;
        const uint64_t resident = static_cast<uint64_t>(dev.cus) * kResidentPerCu;
        if (blocks > resident) blocks = resident;
        k_dense_walk<Ew::Copy><<<dim3(static_cast<uint32_t>(blocks)), kBlock, 0, stream>>>(a, o, nvec, n,
                                                                                          Scal{0.0f, 0.0f});
        return hipGetLastError();
    }
    }
    return hipErrorInvalidValue;
}

hipError_t launch_acc(const float *base, const float *update, float *dst, uint64_t count, uint64_t offset,
                      uint64_t n_update, hipStream_t stream)
{
    if (count == 0) return hipSuccess;
    uint64_t blocks = (count + kBlock - 1) / kBlock;
    if (blocks > 65536) blocks = 65536;
    k_acc<<<dim3(static_cast<uint32_t>(blocks)), kBlock, 0, stream>>>(base, update, dst, count, offset, n_update);
    return hipGetLastError();
}

} // namespace emel
