// launch.hpp -- kernel launchers shared between the host API (api.cpp) and
// the gfx950 kernels (*.hip).  Every launcher receives operands that the
// host guards have already validated; the descriptors carry strides in
// elements (the byte strides divided by the element size, exact because the
// guards require multiples of it).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace emel {

// One operand of an elementwise or row kernel.
struct Operand {
    void *data;
    uint64_t ne[4];
    int64_t st[4]; // element strides
};

enum class Binary : uint32_t { Add = 0, Sub = 1, Mul = 2, Div = 3 };

// Elementwise functors (the kernel instantiations live in elementwise.hip).
enum class Ew : uint32_t {
    Add = 0, Sub, Mul, Div,                                        // binary
    Abs, Neg, Tanh, Elu, Relu, Sigmoid, Gelu, Silu, Exp, Scale,   // unary
    Swiglu,                                                        // fused
    GluRe, GluGe, GluSwi, GluSwiOai, GluGeErf, GluGeQuick,        // OpGlu: a = values, b = gates
    Copy, Sqr, Sqrt,                                               // dup and power.rs
    Add1, LeakyRelu, Clamp, GeluGeneric, SiluBack,                 // generic envelope (generic.rs)
    Sgn, Step, GeluQuick, Hardswish, Hardsigmoid, Expm1, Softplus,  // the other typed unary events (unary.rs)
    GeluErf, Floor, Ceil, Round, Trunc,
    Log, Sin, Cos,                                                 // reductions.rs OpLog / OpSin / OpCos
    ClampStd                                                       // activation.rs OpClamp (std::clamp order)
};

// The scalar parameters an elementwise functor reads: x is Scale's factor,
// Add1's addend and LeakyRelu's slope; Clamp reads [x, y] as [min, max].
struct Scal {
    float x;
    float y;
};

// How a source operand is addressed from the destination ordinal.
enum class Addr : uint32_t {
    SameCoords = 0, // source coordinates == destination coordinates
    Broadcast = 1,  // destination coordinates modulo the source extents
    Ordinal = 2     // the ordinal decoded by the source's own extents
};

struct EwArgs {
    Ew op;
    float scale;  // Scal::x
    float scale2; // Scal::y (Ew::Clamp's maximum)
    Operand a;
    Operand b; // unused by unary ops
    Operand o;
    Addr a_addr;
    Addr b_addr;
    uint64_t count; // destination element count
};

hipError_t launch_elementwise(const EwArgs &args, hipStream_t stream);

// OpAcc over dense buffers (elementwise.rs:262-277): dst[k] = base[k], plus
// update[k - offset] for offset <= k < offset + n_update (one f32 addition).
hipError_t launch_acc(const float *base, const float *update, float *dst, uint64_t count, uint64_t offset,
                      uint64_t n_update, hipStream_t stream);

// Bit copy of `bytes` (a multiple of 16; both pointers 16-byte aligned) with
// one of the streaming shapes of the dense kernels, for measuring what a
// plain stream achieves: 0 one float4 per thread, 1 and 2 four and eight
// float4 per lane (each wave over 256 / 512 consecutive float4), 3 one
// resident generation walking the array grid-stride with the next float4
// in flight.
enum class CopyShape : uint32_t { Flat = 0, Wave4 = 1, Wave8 = 2, Walk = 3 };
hipError_t launch_stream_copy(const void *src, void *dst, uint64_t bytes, CopyShape shape, hipStream_t stream);
// Builds the current device's lookup tables (the GELU table) if not yet
// built, and waits for them on `stream`.
hipError_t prepare_device_tables(hipStream_t stream);

// ---- row kernels (rows.hip) --------------------------------------------

// GenRmsNorm / GenNorm: the generic envelope's arithmetic (generic.rs:1988-2055):
// f64 scale, and for norm the f64 sum of f32 squares of the centered values.
enum class RowOp : uint32_t { RmsNorm = 0, RmsNormMul = 1, Norm = 2, SoftMax = 3, SoftMaxExt = 4, GenRmsNorm = 5,
                              GenNorm = 6 };

struct RowArgs {
    RowOp op;
    Operand x;          // input, rows along dim 0
    Operand y;          // output (same extents for norms; same count for soft_max)
    const float *w;     // RmsNormMul weight row (dense or strided by w_st0)
    int64_t w_st0;
    const uint16_t *mask; // SoftMaxExt f16 mask, dense [ne0, ne1, m2, m3]; may be null
    uint64_t mask_ne2, mask_ne3;
    float eps;
    float scale;
    bool dense_sum; // soft_max: f64 row sum (dense layouts) vs f32 sequential sum
};

hipError_t launch_rows(const RowArgs &args, hipStream_t stream);

// soft_max rows of x (ne[0] columns) with the sequential f32 row sum, into y
// (the same element count, addressed by its own ordinals).
hipError_t launch_softmax_seq(const Operand &x, const Operand &y, hipStream_t stream);

// OpGroupNorm (group_norm.rs:197-241): x and y share extents [W, H, C, B];
// group g of batch b is channels [g C/groups, (g+1) C/groups).
hipError_t launch_group_norm(const Operand &x, const Operand &y, uint32_t groups, float eps, hipStream_t stream);

// ---- reductions (reduce.hip) ---------------------------------------------

enum class RedOp : uint32_t { SumRows = 0, ArgmaxRows = 1, Sum = 2, Mean = 3, Argmax = 4 };

// Scratch of a split-row reduction (both 0 when every row is reduced by a
// single workgroup).  `partials` holds per-chunk partial words, rewritten by
// every launch.  `counters` holds per-row arrival counters: they must be
// zero before the first launch on that memory and every launch leaves them
// zero again, so the counters buffer may hold nothing else.
struct RedScratch {
    uint64_t partials;
    uint64_t counters;
};

struct RedArgs {
    RedOp op;
    Operand x;     // source
    void *dst;     // f32 (sums, mean, argmax index) or i32 (ArgmaxRows)
    Operand dst_view; // destination view (strided writes for SumRows)
    void *partials;   // at least scratch.partials bytes
    void *counters;   // at least scratch.counters bytes, zero at rest
    RedScratch scratch;
};

RedScratch reduce_scratch_bytes(const RedArgs &args);
// Points args' scratch at the device's static reduction scratch (128 KiB,
// shared by every call on the device; set up on the device's first call).
// hipErrorOutOfMemory when the plan needs more than it holds.  Allocates
// nothing.
hipError_t reduce_static_scratch(RedArgs &args, hipStream_t stream);
hipError_t launch_reduce(const RedArgs &args, hipStream_t stream);

// ---- generic-envelope routes (generic.hip) ---------------------------------

// An operand addressed by logical ordinal through its own extents.
struct GView {
    void *data;
    uint64_t ne[4];
    int64_t st[4]; // element strides
};

enum class GenRow : uint32_t { Cumsum = 0, SoftMax, Norm, RmsNorm, SoftMaxBack, RmsNormBack };

// Rows are `width` consecutive ordinals of every operand.
struct GenRowArgs {
    GenRow op;
    GView x; // src0
    GView g; // src1 (SoftMaxBack, RmsNormBack)
    GView y; // dst
    uint64_t rows;
    uint64_t width;
    float eps;
};

hipError_t launch_generic_rows(const GenRowArgs &args, hipStream_t stream);

enum class GenOrd : uint32_t { Fill = 0, Arange, Diag, DiagMaskInf, DiagMaskZero, Concat, RepeatBack };

// One destination element per lane, addressed by destination coordinates.
struct GenOrdArgs {
    GenOrd op;
    GView a; // src0
    GView b; // src1 (Concat)
    GView y; // dst
    float p0, p1;    // Fill value; Arange start and step
    uint64_t n_past; // DiagMask*
    uint32_t axis;   // Concat
};

hipError_t launch_generic_ordinal(const GenOrdArgs &args, hipStream_t stream);

enum class GenWork : uint32_t { L2Norm = 0, CountEqual, MulMatArgmax };
uint64_t generic_workspace_bytes(GenWork which);

hipError_t launch_generic_l2_norm(const GView &x, const GView &y, void *workspace, hipStream_t stream);
// The two halves of l2_norm: the sequential f32 sum of squares (workspace[1])
// and its scale 1/sqrt(sum) (workspace[0]); then y = x * scale.
hipError_t launch_generic_l2_sum(const GView &x, void *workspace, hipStream_t stream);
hipError_t launch_generic_l2_apply(const GView &x, const GView &y, const void *workspace, hipStream_t stream);
hipError_t launch_generic_count_equal(const GView &a, const GView &b, float *dst, void *workspace,
                                      hipStream_t stream);

struct GenMatArgs {
    GView lhs, rhs, y;
    uint64_t k, m, n; // argmax: m = rows of lhs
    bool f16;         // dense F16 operands (strides in halves)
    bool argmax;
    int32_t *index_out;
    void *workspace;
};

hipError_t launch_generic_mul_mat(const GenMatArgs &args, hipStream_t stream);

// ---- row gather (getrows.hip) -------------------------------------------------

enum class RowSrc : uint32_t { F32 = 0, F32Bytes, F16, Bf16, Q4_0, Q8_0, Q4K };

struct GetRowsArgs {
    RowSrc kind;
    const void *src;
    uint64_t src_ne[4];
    int64_t src_st[4];    // effective byte strides (unused for packed sources)
    const int32_t *idx;
    uint64_t idx_ne[3];
    int64_t idx_st[3];    // element strides
    float *dst;           // dense [cols, rows]
    uint64_t rows;        // index count
    uint64_t cols;        // src.ne[0]
};

// Host-checked indices carried in the launch arguments (destination row r
// reads v[r]); matches EMEL_GET_ROWS_INLINE_INDICES.
constexpr uint32_t kInlineIndices = 512;
struct IdxInline {
    int32_t v[kInlineIndices];
};

// Whether launch_get_rows takes the one-workgroup-per-row kernels for these
// arguments (the only ones that read inline indices).
bool get_rows_row_kernels(const GetRowsArgs &args);
// inline_idx: NULL reads args.idx from device memory.
hipError_t launch_get_rows(const GetRowsArgs &args, const IdxInline *inline_idx, hipStream_t stream);

// ---- logits sampler and validator (sampler.hip) -------------------------------

// rows independent SampleTemperatureTopK requests over row-strided buffers
// (strides in elements); the host has checked every guard.
struct SamplerArgs {
    uint32_t rows;
    uint64_t card;
    uint32_t top_k;
    float scale; // 1.0f / temperature
    float *logits;
    int64_t logits_ld;
    int32_t *sorted;
    int64_t sorted_ld;
    float *top_p;
    int32_t *top_i;
    int64_t top_ld;
    int32_t *selected;    // rows
    float *score;         // rows
    int32_t *status;      // rows, may be null: 0 or EMEL_ERR_INVALID_REQUEST (result guard)
    const uint32_t *states; // host: rows start states
    void *workspace;      // sampler_workspace_bytes
};

uint64_t sampler_workspace_bytes(uint32_t rows, uint64_t card, uint32_t top_k);
hipError_t launch_sampler(const SamplerArgs &args, hipStream_t stream);

// Validator Build: ids[i] = i and scores[i] = logits[i] - max for i < n.
uint64_t validator_workspace_bytes(uint64_t n);
hipError_t launch_validator(const float *logits, uint64_t n, int32_t *ids, float *scores, void *workspace,
                            hipStream_t stream);

} // namespace emel
