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
    Copy, Sqr, Sqrt                                                // dup and power.rs
};

// How a source operand is addressed from the destination ordinal.
enum class Addr : uint32_t {
    SameCoords = 0, // source coordinates == destination coordinates
    Broadcast = 1,  // destination coordinates modulo the source extents
    Ordinal = 2     // the ordinal decoded by the source's own extents
};

struct EwArgs {
    Ew op;
    float scale; // Ew::Scale
    Operand a;
    Operand b; // unused by unary ops
    Operand o;
    Addr a_addr;
    Addr b_addr;
    uint64_t count; // destination element count
};

hipError_t launch_elementwise(const EwArgs &args, hipStream_t stream);

// ---- row kernels (rows.hip) --------------------------------------------

enum class RowOp : uint32_t { RmsNorm = 0, RmsNormMul = 1, Norm = 2, SoftMax = 3, SoftMaxExt = 4 };

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

// ---- reductions (reduce.hip) ---------------------------------------------

enum class RedOp : uint32_t { SumRows = 0, ArgmaxRows = 1, Sum = 2, Mean = 3, Argmax = 4 };

struct RedArgs {
    RedOp op;
    Operand x;     // source
    void *dst;     // f32 (sums, mean, argmax index) or i32 (ArgmaxRows)
    Operand dst_view; // destination view (strided writes for SumRows)
    void *workspace;  // per-stream scratch, see reduce_workspace_bytes
};

// Bytes of scratch the reduction needs for its per-chunk partials (0 when
// every row is reduced by a single workgroup).
uint64_t reduce_workspace_bytes(const RedArgs &args);
hipError_t launch_reduce(const RedArgs &args, hipStream_t stream);

} // namespace emel
