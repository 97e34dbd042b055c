/*
 * emel_hip.h -- C ABI of the MI355X (gfx950) implementation of emel.rs's
 * tensor-library hot path: elementwise, broadcast and row-reduction ops.
 *
 * This is the drop-in boundary.  Each entry point replaces one operator
 * event of emel-kernels' portable router (stateforward/emel.rs,
 * crates/emel-kernels/src/any/, cited below as file:line) and keeps its
 * argument meaning, validation order and error classification.  A Rust FFI
 * crate binds these functions one-to-one: #[repr(C)] mirrors of
 * emel_tensor_view / emel_tensor_view_mut and an extern "C" block with the
 * same signatures, status codes mapped onto the reference's error enums.
 *
 * Conventions
 *   - Views mirror the pinned C++ tensor_view {data, type, ne[4], nb[4]}
 *     (tools/emel-kernel-binary-reference/main.cpp:14-30) plus data_bytes,
 *     the byte length of the caller's allocation at data (the Rust slice
 *     length that Layout::validate checks spans against,
 *     tensor_view.rs:397-447).  data is a device pointer for every op.
 *   - nb[0] == 0 selects the implicit row-major layout, as in
 *     Layout::effective_f32_strides (tensor_view.rs:262-277).
 *   - Every op runs the reference's guards on the host before anything is
 *     enqueued.  A rejected request enqueues nothing and never writes dst.
 *   - Ops are asynchronous on `stream` (a hipStream_t; NULL is the null
 *     stream).  emel_stream_synchronize gives the reference's synchronous
 *     run-to-completion semantics.
 *   - dst may be the same view as a source (in place).  Any other overlap
 *     between dst and a source is rejected as EMEL_ERR_INVALID_VIEW.
 *   - There is no CPU fallback: without a usable gfx950 device an accepted
 *     request returns EMEL_ERR_KERNEL_UNAVAILABLE.
 */
#ifndef EMEL_HIP_H
#define EMEL_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define EMEL_HIP_ABI_VERSION 2u

/* Status codes.  One code per variant of the reference's typed errors:
 * BinaryError / BroadcastError / UnaryError / ReductionError /
 * ActivationError {InvalidView, ShapeMismatch, UnexpectedEvent, Internal}
 * (binary.rs:20-29, broadcast.rs:28-38, unary.rs:22-31,
 * reductions.rs:21-30), NormalizationError adds InvalidParameters
 * (normalization.rs:31-42), root Error adds KernelUnavailable
 * (actor.rs:88-101). */
typedef enum emel_status {
    EMEL_OK = 0,
    EMEL_ERR_INVALID_VIEW = 1,
    EMEL_ERR_SHAPE_MISMATCH = 2,
    EMEL_ERR_INVALID_PARAMETERS = 3,
    EMEL_ERR_UNEXPECTED_EVENT = 4,
    EMEL_ERR_INTERNAL = 5,
    EMEL_ERR_KERNEL_UNAVAILABLE = 6, /* no usable gfx950 device */
    EMEL_ERR_DEVICE = 7,             /* a HIP runtime call failed */
    EMEL_ERR_INVALID_ARGUMENT = 8,   /* a required pointer argument is NULL */
    EMEL_ERR_INVALID_SHAPE = 9,      /* root Error::InvalidShape (actor.rs:88-101): dense-slice events */
    EMEL_ERR_UNSUPPORTED_OPERATION = 10, /* root Error::UnsupportedOperation */
    EMEL_ERR_INDEX_OUT_OF_BOUNDS = 11,   /* GetRowsError::IndexOutOfBounds (get_rows.rs:520-535) */
    EMEL_ERR_UNSUPPORTED_SOURCE_STRIDE = 12, /* GetRowsError::UnsupportedSourceStride */
    EMEL_ERR_INVALID_REQUEST = 13, /* emel-logits SamplerError::InvalidRequest / ValidatorError::InvalidRequest
                                      (crates/emel-logits/src/sampler/sm.rs:41-52, validator/sm.rs:15-21) */
    EMEL_ERR_STREAM_CAPTURE = 14,  /* the call would allocate, synchronise or advance host state while its
                                      stream is being captured into a HIP graph (no reference counterpart) */
    EMEL_ERR_INVALID_OFFSET = 15,  /* ElementwiseError::InvalidOffset (elementwise.rs:20-27): OpAcc */
    EMEL_ERR_ZERO_NORM = 16        /* GroupNormError::ZeroNorm (group_norm.rs:15-23): OpL2Norm */
} emel_status;

/* Wire dtype codes, DType::from_code (crates/emel-kernels/src/any/
 * tensor_view.rs:111-158): the codes some entry point of this library reads.
 * Views of any other code (0..255) are carried and validated, never read. */
typedef enum emel_dtype {
    EMEL_DTYPE_F32 = 0,
    EMEL_DTYPE_F16 = 1,
    EMEL_DTYPE_Q4_0 = 2,
    EMEL_DTYPE_Q8_0 = 8,
    EMEL_DTYPE_Q4_K = 12,
    EMEL_DTYPE_I32 = 26,
    EMEL_DTYPE_BF16 = 30
} emel_dtype;

/* Unary wire subop codes, UnarySubOp (unary.rs:101-146).  OpUnary and the
 * generic envelope accept eight of them (abs, neg, tanh, elu, relu, gelu,
 * silu, exp); emel_op_unary_event takes every code that has a typed event
 * (all but XIELU). */
typedef enum emel_unary_subop {
    EMEL_UNARY_ABS = 0,
    EMEL_UNARY_SGN = 1,
    EMEL_UNARY_NEG = 2,
    EMEL_UNARY_STEP = 3,
    EMEL_UNARY_TANH = 4,
    EMEL_UNARY_ELU = 5,
    EMEL_UNARY_RELU = 6,
    EMEL_UNARY_SIGMOID = 7,
    EMEL_UNARY_GELU = 8,
    EMEL_UNARY_GELU_QUICK = 9,
    EMEL_UNARY_SILU = 10,
    EMEL_UNARY_HARDSWISH = 11,
    EMEL_UNARY_HARDSIGMOID = 12,
    EMEL_UNARY_EXP = 13,
    EMEL_UNARY_EXPM1 = 14,
    EMEL_UNARY_SOFTPLUS = 15,
    EMEL_UNARY_GELU_ERF = 16,
    EMEL_UNARY_XIELU = 17,
    EMEL_UNARY_FLOOR = 18,
    EMEL_UNARY_CEIL = 19,
    EMEL_UNARY_ROUND = 20,
    EMEL_UNARY_TRUNC = 21
} emel_unary_subop;

/* GLU wire subop codes, GluSubOp (glu.rs:22-37). */
typedef enum emel_glu_subop {
    EMEL_GLU_REGLU = 0,       /* x * relu(g) */
    EMEL_GLU_GEGLU = 1,       /* x * gelu_tanh(g) */
    EMEL_GLU_SWIGLU = 2,      /* x * silu(g) */
    EMEL_GLU_SWIGLU_OAI = 3,  /* clamped gate and value, alpha 1.702 */
    EMEL_GLU_GEGLU_ERF = 4,   /* x * gelu_erf(g) */
    EMEL_GLU_GEGLU_QUICK = 5  /* x * gelu_quick(g) */
} emel_glu_subop;

typedef enum emel_binary_op {
    EMEL_BINARY_ADD = 0,
    EMEL_BINARY_SUB = 1,
    EMEL_BINARY_MUL = 2,
    EMEL_BINARY_DIV = 3
} emel_binary_op;

/* The first 80 bytes are the pinned C++ tensor_view {data, type, ne, nb}
 * (tools/emel-kernel-binary-reference/main.cpp:14-30, with its 4-byte dtype
 * enum padded to 8): a view in that format becomes this one by setting
 * reserved to 0 and appending data_bytes. */
typedef struct emel_tensor_view {
    const void *data;
    uint32_t dtype;
    uint32_t reserved; /* must be 0 */
    uint64_t ne[4];
    uint64_t nb[4];
    uint64_t data_bytes;
} emel_tensor_view;

typedef struct emel_tensor_view_mut {
    void *data;
    uint32_t dtype;
    uint32_t reserved; /* must be 0 */
    uint64_t ne[4];
    uint64_t nb[4];
    uint64_t data_bytes;
} emel_tensor_view_mut;

typedef void *emel_stream; /* hipStream_t */

/* ---- library / runtime (the FFI crate's device plumbing) ------------- */

uint32_t emel_abi_version(void);
const char *emel_status_string(emel_status status);
/* Detail of the last failure on the calling thread ("" if none). */
const char *emel_last_error(void);
/* Number of visible gfx950 devices (0 when none). */
emel_status emel_device_count(int32_t *count);
emel_status emel_set_device(int32_t device);
emel_status emel_malloc(void **ptr, uint64_t bytes);
emel_status emel_free(void *ptr);
emel_status emel_memcpy_htod(void *dst, const void *src, uint64_t bytes, emel_stream stream);
emel_status emel_memcpy_dtoh(void *dst, const void *src, uint64_t bytes, emel_stream stream);
emel_status emel_stream_create(emel_stream *stream);
emel_status emel_stream_destroy(emel_stream stream);
emel_status emel_stream_synchronize(emel_stream stream);
/* Releases the per-stream reduction workspaces the library holds. */
emel_status emel_release_workspaces(void);

/* Set-up for dispatch that neither allocates nor waits, no counterpart in
 * the reference (whose dispatch never allocates): for callers that capture
 * calls into HIP graphs or run tight serving loops.
 *   emel_stream_reserve grows the scratch that calls on `stream` share (on
 *   the current device) to at least `work_bytes` of workspace and
 *   `counter_bytes` of zeroed reduction counters.  Later calls on the stream
 *   that need no more allocate nothing.  It allocates, and zeroes the
 *   counters on the stream, so it is refused under capture
 *   (EMEL_ERR_STREAM_CAPTURE).
 *   emel_stream_workspace reports the sizes the stream holds now: after one
 *   eager run of a workload they are what that workload needs, for
 *   emel_stream_reserve in a later process.
 *   emel_device_prepare builds the current device's lookup tables (GELU's)
 *   and waits for them, so no later call waits to build them. */
emel_status emel_stream_reserve(emel_stream stream, uint64_t work_bytes, uint64_t counter_bytes);
emel_status emel_stream_workspace(emel_stream stream, uint64_t *work_bytes, uint64_t *counter_bytes);
emel_status emel_device_prepare(emel_stream stream);

/* Measurement reference, no counterpart in the reference: a bit copy of
 * `bytes` device bytes (a multiple of 16, both pointers 16-byte aligned)
 * with one of the streaming shapes the dense kernels use, so a caller can
 * time what a plain stream achieves at a given size.  Asynchronous on
 * `stream`. */
typedef enum emel_copy_shape {
    EMEL_COPY_FLAT = 0,  /* one float4 per thread */
    EMEL_COPY_WAVE4 = 1, /* four float4 per lane, each wave over 256 consecutive float4 */
    EMEL_COPY_WAVE8 = 2, /* eight float4 per lane, each wave over 512 consecutive float4 */
    EMEL_COPY_WALK = 3   /* one resident generation, grid-stride, next float4 in flight */
} emel_copy_shape;
emel_status emel_stream_copy(const void *src, void *dst, uint64_t bytes, uint32_t shape, emel_stream stream);

/* ---- view predicates (host only, no device access) -------------------- */

/* Layout::validate / validate_binary (tensor_view.rs:365-447):
 * allow_singleton_zero_stride != 0 selects the binary-kernel contract. */
emel_status emel_validate_view(const emel_tensor_view *view, int32_t allow_singleton_zero_stride);
/* normalization_view_valid (normalization.rs:237-287). */
emel_status emel_validate_normalization_view(const emel_tensor_view *view);

/* ---- equal-count binary ops --------------------------------------------
 * binary::{OpAdd,OpSub,OpMul,OpDiv}::new(lhs, rhs, output)
 * (binary.rs:47-81; guards :320-340; formulas :383-409; loop :411-424):
 * the three views have equal element counts (shapes may differ) and are
 * paired by logical ordinal.  Bit-exact IEEE f32. */
emel_status emel_op_add(const emel_tensor_view *lhs, const emel_tensor_view *rhs,
                        const emel_tensor_view_mut *out, emel_stream stream);
emel_status emel_op_sub(const emel_tensor_view *lhs, const emel_tensor_view *rhs,
                        const emel_tensor_view_mut *out, emel_stream stream);
emel_status emel_op_mul(const emel_tensor_view *lhs, const emel_tensor_view *rhs,
                        const emel_tensor_view_mut *out, emel_stream stream);
emel_status emel_op_div(const emel_tensor_view *lhs, const emel_tensor_view *rhs,
                        const emel_tensor_view_mut *out, emel_stream stream);

/* ---- row broadcast -------------------------------------------------------
 * broadcast::{OpAddBroadcastRow,OpMulBroadcastRow}::new(src0, src1, dst)
 * (broadcast.rs:53-84; shape rule :334-350; loops :352-390):
 * dst[r,c] = src0[r,c] (+|*) src1[c], src1.ne == [dst.ne0,1,1,1]. */
emel_status emel_op_add_broadcast_row(const emel_tensor_view *src0, const emel_tensor_view *src1,
                                      const emel_tensor_view_mut *dst, emel_stream stream);
emel_status emel_op_mul_broadcast_row(const emel_tensor_view *src0, const emel_tensor_view *src1,
                                      const emel_tensor_view_mut *dst, emel_stream stream);

/* ---- 4-D modulo broadcast ------------------------------------------------
 * Replaces the reference composition OpRepeat(src1 -> dst.ne)
 * (generic.rs:1641-1665, guard :964-983) followed by the equal-count binary
 * op (binary.rs:411-424): dst[i] = src0[i] op src1[i0%n0,i1%n1,i2%n2,i3%n3]
 * with src0.ne == dst.ne and each src1.ne[d] dividing dst.ne[d]. */
emel_status emel_op_binary_broadcast(emel_binary_op op, const emel_tensor_view *src0,
                                     const emel_tensor_view *src1, const emel_tensor_view_mut *dst,
                                     emel_stream stream);

/* ---- unary ----------------------------------------------------------------
 * unary::OpUnary::new(subop, input, output) (unary.rs:150-172, guards
 * :985-1027): accepts abs, neg, tanh, elu, relu, gelu, silu, exp; any
 * failed guard reports EMEL_ERR_UNEXPECTED_EVENT, as OpUnary does. */
emel_status emel_op_unary(emel_unary_subop subop, const emel_tensor_view *in,
                          const emel_tensor_view_mut *out, emel_stream stream);
/* unary::OpSilu::new(input, output) (unary.rs:82, formula :595-600):
 * x / (1 + expf(-x)) with expf bit-identical to glibc's. */
emel_status emel_op_silu(const emel_tensor_view *in, const emel_tensor_view_mut *out, emel_stream stream);
/* unary::OpGelu::new(input, output) (unary.rs:80, formula :522-586):
 * fp16-rounded tanh approximation with tanhf bit-identical to glibc's. */
emel_status emel_op_gelu(const emel_tensor_view *in, const emel_tensor_view_mut *out, emel_stream stream);
/* The typed unary events unary::{OpAbs, OpSgn, OpNeg, OpStep, OpTanh, OpElu,
 * OpRelu, OpSigmoid, OpGelu, OpGeluQuick, OpSilu, OpHardswish,
 * OpHardsigmoid, OpExp, OpExpm1, OpSoftplus, OpGeluErf, OpFloor, OpCeil,
 * OpRound, OpTrunc}::new(input, output) (unary.rs:72-92), selected by the
 * UnarySubOp code of their formula (unary.rs:472-610): event is an
 * emel_unary_subop other than EMEL_UNARY_XIELU, which has no typed event
 * (EMEL_ERR_UNEXPECTED_EVENT).  Guards (impl_unary_context, unary.rs:702-728):
 * both views valid, else INVALID_VIEW; equal element counts, else
 * SHAPE_MISMATCH; applied by logical ordinal.  exp, expm1, tanh and ln_1p are
 * bit-identical to glibc's expf, expm1f, tanhf and log1pf. */
emel_status emel_op_unary_event(uint32_t event, const emel_tensor_view *in, const emel_tensor_view_mut *out,
                                emel_stream stream);
/* reductions::{OpLog, OpSin, OpCos}::new(src, dst) (reductions.rs:45-90,
 * guards :508-517, effects :640-668): f32::ln / sin / cos elementwise by
 * ordinal, bit-identical to glibc's logf / sinf / cosf.  Views valid, else
 * INVALID_VIEW; equal element counts, else SHAPE_MISMATCH. */
emel_status emel_op_log(const emel_tensor_view *in, const emel_tensor_view_mut *out, emel_stream stream);
emel_status emel_op_sin(const emel_tensor_view *in, const emel_tensor_view_mut *out, emel_stream stream);
emel_status emel_op_cos(const emel_tensor_view *in, const emel_tensor_view_mut *out, emel_stream stream);
/* Fused SwiGLU: the reference chain OpSilu(gate) then equal-count OpMul by
 * up (unary.rs:595-600, binary.rs:411-424) in one pass, keeping both f32
 * roundings.  The three views have identical shapes. */
emel_status emel_op_swiglu(const emel_tensor_view *gate, const emel_tensor_view *up,
                           const emel_tensor_view_mut *out, emel_stream stream);

/* ---- dense-slice root events ----------------------------------------------------
 * The root kernel's contiguous-buffer events (event.rs:133-259, :523-568):
 * event::OpDup (copy), event::OpAdd / OpSub / OpMul / OpDiv and event::OpSqr
 * / OpSqrt, each over caller slices of `len` floats.  Guards (actor.rs:
 * 2498-2560; op_sqr / op_sqrt :1521-1555 with dense_power_layout :122-125):
 * every length non-zero and all lengths equal, otherwise the root
 * Error::InvalidShape (EMEL_ERR_INVALID_SHAPE).  An output that partially
 * overlaps an input (impossible for Rust's borrowed slices) is
 * EMEL_ERR_INVALID_ARGUMENT; the output may be exactly an input. */
emel_status emel_slice_dup(const float *input, uint64_t input_len, float *output, uint64_t output_len,
                           emel_stream stream);
emel_status emel_slice_add(const float *lhs, uint64_t lhs_len, const float *rhs, uint64_t rhs_len, float *output,
                           uint64_t output_len, emel_stream stream);
emel_status emel_slice_sub(const float *lhs, uint64_t lhs_len, const float *rhs, uint64_t rhs_len, float *output,
                           uint64_t output_len, emel_stream stream);
emel_status emel_slice_mul(const float *lhs, uint64_t lhs_len, const float *rhs, uint64_t rhs_len, float *output,
                           uint64_t output_len, emel_stream stream);
emel_status emel_slice_div(const float *lhs, uint64_t lhs_len, const float *rhs, uint64_t rhs_len, float *output,
                           uint64_t output_len, emel_stream stream);
emel_status emel_slice_sqr(const float *input, uint64_t input_len, float *output, uint64_t output_len,
                           emel_stream stream);
emel_status emel_slice_sqrt(const float *input, uint64_t input_len, float *output, uint64_t output_len,
                            emel_stream stream);

/* ---- square and square root over views -----------------------------------------
 * power::OpSqr / OpSqrt::new(input, output) (power.rs:46-73; guards
 * :266-273; v * v and IEEE sqrt(v) over logical ordinals): both views must
 * validate (EMEL_ERR_INVALID_VIEW) and hold equal element counts
 * (EMEL_ERR_SHAPE_MISMATCH), as PowerError reports them. */
emel_status emel_op_sqr(const emel_tensor_view *in, const emel_tensor_view_mut *out, emel_stream stream);
emel_status emel_op_sqrt(const emel_tensor_view *in, const emel_tensor_view_mut *out, emel_stream stream);

/* ---- gated linear units --------------------------------------------------------
 * glu::OpGlu::new(input, output, subop) (glu.rs:69-92; split_len :85-91;
 * gates :103-129; apply_split :131-141; SwiGluOai :258-270): input is a dense
 * slice of input_len floats, values in its first half and gates in its
 * second; output gets input_len / 2 floats, output[i] = values[i] *
 * gate(gates[i]).  GluError::InvalidShape (empty or odd input, output not
 * half of it) is EMEL_ERR_SHAPE_MISMATCH; an unknown subop code is
 * EMEL_ERR_UNEXPECTED_EVENT (no transition of the reference's machine
 * accepts it); output overlapping input (impossible for Rust's borrowed
 * slices) is EMEL_ERR_INVALID_ARGUMENT.  Lengths count floats. */
emel_status emel_op_glu(emel_glu_subop subop, const float *input, uint64_t input_len, float *output,
                        uint64_t output_len, emel_stream stream);

/* ---- scale ------------------------------------------------------------------
 * activation::OpScale::new(input, output, scale) (activation.rs:58-72,
 * guard :352-364, loop :366-377). */
emel_status emel_op_scale(const emel_tensor_view *in, const emel_tensor_view_mut *out, float scale,
                          emel_stream stream);

/* ---- row normalization -------------------------------------------------------
 * normalization::OpRmsNorm::new(input, output, epsilon)
 * (normalization.rs:80-96; guards :364-386; run_rms_norm :343-362):
 * per row, s = sum_f64(f32(x*x)), k = 1/sqrtf(f32(s/n) + eps), y = x*k. */
emel_status emel_op_rms_norm(const emel_tensor_view *in, const emel_tensor_view_mut *out, float epsilon,
                             emel_stream stream);
/* Fused rms_norm then OpMulBroadcastRow by weight (broadcast.rs:372-390):
 * y = (x*k)*w[c], two f32 roundings.  Both ops' guards are checked first. */
emel_status emel_op_rms_norm_mul(const emel_tensor_view *in, const emel_tensor_view *weight,
                                 const emel_tensor_view_mut *out, float epsilon, emel_stream stream);
/* normalization::OpNorm::new(input, output, epsilon) (run_norm :316-341). */
emel_status emel_op_norm(const emel_tensor_view *in, const emel_tensor_view_mut *out, float epsilon,
                         emel_stream stream);

/* ---- row reductions ------------------------------------------------------------
 * reductions::OpSoftMax::new(src, dst) (reductions.rs:152-163; shape
 * :473-495; dense f64-sum path :565-601; strided f32-sum path :603-638). */
emel_status emel_op_soft_max(const emel_tensor_view *src, const emel_tensor_view_mut *dst, emel_stream stream);
/* Scaled + masked soft_max: the reference composition OpScale
 * (activation.rs:372) -> equal-count OpAdd of the f16 mask decoded by
 * fp16_to_f32 (quant.rs:287-300) -> dense OpSoftMax, per (ne2,ne3) slice.
 * mask (may be NULL) is dense f16 [ne0, ne1, m2, m3], m2 | ne2, m3 | ne3. */
emel_status emel_op_soft_max_ext(const emel_tensor_view *src, const emel_tensor_view *mask, float scale,
                                 const emel_tensor_view_mut *dst, emel_stream stream);
/* reductions::OpSumRows::new(src, dst) (reductions.rs:107-118, :460-463,
 * :684-700): dst.ne == [1, ne1, ne2, ne3], f64 accumulation. */
emel_status emel_op_sum_rows(const emel_tensor_view *src, const emel_tensor_view_mut *dst, emel_stream stream);
/* reductions::OpSum / OpMean (reductions.rs:88-133, :670-713): scalar dst. */
emel_status emel_op_sum(const emel_tensor_view *src, const emel_tensor_view_mut *dst, emel_stream stream);
emel_status emel_op_mean(const emel_tensor_view *src, const emel_tensor_view_mut *dst, emel_stream stream);
/* reductions::OpArgmax::new(src, dst) (reductions.rs:137-148, :715-730):
 * whole tensor -> f32 scalar index of the first maximum. */
emel_status emel_op_argmax(const emel_tensor_view *src, const emel_tensor_view_mut *dst, emel_stream stream);
/* Per-row argmax: one OpArgmax per row view ne=[ne0,1,1,1]; dst is I32
 * with ne == [1, ne1, ne2, ne3] (first maximum; NaN never wins; a NaN in
 * column 0 yields 0, exactly as the sequential strict-> scan). */
emel_status emel_op_argmax_rows(const emel_tensor_view *src, const emel_tensor_view_mut *dst,
                                emel_stream stream);
/* ---- typed events of activation.rs, elementwise.rs, diag.rs, group_norm.rs ---- */

/* activation::OpClamp::new(input, output, min, max) (activation.rs:78-96,
 * effect :403-421): std::clamp's comparisons -- below min gives min, else
 * above max gives max, NaN passes through.  activation::OpLeakyRelu::new(
 * input, output, negative_slope) (:118-140): x < 0 ? x * slope : x.
 * activation::OpSiluBack::new(input, gradient, output) (:98-116, :467-480):
 * gradient * s (1 + x (1 - s)), s = 1 / (1 + expf(-x)).  Guards: views valid,
 * else INVALID_VIEW; identical extents, else SHAPE_MISMATCH. */
emel_status emel_op_clamp(const emel_tensor_view *in, const emel_tensor_view_mut *out, float min, float max,
                          emel_stream stream);
emel_status emel_op_leaky_relu(const emel_tensor_view *in, const emel_tensor_view_mut *out, float negative_slope,
                               emel_stream stream);
emel_status emel_op_silu_back(const emel_tensor_view *in, const emel_tensor_view *gradient,
                              const emel_tensor_view_mut *out, emel_stream stream);
/* elementwise::OpAdd1::new(src, scalar, dst) (elementwise.rs:51-62, :262-271):
 * dst = src + scalar; views valid, identical extents. */
emel_status emel_op_add1(const emel_tensor_view *src, float scalar, const emel_tensor_view_mut *dst,
                         emel_stream stream);
/* elementwise::OpAcc::new(base, update, dst, offset) (elementwise.rs:64-80,
 * guards :216-243, effect :273-288): dst = base, then dst[offset + i] +=
 * update[i].  base and dst identical extents (SHAPE_MISMATCH); all three dense
 * F32 (INVALID_VIEW); offset + count(update) <= count(dst) (INVALID_OFFSET).
 * dst may be base itself. */
emel_status emel_op_acc(const emel_tensor_view *base, const emel_tensor_view *update, const emel_tensor_view_mut *dst,
                        uint64_t offset, emel_stream stream);
/* diag::OpDiag::new(input, output) (diag.rs:38-65, :332-344): output (n*n,
 * zeroed) gets input on its diagonal; input_len > 0 and output_len == n*n,
 * else INVALID_SHAPE.  diag::OpDiagMaskInf / OpDiagMaskZero::new(input,
 * output, n_past) (:67-105, :144-160): a square matrix copied with -inf / 0
 * where column > row + n_past; n_past >= 0, equal lengths, a square length,
 * else INVALID_SHAPE.  The slices are device memory; the masks may run in
 * place. */
emel_status emel_op_diag(const float *input, uint64_t input_len, float *output, uint64_t output_len,
                         emel_stream stream);
emel_status emel_op_diag_mask_inf(const float *input, uint64_t input_len, float *output, uint64_t output_len,
                                  int32_t n_past, emel_stream stream);
emel_status emel_op_diag_mask_zero(const float *input, uint64_t input_len, float *output, uint64_t output_len,
                                   int32_t n_past, emel_stream stream);
/* group_norm::OpGroupNorm::new(input, output, groups, epsilon)
 * (group_norm.rs:49-66, guards :179-196, run_group_norm :205-241): per batch
 * and group of C/groups channels of a [W, H, C, B] view, mean and variance of
 * the group's f32 elements summed in f64, y = (x - mean) / sqrt(var + eps).
 * INVALID_VIEW (normalization_view_valid), SHAPE_MISMATCH, INVALID_PARAMETERS
 * (groups 0 or not dividing C, epsilon negative or not finite).  Within 1e-5
 * of the sequential f64 sums. */
emel_status emel_op_group_norm(const emel_tensor_view *in, const emel_tensor_view_mut *out, uint64_t groups,
                               float epsilon, emel_stream stream);
/* group_norm::OpL2Norm::new(input, output) (group_norm.rs:68-78, :244-268):
 * y = x / sqrt(sum of x*x), the sum sequential in f32 over the whole view.
 * A sum that is not positive is EMEL_ERR_ZERO_NORM with nothing written: the
 * call reads the sum back and waits for it, so it cannot be captured
 * (EMEL_ERR_STREAM_CAPTURE). */
emel_status emel_op_l2_norm(const emel_tensor_view *in, const emel_tensor_view_mut *out, emel_stream stream);

/* emel_op_argmax_rows without any allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  Same guards, statuses and results as emel_op_argmax_rows;
 * the split-row partials and arrival counters live in a static 128 KiB
 * per-device array (64 KiB counters, 64 KiB partials), set up on the
 * device's first call.  Every shape argmax_rows accepts fits; a plan that
 * did not would return EMEL_ERR_INVALID_PARAMETERS.  All calls on one
 * device share that array: calls that overlap on the device (concurrent
 * streams, or graphs replayed concurrently) race and must be serialised by
 * the caller.  A race can leave a row's arrival counter non-zero; every
 * later call on that device then merges the wrong partials and returns
 * wrong indices with no error, until the process ends (a new process
 * starts with the array zeroed).  The first call on a device may be made
 * under HIP graph capture: its set-up kernel is captured with it. */
emel_status emel_op_argmax_rows_no_alloc(const emel_tensor_view *src, const emel_tensor_view_mut *dst,
                                         emel_stream stream);

/* ---- row gather -----------------------------------------------------------------
 * get_rows::OpGetRows / OpGetRowsF32Bytes / OpGetRowsF16 / OpGetRowsBf16 /
 * OpGetRowsQ4_0 / OpGetRowsQ8_0 / OpGetRowsQ4K::new(source, indices,
 * destination) (get_rows.rs:219-510; guards :855-1452; actions :1453-2003):
 * dst row (i0, i1, i2) = source row indices[i0, i1, i2] of batch (i1, i2),
 * converted to f32.  dst is dense F32 [src.ne0, idx.ne0, idx.ne1, idx.ne2];
 * src.ne2 == idx.ne1 and src.ne3 == idx.ne2.
 *
 * The index tensor mirrors IndexView (get_rows.rs:42-196): int32 values,
 * three extents, byte strides.  explicit_strides == 0 is IndexView::new
 * (row-major); 1 is IndexView::with_strides (nb[0] == 0 still selects
 * row-major).  len counts int32 elements at data (the Rust slice length).
 *
 * The reference checks every index against the source row count before
 * writing anything, and so does every call here, on the host:
 *   on_host == 1: data is host memory, as the reference's &[i32] is.  The
 *     indices are checked in place; up to EMEL_GET_ROWS_INLINE_INDICES of
 *     them then travel to the kernel inside its launch arguments (the call
 *     is asynchronous and can be captured into a HIP graph, which then
 *     replays the indices it was captured with); more are uploaded, and the
 *     call waits for that copy.
 *   on_host == 0: data is device memory.  The call copies the index span
 *     to the host on `stream` and waits for it before checking.
 * Statuses: INVALID_VIEW, SHAPE_MISMATCH, UNSUPPORTED_SOURCE_STRIDE (F32
 * only), INDEX_OUT_OF_BOUNDS, in the reference's guard order. */
#define EMEL_GET_ROWS_INLINE_INDICES 512u
typedef struct emel_index_view {
    const int32_t *data;
    uint64_t len;     /* int32 elements at data */
    uint64_t ne[3];
    uint64_t nb[3];   /* byte strides (explicit_strides == 1) */
    uint32_t explicit_strides;
    uint32_t on_host; /* 1: data is host memory; 0: device memory */
} emel_index_view;

/* F32 source: rows located by nb[1..3]; each row copies ne0 contiguous
 * floats from its start (the pinned memcpy, whatever nb[0] is). */
emel_status emel_op_get_rows(const emel_tensor_view *src, const emel_index_view *indices,
                             const emel_tensor_view_mut *dst, emel_stream stream);
/* F32 source read byte-wise: outer byte strides need not be multiples of 4. */
emel_status emel_op_get_rows_f32_bytes(const emel_tensor_view *src, const emel_index_view *indices,
                                       const emel_tensor_view_mut *dst, emel_stream stream);
/* F16 / BF16 sources (dtype 1 / 30), element-strided, widened exactly. */
emel_status emel_op_get_rows_f16(const emel_tensor_view *src, const emel_index_view *indices,
                                 const emel_tensor_view_mut *dst, emel_stream stream);
emel_status emel_op_get_rows_bf16(const emel_tensor_view *src, const emel_index_view *indices,
                                  const emel_tensor_view_mut *dst, emel_stream stream);
/* Packed quantized sources (dtype 2 / 8 / 12, nb = [1, row bytes, ...]):
 * Q4_0 and Q8_0 blocks of 32 values (quant.rs:71-206), Q4_K blocks of 256
 * (quant_more.rs:402-469, scale/min unpacking :952-961). */
emel_status emel_op_get_rows_q4_0(const emel_tensor_view *src, const emel_index_view *indices,
                                  const emel_tensor_view_mut *dst, emel_stream stream);
emel_status emel_op_get_rows_q8_0(const emel_tensor_view *src, const emel_index_view *indices,
                                  const emel_tensor_view_mut *dst, emel_stream stream);
emel_status emel_op_get_rows_q4_k(const emel_tensor_view *src, const emel_index_view *indices,
                                  const emel_tensor_view_mut *dst, emel_stream stream);

/* ---- generic wire envelope ----------------------------------------------------
 * event::GenericEvent::new(GenericRequest::new(operation, src0, src1, src2,
 * dst, OpParams).with_unary(..).with_index_out(..)) (generic.rs:634-797):
 * the pinned emel.cpp operation struct, one entry point for every opcode.
 *
 * Operation codes: KernelOperation (generic.rs:24-337), 95 entries. */
typedef enum emel_generic_op {
    EMEL_GENERIC_DUP = 0, EMEL_GENERIC_ADD, EMEL_GENERIC_ADD_ID, EMEL_GENERIC_ADD1, EMEL_GENERIC_ACC,
    EMEL_GENERIC_SUB, EMEL_GENERIC_MUL, EMEL_GENERIC_DIV, EMEL_GENERIC_SQR, EMEL_GENERIC_SQRT,
    EMEL_GENERIC_LOG, EMEL_GENERIC_SIN, EMEL_GENERIC_COS, EMEL_GENERIC_SUM, EMEL_GENERIC_SUM_ROWS,
    EMEL_GENERIC_CUMSUM, EMEL_GENERIC_MEAN, EMEL_GENERIC_ARGMAX, EMEL_GENERIC_COUNT_EQUAL, EMEL_GENERIC_REPEAT,
    EMEL_GENERIC_REPEAT_BACK, EMEL_GENERIC_CONCAT, EMEL_GENERIC_SILU_BACK, EMEL_GENERIC_NORM,
    EMEL_GENERIC_RMS_NORM, EMEL_GENERIC_RMS_NORM_BACK, EMEL_GENERIC_GROUP_NORM, EMEL_GENERIC_L2_NORM,
    EMEL_GENERIC_MUL_MAT, EMEL_GENERIC_MUL_MAT_ARGMAX, EMEL_GENERIC_MUL_MAT_ID, EMEL_GENERIC_OUT_PROD,
    EMEL_GENERIC_SCALE, EMEL_GENERIC_SET, EMEL_GENERIC_CPY, EMEL_GENERIC_CONT, EMEL_GENERIC_RESHAPE,
    EMEL_GENERIC_VIEW, EMEL_GENERIC_PERMUTE, EMEL_GENERIC_TRANSPOSE, EMEL_GENERIC_GET_ROWS,
    EMEL_GENERIC_GET_ROWS_BACK, EMEL_GENERIC_SET_ROWS, EMEL_GENERIC_DIAG, EMEL_GENERIC_DIAG_MASK_INF,
    EMEL_GENERIC_DIAG_MASK_ZERO, EMEL_GENERIC_SOFT_MAX, EMEL_GENERIC_SOFT_MAX_BACK, EMEL_GENERIC_ROPE,
    EMEL_GENERIC_ROPE_BACK, EMEL_GENERIC_CLAMP, EMEL_GENERIC_CONV_TRANSPOSE_1D, EMEL_GENERIC_IM2COL,
    EMEL_GENERIC_IM2COL_BACK, EMEL_GENERIC_IM2COL_3D, EMEL_GENERIC_CONV_2D, EMEL_GENERIC_CONV_3D,
    EMEL_GENERIC_CONV_2D_DW, EMEL_GENERIC_CONV_TRANSPOSE_2D, EMEL_GENERIC_POOL_1D, EMEL_GENERIC_POOL_2D,
    EMEL_GENERIC_POOL_2D_BACK, EMEL_GENERIC_UPSCALE, EMEL_GENERIC_PAD, EMEL_GENERIC_PAD_REFLECT_1D,
    EMEL_GENERIC_ROLL, EMEL_GENERIC_ARANGE, EMEL_GENERIC_TIMESTEP_EMBEDDING, EMEL_GENERIC_ARGSORT,
    EMEL_GENERIC_TOP_K, EMEL_GENERIC_LEAKY_RELU, EMEL_GENERIC_TRI, EMEL_GENERIC_FILL,
    EMEL_GENERIC_FLASH_ATTN_EXT, EMEL_GENERIC_FLASH_ATTN_BACK, EMEL_GENERIC_SSM_CONV, EMEL_GENERIC_SSM_SCAN,
    EMEL_GENERIC_WIN_PART, EMEL_GENERIC_WIN_UNPART, EMEL_GENERIC_GET_REL_POS, EMEL_GENERIC_ADD_REL_POS,
    EMEL_GENERIC_RWKV_WKV6, EMEL_GENERIC_GATED_LINEAR_ATTN, EMEL_GENERIC_RWKV_WKV7, EMEL_GENERIC_SOLVE_TRI,
    EMEL_GENERIC_UNARY, EMEL_GENERIC_MAP_CUSTOM1, EMEL_GENERIC_MAP_CUSTOM2, EMEL_GENERIC_MAP_CUSTOM3,
    EMEL_GENERIC_CUSTOM, EMEL_GENERIC_CROSS_ENTROPY_LOSS, EMEL_GENERIC_CROSS_ENTROPY_LOSS_BACK,
    EMEL_GENERIC_OPT_STEP_ADAMW, EMEL_GENERIC_OPT_STEP_SGD, EMEL_GENERIC_GLU,
    EMEL_GENERIC_OPERATION_COUNT /* 95, GENERIC_OPERATION_COUNT (generic.rs:19) */
} emel_generic_op;

/* The pinned operation struct (tools/emel-kernel-*-reference/main.cpp:
 * tensor_view src0/src1/src2/dst, op_params[64] + op_params_size, subop,
 * index_out).  Absent views are NULL.  Views of any wire dtype (0..255) are
 * accepted for validation; data pointers are device pointers, and so is
 * index_out (op_mul_mat_argmax's row, written on the device). */
typedef struct emel_generic_request {
    uint32_t operation;   /* emel_generic_op */
    uint32_t unary_subop; /* UnarySubOp wire code, read by EMEL_GENERIC_UNARY (0..21) */
    uint32_t glu_subop;   /* GluSubOp wire code (carried; no maintained route reads it) */
    uint32_t pool_subop;  /* PoolSubOp wire code (carried; no maintained route reads it) */
    const emel_tensor_view *src0;
    const emel_tensor_view *src1;
    const emel_tensor_view *src2;
    const emel_tensor_view_mut *dst;
    uint8_t op_params[64];
    uint32_t op_params_size; /* initialised prefix of op_params, <= 64 */
    uint32_t reserved;       /* must be 0 */
    int32_t *index_out;      /* NULL when absent */
} emel_generic_request;

/* Dispatch in the reference machine's order (sm.rs:318-426, guards
 * actor.rs:2655-2983):
 *   1. the operation's maintained F32 route (generic.rs:848-1262) passes ->
 *      executed on the device (formulas generic.rs:1264-2055);
 *   2. else the request validates (GenericRequest::validate, :769-789) but a
 *      maintained operation's predicate fails -> EMEL_ERR_INVALID_SHAPE;
 *   3. else the request validates -> EMEL_ERR_UNSUPPORTED_OPERATION;
 *   4. else EMEL_ERR_INVALID_SHAPE.
 * Routed on the device: dup, add, sub, mul, div, add1, scale, clamp,
 * leaky_relu, silu_back, cumsum, repeat, repeat_back, concat, diag,
 * diag_mask_inf/zero, soft_max, soft_max_back, norm, rms_norm, rms_norm_back,
 * l2_norm, count_equal, fill, arange, sum, mean, argmax, sqr, sqrt, log, sin,
 * cos (glibc-exact logf/sinf/cosf), unary (abs, neg, tanh, elu, relu, gelu,
 * silu, exp), mul_mat (F32 and F16) and mul_mat_argmax.  Divergences, each
 * reported before anything is enqueued:
 *   - views the reference reads byte-wise but that are not element-aligned
 *     (an F32 data pointer or stride not a multiple of 4), and destinations
 *     whose elements may overlap one another, are
 *     EMEL_ERR_UNSUPPORTED_OPERATION;
 *   - a routed request whose last element extends past data_bytes (the
 *     reference checks one byte and then panics reading four) is
 *     EMEL_ERR_INVALID_SHAPE;
 *   - dst overlapping a source (impossible for Rust's borrowed slices) is
 *     EMEL_ERR_INVALID_ARGUMENT, except dst being exactly a source view for
 *     the per-element and per-row routes.
 * A NULL request, an operation code >= 95, a subop or dtype code outside its
 * wire range, op_params_size > 64 or reserved != 0 (none representable in
 * the reference's types) is EMEL_ERR_INVALID_ARGUMENT. */
emel_status emel_generic_dispatch(const emel_generic_request *request, emel_stream stream);

/* ---- emel-logits: native sampler and candidate validator ----------------------
 * crates/emel-logits/src/sampler/sm.rs and validator/sm.rs (paths below are
 * relative to crates/emel-logits/src/).  Buffers are device memory unless
 * marked HOST.  Lengths are element counts, the Rust slice lengths the
 * reference's guards read. */

/* Sampler::sample_temperature_top_k(SampleTemperatureTopK::new(card,
 * temperature, top_k, logits, sorted_indices, top_probabilities,
 * top_indices, random_state, selected_token_out, selected_score_out))
 * (sampler/sm.rs:148-195, :380-392).
 *
 * Guard (guard_temperature_valid, sm.rs:729-747): card > 0, 0 < top_k <=
 * card, temperature finite and > 0, logits_len and sorted_indices_len >=
 * card, top_probabilities_len and top_indices_len >= top_k, random_state
 * not a multiple of 2^31 - 1.  A failed guard is EMEL_ERR_INVALID_REQUEST
 * with nothing written.  Otherwise, in order (sm.rs:759-847):
 *   logits[i] *= 1/temperature; softmax in place (f32::max fold, expf,
 *   a sequential f32 sum -- reproduced exactly --, division);
 *   top_probabilities / top_indices = the top_k probabilities and their
 *   indices, descending by f32::total_cmp (equal probabilities by ascending
 *   index: the reference's sort_unstable leaves their order unspecified);
 *   slot j draws the (j+1)-th Park-Miller state (x16807 mod 2^31 - 1) and
 *   races top_probabilities[j] / -ln(state / 2^31); the first maximal race
 *   gives selected_token_out and selected_score_out.
 * random_state (HOST) is updated to the state after top_k draws before the
 * call returns.  sorted_indices is the reference's sort scratch: its first
 * top_k entries receive the ranked indices, the rest is not written.
 * The result guard (guard_temperature_result_valid, sm.rs:849-858: token in
 * [0, card) and score finite) is evaluated on the device and written to
 * status_out (EMEL_OK or EMEL_ERR_INVALID_REQUEST) when status_out is not
 * NULL; the outputs are written either way, as in the reference.
 * After the guard, NULL buffers, overlapping buffers, pointers that are not
 * 4-byte aligned and card > 2^31 - 1 are EMEL_ERR_INVALID_ARGUMENT (a NULL
 * request or random_state before it). */
typedef struct emel_sample_temperature_top_k_request {
    uint64_t card;
    float temperature;
    uint32_t reserved; /* must be 0 */
    uint64_t top_k;
    float *logits;                  uint64_t logits_len;            /* in place: probabilities on return */
    int32_t *sorted_indices;        uint64_t sorted_indices_len;
    float *top_probabilities;       uint64_t top_probabilities_len;
    int32_t *top_indices;           uint64_t top_indices_len;
    uint32_t *random_state;         /* HOST, read and updated */
    int32_t *selected_token_out;
    float *selected_score_out;
    int32_t *status_out;            /* may be NULL */
} emel_sample_temperature_top_k_request;

emel_status emel_sample_temperature_top_k(const emel_sample_temperature_top_k_request *request, emel_stream stream);

/* `rows` independent requests in one call (a batch of sequences sampled at
 * once): row r uses logits + r*logits_stride, sorted_indices +
 * r*sorted_stride, top_probabilities / top_indices + r*top_stride,
 * random_state[r], selected_token_out[r], selected_score_out[r] and
 * status_out[r].  The lengths in the request are the whole buffers'; every
 * row must fit (strides >= card resp. top_k).  The guard covers every row:
 * one failing row rejects the call. */
typedef struct emel_sample_rows {
    uint64_t rows;
    uint64_t logits_stride;
    uint64_t sorted_stride;
    uint64_t top_stride;
} emel_sample_rows;

emel_status emel_sample_temperature_top_k_rows(const emel_sample_temperature_top_k_request *request,
                                               const emel_sample_rows *rows, emel_stream stream);

/* Sampler::sample_preselected(SamplePreselected::new(vocab_size,
 * selected_token)) (sampler/sm.rs:129-146, :366-378, guard :685-695):
 * host-only; writes *token_out (HOST) on success. */
emel_status emel_sample_preselected(uint64_t vocab_size, int32_t selected_token, int32_t *token_out);

/* ValidatorError (validator/sm.rs:15-21) discriminants, as *error_out. */
typedef enum emel_validator_error {
    EMEL_VALIDATOR_NONE = 0,
    EMEL_VALIDATOR_INVALID_REQUEST = 1,
    EMEL_VALIDATOR_BACKEND_ERROR = 2,
    EMEL_VALIDATOR_INTERNAL_ERROR = 3,
    EMEL_VALIDATOR_UNTRACKED = 4
} emel_validator_error;

/* Validator::process_event(Build::new(logits, vocab_size, candidate_ids,
 * candidate_scores, candidate_capacity, candidate_count_out, error_out))
 * (validator/sm.rs:33-66, :170-230).  candidate_count_out and error_out are
 * HOST scalars: reset to 0 / NONE, then on a failed guard (vocab_size > 0,
 * candidate_capacity >= vocab_size, each slice length >= vocab_size and
 * below 2^31) 0 / INVALID_REQUEST with EMEL_ERR_INVALID_REQUEST.  Otherwise
 * candidate_ids[i] = i and candidate_scores[i] = logits[i] - max for
 * i < vocab_size, where max starts at logits[0] and moves on strictly
 * greater values; *candidate_count_out = vocab_size. */
emel_status emel_logits_validator_build(const float *logits, uint64_t logits_len, int32_t vocab_size,
                                        int32_t *candidate_ids, uint64_t candidate_ids_len,
                                        float *candidate_scores, uint64_t candidate_scores_len,
                                        int32_t candidate_capacity, int32_t *candidate_count_out,
                                        int32_t *error_out, emel_stream stream);

#ifdef __cplusplus
}
#endif
#endif
