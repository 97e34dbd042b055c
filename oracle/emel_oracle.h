/*
 * emel_oracle.h -- CPU restatement of the emel.rs portable ("any") kernel
 * path for the elementwise, broadcast and row-reduction ops.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker the HIP product is
 * compared against.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it.  The product (libemel_hip.so) never links,
 * loads or calls it.
 *
 * Every function restates the reference algorithm with the same rounding
 * order (compiled with -ffp-contract=off) and calls glibc expf/tanhf/sqrtf
 * exactly where Rust std's f32::exp/tanh/sqrt are called.  Reference paths
 * are relative to stateforward/emel.rs:crates/emel-kernels/src/any/.
 */
#ifndef EMEL_ORACLE_H
#define EMEL_ORACLE_H

#include <math.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Same memory layout as emel_tensor_view in include/emel_hip.h. */
typedef struct orc_view {
    void *data;          /* host pointer */
    uint32_t dtype;      /* wire dtype code: F32=0, F16=1, I32=26 */
    uint32_t reserved;
    uint64_t ne[4];
    uint64_t nb[4];
    uint64_t data_bytes; /* bytes owned at data (Rust slice len * 4) */
} orc_view;

/* Status codes: identical numbering to emel_status in include/emel_hip.h. */
enum {
    ORC_OK = 0,
    ORC_INVALID_VIEW = 1,
    ORC_SHAPE_MISMATCH = 2,
    ORC_INVALID_PARAMETERS = 3,
    ORC_UNEXPECTED_EVENT = 4,
    ORC_INVALID_ARGUMENT = 8,        /* a value no reference type can hold */
    ORC_INVALID_SHAPE = 9,           /* root Error::InvalidShape */
    ORC_UNSUPPORTED_OPERATION = 10,  /* root Error::UnsupportedOperation */
    ORC_INDEX_OUT_OF_BOUNDS = 11,    /* GetRowsError::IndexOutOfBounds */
    ORC_UNSUPPORTED_SOURCE_STRIDE = 12, /* GetRowsError::UnsupportedSourceStride */
    ORC_INVALID_REQUEST = 13,        /* emel-logits SamplerError / ValidatorError::InvalidRequest */
    ORC_INVALID_OFFSET = 15,         /* ElementwiseError::InvalidOffset */
    ORC_ZERO_NORM = 16,              /* GroupNormError::ZeroNorm */
    ORC_PANIC = 99,                  /* the reference's guard passes and its executor panics */
};

enum { ORC_ADD = 0, ORC_SUB = 1, ORC_MUL = 2, ORC_DIV = 3 };

/* View validation (tensor_view.rs:365-447, normalization.rs:237-287). */
int orc_layout_validate(const orc_view *v, int allow_singleton_zero_stride);
int orc_normalization_view_valid(const orc_view *v);

/* Ops.  Each returns an ORC_* status; dst is untouched on rejection. */
int orc_op_binary(int op, const orc_view *lhs, const orc_view *rhs, const orc_view *dst);
int orc_op_broadcast_row(int op, const orc_view *src0, const orc_view *src1, const orc_view *dst);
int orc_op_unary(int subop, const orc_view *in, const orc_view *out);       /* OpUnary */
int orc_op_unary_event(int subop, const orc_view *in, const orc_view *out); /* the 21 typed unary events */
int orc_op_log(const orc_view *in, const orc_view *out);                    /* reductions::OpLog */
int orc_op_sin(const orc_view *in, const orc_view *out);                    /* reductions::OpSin */
int orc_op_cos(const orc_view *in, const orc_view *out);                    /* reductions::OpCos */
/* activation.rs, elementwise.rs, diag.rs, group_norm.rs typed events. */
int orc_op_clamp(const orc_view *in, const orc_view *out, float min, float max);
int orc_op_leaky_relu(const orc_view *in, const orc_view *out, float slope);
int orc_op_silu_back(const orc_view *in, const orc_view *grad, const orc_view *out);
int orc_op_add1(const orc_view *src, float scalar, const orc_view *dst);
int orc_op_acc(const orc_view *base, const orc_view *update, const orc_view *dst, uint64_t offset);
int orc_op_diag(const float *in, uint64_t in_len, float *out, uint64_t out_len);
int orc_op_diag_mask(int inf, const float *in, uint64_t in_len, float *out, uint64_t out_len, int32_t n_past);
int orc_op_group_norm(const orc_view *in, const orc_view *out, uint64_t groups, float eps);
int orc_op_l2_norm(const orc_view *in, const orc_view *out);
int orc_op_scale(const orc_view *in, const orc_view *out, float scale);
int orc_op_rms_norm(const orc_view *in, const orc_view *out, float eps);
int orc_op_norm(const orc_view *in, const orc_view *out, float eps);
int orc_op_soft_max(const orc_view *src, const orc_view *dst);
int orc_op_sum_rows(const orc_view *src, const orc_view *dst);
int orc_op_sum(const orc_view *src, const orc_view *dst);
int orc_op_mean(const orc_view *src, const orc_view *dst);
int orc_op_argmax(const orc_view *src, const orc_view *dst);
int orc_op_repeat(const orc_view *src, const orc_view *dst);

/* Compositions of reference ops (the configured semantics the reference has
 * no single op for).  Each is a sequence of the calls above. */
int orc_soft_max_ext(const orc_view *src, const orc_view *mask, float scale, const orc_view *dst);
int orc_argmax_rows(const orc_view *src, const orc_view *dst_i32);
int orc_binary_bcast(int op, const orc_view *src0, const orc_view *src1, const orc_view *dst);
int orc_rms_norm_mul(const orc_view *in, const orc_view *weight, const orc_view *out, float eps);
int orc_swiglu(const orc_view *gate, const orc_view *up, const orc_view *out);

/* Dense-slice root events (event.rs:133-259, :523-568; guards actor.rs:
 * 2498-2560, op_sqr/op_sqrt :1521-1555) and the view power ops (power.rs). */
int orc_slice_dup(const float *in, uint64_t in_len, float *out, uint64_t out_len);
int orc_slice_binary(int op, const float *lhs, uint64_t lhs_len, const float *rhs, uint64_t rhs_len, float *out,
                     uint64_t out_len);
int orc_slice_power(int sqrt_, const float *in, uint64_t in_len, float *out, uint64_t out_len);
int orc_op_power(int sqrt_, const orc_view *in, const orc_view *out);

/* OpGlu over a dense slice [values | gates] of 2n floats into n floats
 * (glu.rs:22-160, :258-270).  subop: GluSubOp wire code 0..5. */
enum { ORC_REGLU = 0, ORC_GEGLU = 1, ORC_SWIGLU = 2, ORC_SWIGLU_OAI = 3, ORC_GEGLU_ERF = 4, ORC_GEGLU_QUICK = 5 };
int orc_op_glu(int subop, const float *input, uint64_t input_len, float *output, uint64_t output_len);
float orc_glu_gate(int subop, float gate); /* the gate function alone (not SwiGluOai) */

/* The generic wire envelope (generic.rs, sm.rs:318-426), in
 * emel_oracle_generic.c.  Same layout as emel_generic_request in
 * include/emel_hip.h, with host pointers.  Returns ORC_OK, ORC_INVALID_SHAPE,
 * ORC_UNSUPPORTED_OPERATION or ORC_PANIC (a passed guard whose executor
 * reads or writes a partial last element). */
typedef struct orc_generic_request {
    uint32_t operation;
    uint32_t unary_subop;
    uint32_t glu_subop;
    uint32_t pool_subop;
    const orc_view *src0;
    const orc_view *src1;
    const orc_view *src2;
    const orc_view *dst;
    uint8_t op_params[64];
    uint32_t op_params_size;
    uint32_t reserved;
    int32_t *index_out;
} orc_generic_request;
int orc_generic(const orc_generic_request *request);

/* Row gather (get_rows.rs), in emel_oracle_getrows.c.  The index view has
 * the emel_index_view layout of include/emel_hip.h with a host pointer. */
typedef struct orc_index_view {
    const int32_t *data;
    uint64_t len; /* int32 elements */
    uint64_t ne[3];
    uint64_t nb[3];
    uint32_t explicit_strides;
    uint32_t reserved;
} orc_index_view;
enum { ORC_GR_F32 = 0, ORC_GR_F32_BYTES, ORC_GR_F16, ORC_GR_BF16, ORC_GR_Q4_0, ORC_GR_Q8_0, ORC_GR_Q4_K };
int orc_get_rows(int kind, const orc_view *src, const orc_index_view *indices, const orc_view *dst);

/* Rust f32::max / f32::min.  They lower to LLVM maxnum / minnum, which on
 * x86_64 return the other operand whenever one is NaN, signaling NaN
 * included; glibc fmaxf / fminf instead return a quieted NaN for a
 * signaling operand (IEEE 754-2008 maxNum).  Equal operands (+0 and -0)
 * are left to fmaxf / fminf: their sign is not pinned by the reference. */
static inline float rust_maxf(float a, float b) { return a != a ? b : (b != b ? a : fmaxf(a, b)); }
static inline float rust_minf(float a, float b) { return a != a ? b : (b != b ? a : fminf(a, b)); }

/* Scalar helpers (unary.rs:522-600, quant.rs:287-300). */
/* emel-logits (emel_oracle_sampler.c): the native temperature/top-k
 * sampler and the candidate validator, host slices. */
uint32_t orc_park_miller_next(uint32_t state);
float orc_sampler_softmax(float *values, uint64_t card);
int orc_sample_temperature_top_k(uint64_t card, float temperature, uint64_t top_k, float *logits,
                                 uint64_t logits_len, int32_t *sorted_indices, uint64_t sorted_len,
                                 float *top_probabilities, uint64_t top_probabilities_len, int32_t *top_indices,
                                 uint64_t top_indices_len, uint32_t *random_state, int32_t *selected_token_out,
                                 float *selected_score_out);
int orc_validator_build(const float *logits, uint64_t logits_len, int32_t vocab_size, int32_t *candidate_ids,
                        uint64_t ids_len, float *candidate_scores, uint64_t scores_len, int32_t candidate_capacity,
                        int32_t *candidate_count_out, int32_t *error_out);

float orc_silu(float x);
float orc_gelu(float x);
uint16_t orc_fp32_to_fp16(float x);
float orc_fp16_to_f32(uint16_t h);

#ifdef __cplusplus
}
#endif
#endif
