/*
 * emel_oracle.c -- CPU restatement of the emel.rs portable kernel path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the product).  See
 * emel_oracle.h.  Build: oracle/Makefile (gcc -O2 -ffp-contract=off).
 *
 * Reference file:line citations are relative to
 * stateforward/emel.rs:crates/emel-kernels/src/any/.
 *
 * Pinning (what checks each function against something other than itself):
 *   - golden output bits of the reference's parity manifests
 *     (snapshots/parity/kernel-{binary,broadcast,softmax,normalization,
 *     unary,elementwise,activation}/manifest.txt) and the reference's
 *     known-answer unit tests (files under tests/any/): tests/test_oracle_golden.py;
 *   - closed forms and invariants (numpy IEEE float32 ops, softmax row sums,
 *     argmax == lowest index of max, repeat-index formula, brute force on
 *     tiny shapes): tests/test_oracle_properties.py.
 *   - orc_soft_max_ext / orc_argmax_rows / orc_binary_bcast / orc_swiglu /
 *     orc_rms_norm_mul are compositions of pinned ops; each is additionally
 *     checked against its special-case reduction (zero mask + scale 1 ==
 *     OpSoftMax, src1 row shape == OpMulBroadcastRow, ...).
 */
#include "emel_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

typedef unsigned __int128 u128;

/* ------------------------------------------------------------------ */
/* Views (tensor_view.rs)                                              */
/* ------------------------------------------------------------------ */

#define DT_F32 0u
#define DT_F16 1u
#define DT_I32 26u

/* Layout::element_count, tensor_view.rs:343-357: zero extent -> None. */
static int element_count(const orc_view *v, uint64_t *count)
{
    u128 c = 1;
    for (int d = 0; d < 4; d++) {
        if (v->ne[d] == 0) return 0;
        c *= v->ne[d];
        if (c > (u128)UINT64_MAX) return 0;
    }
    *count = (uint64_t)c;
    return 1;
}

/* Layout::effective_f32_strides, tensor_view.rs:262-277: nb[0]==0 is the
 * implicit contiguous form; F32 only. */
static int effective_strides(const orc_view *v, uint64_t st[4])
{
    if (v->dtype != DT_F32) return 0;
    if (v->nb[0] != 0) {
        memcpy(st, v->nb, sizeof(uint64_t) * 4);
        return 1;
    }
    u128 s = 4;
    st[0] = 4;
    for (int d = 1; d < 4; d++) {
        s *= v->ne[d - 1];
        if (s > (u128)UINT64_MAX) return 0;
        st[d] = (uint64_t)s;
    }
    return 1;
}

/* Layout::validate_element_storage, tensor_view.rs:397-447. */
int orc_layout_validate(const orc_view *v, int allow_singleton_zero)
{
    uint64_t count, st[4];
    if (v->dtype != DT_F32) return ORC_INVALID_VIEW;
    if (!element_count(v, &count)) return ORC_INVALID_VIEW;
    if (!effective_strides(v, st)) return ORC_INVALID_VIEW;
    for (int d = 0; d < 4; d++) {
        int singleton_zero = allow_singleton_zero && v->ne[d] == 1 && st[d] == 0;
        if (!singleton_zero && (st[d] < 4 || st[d] % 4 != 0)) return ORC_INVALID_VIEW;
    }
    u128 max_offset = 0;
    for (int d = 0; d < 4; d++) max_offset += (u128)(v->ne[d] - 1) * st[d];
    if (max_offset + 4 > (u128)v->data_bytes) return ORC_INVALID_VIEW;
    return ORC_OK;
}

/* normalization_view_valid, normalization.rs:237-287. */
int orc_normalization_view_valid(const orc_view *v)
{
    uint64_t st[4];
    if (v->dtype != DT_F32 || v->ne[0] == 0) return 0;
    if (v->nb[0] != 0) {
        if (v->nb[0] < 4 || v->nb[0] % 4 != 0) return 0;
        for (int d = 0; d < 4; d++)
            if (v->ne[d] > 1 && v->nb[d] == 0) return 0;
    }
    for (int d = 0; d < 4; d++)
        if (v->ne[d] == 0) return 0;
    if (!effective_strides(v, st)) return 0;
    for (int d = 0; d < 4; d++)
        if (st[d] < 4 || st[d] % 4 != 0) return 0;
    u128 max_offset = 0;
    for (int d = 0; d < 4; d++) max_offset += (u128)(v->ne[d] - 1) * st[d];
    return max_offset + 4 <= (u128)v->data_bytes;
}

/* A validated view resolved for ordinal addressing (TensorView::new,
 * tensor_view.rs:690-701: count defaults to 0, strides to nb). */
typedef struct {
    float *data;
    uint64_t ne[4];
    uint64_t st[4];
    uint64_t count;
} rview;

static rview resolve(const orc_view *v)
{
    rview r;
    r.data = (float *)v->data;
    memcpy(r.ne, v->ne, sizeof r.ne);
    if (!effective_strides(v, r.st)) memcpy(r.st, v->nb, sizeof r.st);
    if (!element_count(v, &r.count)) r.count = 0;
    return r;
}

/* TensorView::element_index, tensor_view.rs:778-789. */
static inline uint64_t element_index(const rview *r, uint64_t ordinal)
{
    uint64_t rem = ordinal, off = 0;
    for (int d = 0; d < 4; d++) {
        off += (rem % r->ne[d]) * r->st[d];
        rem /= r->ne[d];
    }
    return off / 4;
}

static inline float rd(const rview *r, uint64_t ordinal) { return r->data[element_index(r, ordinal)]; }
static inline void wr(const rview *r, uint64_t ordinal, float v) { r->data[element_index(r, ordinal)] = v; }

static int same_ne(const orc_view *a, const orc_view *b)
{
    return memcmp(a->ne, b->ne, sizeof a->ne) == 0;
}

static uint64_t count_or_zero(const orc_view *v)
{
    uint64_t c;
    return element_count(v, &c) ? c : 0;
}

/* ------------------------------------------------------------------ */
/* Binary equal-count add/sub/mul/div (binary.rs:320-424)              */
/* ------------------------------------------------------------------ */

static inline float apply_binary(int op, float a, float b)
{
    switch (op) { /* binary.rs:383-409: plain IEEE operations */
    case ORC_ADD: return a + b;
    case ORC_SUB: return a - b;
    case ORC_MUL: return a * b;
    default: return a / b;
    }
}

int orc_op_binary(int op, const orc_view *lhs, const orc_view *rhs, const orc_view *dst)
{
    /* views_valid (binary.rs:320-331): validate_binary for all three. */
    if (orc_layout_validate(lhs, 1) || orc_layout_validate(rhs, 1) || orc_layout_validate(dst, 1))
        return ORC_INVALID_VIEW;
    /* shape_valid (binary.rs:333-340): equal logical element counts. */
    uint64_t n = count_or_zero(dst);
    if (count_or_zero(lhs) != count_or_zero(rhs) || count_or_zero(lhs) != n)
        return ORC_SHAPE_MISMATCH;
    rview a = resolve(lhs), b = resolve(rhs), o = resolve(dst);
    /* execute::<F> (binary.rs:411-424): loop over logical ordinals. */
    for (uint64_t k = 0; k < n; k++) wr(&o, k, apply_binary(op, rd(&a, k), rd(&b, k)));
    return ORC_OK;
}

/* ------------------------------------------------------------------ */
/* Row broadcast add/mul (broadcast.rs:321-390)                        */
/* ------------------------------------------------------------------ */

static int broadcast_row_guard(const orc_view *src0, const orc_view *src1, const orc_view *dst)
{
    if (orc_layout_validate(src0, 1) || orc_layout_validate(src1, 1) || orc_layout_validate(dst, 1))
        return ORC_INVALID_VIEW;
    /* shape_valid, broadcast.rs:334-350. */
    const uint64_t *d = dst->ne, *s1 = src1->ne;
    if (!(same_ne(src0, dst) && d[0] > 0 && s1[0] == d[0] && s1[1] == 1 && s1[2] == 1 && s1[3] == 1 &&
          d[1] > 0 && count_or_zero(dst) > count_or_zero(src1)))
        return ORC_SHAPE_MISMATCH;
    return ORC_OK;
}

int orc_op_broadcast_row(int op, const orc_view *src0, const orc_view *src1, const orc_view *dst)
{
    int s = broadcast_row_guard(src0, src1, dst);
    if (s) return s;
    rview a = resolve(src0), b = resolve(src1), o = resolve(dst);
    uint64_t cols = b.count, rows = o.count / cols;
    /* execute_{add,mul}_broadcast, broadcast.rs:352-390. */
    for (uint64_t r = 0; r < rows; r++)
        for (uint64_t c = 0; c < cols; c++) {
            uint64_t k = r * cols + c;
            wr(&o, k, apply_binary(op, rd(&a, k), rd(&b, c)));
        }
    return ORC_OK;
}

/* ------------------------------------------------------------------ */
/* fp16 conversion (unary.rs:546-586, quant.rs:287-300)                */
/* ------------------------------------------------------------------ */

static inline float f_from_bits(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
static inline uint32_t bits_from_f(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

uint16_t orc_fp32_to_fp16(float value)
{
    const float scale_to_inf = f_from_bits(0x77800000u);
    const float scale_to_zero = f_from_bits(0x08800000u);
    float base = (fabsf(value) * scale_to_inf) * scale_to_zero;
    uint32_t w = bits_from_f(value);
    uint32_t doubled = w + w;
    uint32_t sign = w & 0x80000000u;
    uint32_t bias = doubled & 0xff000000u;
    if (bias < 0x71000000u) bias = 0x71000000u;
    base += f_from_bits((bias >> 1) + 0x07800000u);
    uint32_t bb = bits_from_f(base);
    uint32_t exponent = (bb >> 13) & 0x00007c00u;
    uint32_t mantissa = bb & 0x00000fffu;
    uint32_t nonsign = exponent + mantissa;
    return (uint16_t)((sign >> 16) | (doubled > 0xff000000u ? 0x7e00u : nonsign));
}

float orc_fp16_to_f32(uint16_t h)
{
    uint32_t w = (uint32_t)h << 16;
    uint32_t sign = w & 0x80000000u;
    uint32_t doubled = w + w;
    uint32_t exp_offset = 0xe0u << 23;
    float normalized = f_from_bits((doubled >> 4) + exp_offset) * f_from_bits(0x07800000u);
    float denormalized = f_from_bits((doubled >> 17) | (126u << 23)) - 0.5f;
    uint32_t result = doubled < (1u << 27) ? (sign | bits_from_f(denormalized)) : (sign | bits_from_f(normalized));
    return f_from_bits(result);
}

/* ------------------------------------------------------------------ */
/* Unary family (unary.rs)                                             */
/* ------------------------------------------------------------------ */

/* Wire subop codes, unary.rs:101-146. */
enum { SUB_ABS = 0, SUB_SGN = 1, SUB_NEG = 2, SUB_STEP = 3, SUB_TANH = 4, SUB_ELU = 5, SUB_RELU = 6,
       SUB_SIGMOID = 7, SUB_GELU = 8, SUB_GELU_QUICK = 9, SUB_SILU = 10, SUB_HARDSWISH = 11,
       SUB_HARDSIGMOID = 12, SUB_EXP = 13, SUB_EXPM1 = 14, SUB_SOFTPLUS = 15, SUB_GELU_ERF = 16,
       SUB_XIELU = 17, SUB_FLOOR = 18, SUB_CEIL = 19, SUB_ROUND = 20, SUB_TRUNC = 21 };
/* Not wire codes: the reductions.rs elementwise events, routed through the
 * same loop. */
enum { MATH_LOG = 100, MATH_SIN = 101, MATH_COS = 102 };

/* SiluFormula, unary.rs:595-600: value / (1 + exp(-value)). */
float orc_silu(float x) { return x / (1.0f + expf(-x)); }

/* GeluFormula, unary.rs:522-541. */
float orc_gelu(float value)
{
    if (value <= -10.0f) return 0.0f;
    if (value >= 10.0f) return value;
    float q = orc_fp16_to_f32(orc_fp32_to_fp16(value));
    float a = 0.5f * q * (1.0f + tanhf(0.7978846f * (q + 0.044715f * q * q * q)));
    return orc_fp16_to_f32(orc_fp32_to_fp16(a));
}

/* f32::clamp(self, 0.0, 6.0): below min -> min, then above max -> max; NaN
 * passes through. */
static float clamp06(float v)
{
    if (v < 0.0f) v = 0.0f;
    if (v > 6.0f) v = 6.0f;
    return v;
}

/* GeluErfFormula, unary.rs:567-581 (Abramowitz-Stegun erf, separate
 * roundings). */
static float gelu_erf(float value)
{
    const float sign = value < 0.0f ? -1.0f : 1.0f;
    const float x = fabsf(value) / 1.41421356237309504880f; /* core::f32::consts::SQRT_2 */
    const float t = 1.0f / (1.0f + 0.3275911f * x);
    const float polynomial =
        (((((1.0614054f * t - 1.4531521f) * t) + 1.4214138f) * t - 0.28449672f) * t + 0.2548296f) * t;
    const float erf = sign * (1.0f - polynomial * expf(-x * x));
    return 0.5f * value * (1.0f + erf);
}

static float apply_unary(int subop, float x)
{
    switch (subop) { /* unary.rs:472-610 */
    case SUB_ABS: return fabsf(x);
    case SUB_SGN: return isnan(x) ? __builtin_nanf("") : copysignf(1.0f, x); /* f32::signum: +-0 -> +-1, NaN -> f32::NAN (0x7fc00000) */
    case SUB_NEG: return -x;
    case SUB_STEP: return x > 0.0f ? 1.0f : 0.0f;
    case SUB_TANH: return tanhf(x);
    case SUB_ELU: return x >= 0.0f ? x : expm1f(x);
    case SUB_RELU: return rust_maxf(x, 0.0f); /* f32::max: any NaN -> 0; the sign of max(-0, +0) is unpinned by the reference, +0 here */
    case SUB_SIGMOID: return 1.0f / (1.0f + expf(-x));
    case SUB_GELU: return orc_gelu(x);
    case SUB_GELU_QUICK: return 0.5f * x * (1.0f + tanhf(0.7978846f * x * (1.0f + 0.044715f * x * x)));
    case SUB_SILU: return orc_silu(x);
    case SUB_HARDSWISH: return x * clamp06(x + 3.0f) / 6.0f;
    case SUB_HARDSIGMOID: return clamp06(x + 3.0f) / 6.0f;
    case SUB_EXPM1: return expm1f(x);
    case SUB_SOFTPLUS: return log1pf(expf(x)); /* value.exp().ln_1p() */
    case SUB_GELU_ERF: return gelu_erf(x);
    case SUB_FLOOR: return floorf(x);
    case SUB_CEIL: return ceilf(x);
    case SUB_ROUND: return roundf(x); /* halfway away from zero */
    case SUB_TRUNC: return truncf(x);
    case MATH_LOG: return logf(x); /* reductions.rs:640-668 */
    case MATH_SIN: return sinf(x);
    case MATH_COS: return cosf(x);
    default: return expf(x);
    }
}

/* Codes with a typed event (unary.rs:72-92): every wire code but XIELU. */
static int unary_known(int subop)
{
    return subop >= SUB_ABS && subop <= SUB_TRUNC && subop != SUB_XIELU;
}

static void unary_execute(int subop, const orc_view *in, const orc_view *out)
{
    rview a = resolve(in), o = resolve(out);
    /* execute::<F>, unary.rs:674-685 (execute_dense :687-700 yields the same
     * values over a dense view of exactly count elements). */
    for (uint64_t k = 0; k < a.count; k++) wr(&o, k, apply_unary(subop, rd(&a, k)));
}

/* Dedicated events OpSilu/OpGelu/...: impl_unary_context, unary.rs:702-728. */
int orc_op_unary_event(int subop, const orc_view *in, const orc_view *out)
{
    if (!unary_known(subop)) return ORC_UNEXPECTED_EVENT;
    if (orc_layout_validate(in, 0) || orc_layout_validate(out, 0)) return ORC_INVALID_VIEW;
    if (count_or_zero(in) != count_or_zero(out)) return ORC_SHAPE_MISMATCH;
    unary_execute(subop, in, out);
    return ORC_OK;
}

/* reductions::OpLog / OpSin / OpCos (reductions.rs:45-90): guard_unary_*
 * (:508-517) -- both views valid, else InvalidView; equal counts, else
 * ShapeMismatch -- then f32::ln / sin / cos by ordinal (:640-668). */
static int math_event(int which, const orc_view *in, const orc_view *out)
{
    if (orc_layout_validate(in, 0) || orc_layout_validate(out, 0)) return ORC_INVALID_VIEW;
    if (count_or_zero(in) != count_or_zero(out)) return ORC_SHAPE_MISMATCH;
    unary_execute(which, in, out);
    return ORC_OK;
}
int orc_op_log(const orc_view *in, const orc_view *out) { return math_event(MATH_LOG, in, out); }
int orc_op_sin(const orc_view *in, const orc_view *out) { return math_event(MATH_SIN, in, out); }
int orc_op_cos(const orc_view *in, const orc_view *out) { return math_event(MATH_COS, in, out); }

/* OpUnary{subop}, unary.rs:985-1027: only eight subops are accepted and every
 * failed guard (subop, view or shape) reports UnexpectedEvent. */
int orc_op_unary(int subop, const orc_view *in, const orc_view *out)
{
    int accepted = subop == SUB_ABS || subop == SUB_NEG || subop == SUB_TANH || subop == SUB_ELU ||
                   subop == SUB_RELU || subop == SUB_GELU || subop == SUB_SILU || subop == SUB_EXP;
    if (!accepted || orc_layout_validate(in, 0) || orc_layout_validate(out, 0) ||
        count_or_zero(in) != count_or_zero(out))
        return ORC_UNEXPECTED_EVENT;
    unary_execute(subop, in, out);
    return ORC_OK;
}

/* ------------------------------------------------------------------ */
/* Scale (activation.rs:327-377)                                       */
/* ------------------------------------------------------------------ */

int orc_op_scale(const orc_view *in, const orc_view *out, float scale)
{
    if (orc_layout_validate(in, 0) || orc_layout_validate(out, 0)) return ORC_INVALID_VIEW;
    if (!same_ne(in, out)) return ORC_SHAPE_MISMATCH;
    rview a = resolve(in), o = resolve(out);
    for (uint64_t k = 0; k < a.count; k++) wr(&o, k, rd(&a, k) * scale);
    return ORC_OK;
}

/* ------------------------------------------------------------------ */
/* Normalization (normalization.rs:289-362, guards :364-386)           */
/* ------------------------------------------------------------------ */

static int norm_guard(const orc_view *in, const orc_view *out, float eps)
{
    if (!orc_normalization_view_valid(in) || !orc_normalization_view_valid(out)) return ORC_INVALID_VIEW;
    if (!same_ne(in, out)) return ORC_SHAPE_MISMATCH;
    if (!(isfinite(eps) && eps >= 0.0f)) return ORC_INVALID_PARAMETERS;
    return ORC_OK;
}

/* run_rms_norm, normalization.rs:343-362. */
int orc_op_rms_norm(const orc_view *in, const orc_view *out, float eps)
{
    int s = norm_guard(in, out, eps);
    if (s) return s;
    rview a = resolve(in), o = resolve(out);
    uint64_t cols = a.ne[0], rows = a.count / cols;
    for (uint64_t r = 0; r < rows; r++) {
        uint64_t start = r * cols, end = start + cols;
        double sum = 0.0;
        for (uint64_t k = start; k < end; k++) {
            float v = rd(&a, k);
            sum += (double)(v * v);
        }
        float mean = (float)(sum / (double)cols);
        float scale = 1.0f / sqrtf(mean + eps);
        for (uint64_t k = start; k < end; k++) wr(&o, k, rd(&a, k) * scale);
    }
    return ORC_OK;
}

/* run_norm, normalization.rs:316-341. */
int orc_op_norm(const orc_view *in, const orc_view *out, float eps)
{
    int s = norm_guard(in, out, eps);
    if (s) return s;
    rview a = resolve(in), o = resolve(out);
    uint64_t cols = a.ne[0], rows = a.count / cols;
    for (uint64_t r = 0; r < rows; r++) {
        uint64_t start = r * cols, end = start + cols;
        double sum = 0.0;
        for (uint64_t k = start; k < end; k++) sum += (double)rd(&a, k);
        float mean = (float)(sum / (double)cols);
        double var_sum = 0.0;
        for (uint64_t k = start; k < end; k++) {
            float c = rd(&a, k) - mean;
            var_sum += (double)c * (double)c;
        }
        float variance = (float)(var_sum / (double)cols);
        float scale = 1.0f / sqrtf(variance + eps);
        for (uint64_t k = start; k < end; k++) wr(&o, k, (rd(&a, k) - mean) * scale);
    }
    return ORC_OK;
}

/* ------------------------------------------------------------------ */
/* Reductions (reductions.rs:456-730)                                  */
/* ------------------------------------------------------------------ */

static int reduce_views_valid(const orc_view *src, const orc_view *dst)
{
    return orc_layout_validate(src, 0) == ORC_OK && orc_layout_validate(dst, 0) == ORC_OK;
}

/* soft_max_dense_layout, reductions.rs:488-495. */
static int soft_max_dense_layout(const orc_view *v)
{
    uint64_t st[4];
    if (v->nb[0] == 0) return effective_strides(v, st);
    if (v->dtype != DT_F32) return 0;
    u128 expected = 4;
    for (int d = 0; d < 4; d++) {
        if (v->nb[d] != expected) return 0;
        expected *= v->ne[d];
        if (expected > (u128)UINT64_MAX) return 0;
    }
    return 1;
}

/* effect_soft_max_{dense,sparse}_execute, reductions.rs:565-638. */
int orc_op_soft_max(const orc_view *src, const orc_view *dst)
{
    if (!reduce_views_valid(src, dst)) return ORC_INVALID_VIEW;
    /* soft_max_shape_valid, reductions.rs:473-484. */
    uint64_t width = src->ne[0], n = count_or_zero(src);
    if (!(width > 0 && n > 0 && n % width == 0 && n == count_or_zero(dst))) return ORC_SHAPE_MISMATCH;
    int dense = soft_max_dense_layout(src) && soft_max_dense_layout(dst);
    rview a = resolve(src), o = resolve(dst);
    uint64_t rows = n / width;
    for (uint64_t r = 0; r < rows; r++) {
        uint64_t off = r * width;
        float m = rd(&a, off);
        for (uint64_t c = 1; c < width; c++) {
            float v = rd(&a, off + c);
            if (v > m) m = v;
        }
        if (dense) {
            double sum = 0.0;
            for (uint64_t c = 0; c < width; c++) {
                float e = expf(rd(&a, off + c) - m);
                wr(&o, off + c, e);
                sum += (double)e;
            }
            float den = (float)sum;
            for (uint64_t c = 0; c < width; c++) wr(&o, off + c, rd(&o, off + c) / den);
        } else {
            float sum = 0.0f;
            for (uint64_t c = 0; c < width; c++) {
                float e = expf(rd(&a, off + c) - m);
                wr(&o, off + c, e);
                sum += e;
            }
            for (uint64_t c = 0; c < width; c++) wr(&o, off + c, rd(&o, off + c) / sum);
        }
    }
    return ORC_OK;
}

/* effect_sum_rows_execute, reductions.rs:684-700 (guard rows_output :460-463). */
int orc_op_sum_rows(const orc_view *src, const orc_view *dst)
{
    if (!reduce_views_valid(src, dst)) return ORC_INVALID_VIEW;
    if (!(dst->ne[0] == 1 && dst->ne[1] == src->ne[1] && dst->ne[2] == src->ne[2] && dst->ne[3] == src->ne[3]))
        return ORC_SHAPE_MISMATCH;
    rview a = resolve(src), o = resolve(dst);
    uint64_t width = a.ne[0], rows = a.count / width;
    for (uint64_t r = 0; r < rows; r++) {
        double sum = 0.0;
        for (uint64_t c = 0; c < width; c++) sum += (double)rd(&a, r * width + c);
        wr(&o, r, (float)sum);
    }
    return ORC_OK;
}

static int scalar_output(const orc_view *dst)
{
    return dst->ne[0] == 1 && dst->ne[1] == 1 && dst->ne[2] == 1 && dst->ne[3] == 1;
}

/* effect_sum_execute, reductions.rs:670-682. */
int orc_op_sum(const orc_view *src, const orc_view *dst)
{
    if (!reduce_views_valid(src, dst)) return ORC_INVALID_VIEW;
    if (!scalar_output(dst)) return ORC_SHAPE_MISMATCH;
    rview a = resolve(src), o = resolve(dst);
    double sum = 0.0;
    for (uint64_t k = 0; k < a.count; k++) sum += (double)rd(&a, k);
    wr(&o, 0, (float)sum);
    return ORC_OK;
}

/* effect_mean_execute, reductions.rs:702-713. */
int orc_op_mean(const orc_view *src, const orc_view *dst)
{
    if (!reduce_views_valid(src, dst)) return ORC_INVALID_VIEW;
    if (!scalar_output(dst)) return ORC_SHAPE_MISMATCH;
    rview a = resolve(src), o = resolve(dst);
    double sum = 0.0;
    for (uint64_t k = 0; k < a.count; k++) sum += (double)rd(&a, k);
    wr(&o, 0, (float)(sum / (double)a.count));
    return ORC_OK;
}

/* effect_argmax_execute, reductions.rs:715-730: start at element 0, strict >
 * (first maximum wins; NaNs never win; a NaN at element 0 yields 0), index
 * written as f32. */
static uint64_t argmax_scan(const rview *a, uint64_t base, uint64_t n)
{
    uint64_t best = 0;
    float bv = rd(a, base);
    for (uint64_t k = 1; k < n; k++) {
        float v = rd(a, base + k);
        if (v > bv) { bv = v; best = k; }
    }
    return best;
}

int orc_op_argmax(const orc_view *src, const orc_view *dst)
{
    if (!reduce_views_valid(src, dst)) return ORC_INVALID_VIEW;
    if (!scalar_output(dst)) return ORC_SHAPE_MISMATCH;
    rview a = resolve(src), o = resolve(dst);
    wr(&o, 0, (float)argmax_scan(&a, 0, a.count));
    return ORC_OK;
}

/* execute_generic_repeat, generic.rs:1641-1665, guard repeat_shape_valid
 * :964-983 (target extents are multiples of source extents). */
int orc_op_repeat(const orc_view *src, const orc_view *dst)
{
    if (orc_layout_validate(src, 0) || orc_layout_validate(dst, 0)) return ORC_INVALID_VIEW;
    for (int d = 0; d < 4; d++)
        if (dst->ne[d] % src->ne[d] != 0) return ORC_SHAPE_MISMATCH;
    rview a = resolve(src), o = resolve(dst);
    for (uint64_t k = 0; k < o.count; k++) {
        uint64_t rem = k, so = 0, sm = 1;
        for (int d = 0; d < 4; d++) {
            uint64_t c = rem % o.ne[d];
            rem /= o.ne[d];
            so += (c % a.ne[d]) * sm; /* encode_ordinal over the source extents */
            sm *= a.ne[d];
        }
        wr(&o, k, rd(&a, so));
    }
    return ORC_OK;
}

/* ------------------------------------------------------------------ */
/* Compositions                                                        */
/* ------------------------------------------------------------------ */

static orc_view dense_f32(float *data, const uint64_t ne[4])
{
    orc_view v;
    memset(&v, 0, sizeof v);
    v.data = data;
    v.dtype = DT_F32;
    memcpy(v.ne, ne, sizeof v.ne);
    v.nb[0] = 4;
    for (int d = 1; d < 4; d++) v.nb[d] = v.nb[d - 1] * ne[d - 1];
    v.data_bytes = v.nb[3] * ne[3];
    return v;
}

/* Scaled + masked soft_max: per (ne2, ne3) slice, OpScale (activation.rs:372)
 * -> equal-count OpAdd with the f16 mask decoded by fp16_to_f32
 * (quant.rs:287-300) -> OpSoftMax (reductions.rs:565-601, dense).  The mask
 * is dense f16 [ne0, ne1, m2, m3] with m2 | ne2 and m3 | ne3 (broadcast by
 * modulo, as OpRepeat would).  A null mask adds nothing. */
int orc_soft_max_ext(const orc_view *src, const orc_view *mask, float scale, const orc_view *dst)
{
    if (!reduce_views_valid(src, dst)) return ORC_INVALID_VIEW;
    if (!same_ne(src, dst)) return ORC_SHAPE_MISMATCH;
    rview a = resolve(src), o = resolve(dst);
    uint64_t ne0 = a.ne[0], ne1 = a.ne[1], plane = ne0 * ne1;
    const uint16_t *m = NULL;
    if (mask) {
        if (mask->dtype != DT_F16) return ORC_INVALID_VIEW;
        if (mask->ne[0] != ne0 || mask->ne[1] != ne1 || mask->ne[2] == 0 || mask->ne[3] == 0 ||
            a.ne[2] % mask->ne[2] || a.ne[3] % mask->ne[3])
            return ORC_SHAPE_MISMATCH;
        if (mask->nb[0] != 2 || mask->nb[1] != 2 * ne0 || mask->nb[2] != 2 * plane ||
            mask->nb[3] != 2 * plane * mask->ne[2] || mask->data_bytes < 2 * plane * mask->ne[2] * mask->ne[3])
            return ORC_INVALID_VIEW;
        m = (const uint16_t *)mask->data;
    }
    float *tmp = malloc(sizeof(float) * plane);
    float *tmp2 = malloc(sizeof(float) * plane);
    float *mf = malloc(sizeof(float) * plane);
    if (!tmp || !tmp2 || !mf) { free(tmp); free(tmp2); free(mf); return ORC_INVALID_PARAMETERS; }
    uint64_t pne[4] = {ne0, ne1, 1, 1};
    orc_view tv = dense_f32(tmp, pne), tv2 = dense_f32(tmp2, pne), mv = dense_f32(mf, pne);
    for (uint64_t i3 = 0; i3 < a.ne[3]; i3++)
        for (uint64_t i2 = 0; i2 < a.ne[2]; i2++) {
            /* slice views of src/dst at (i2, i3) */
            orc_view sv = *src, dv = *dst;
            uint64_t so = i2 * a.st[2] + i3 * a.st[3], doff = i2 * o.st[2] + i3 * o.st[3];
            sv.data = (char *)src->data + so;
            sv.data_bytes = src->data_bytes - so;
            dv.data = (char *)dst->data + doff;
            dv.data_bytes = dst->data_bytes - doff;
            /* 2-D slice views: dims 2 and 3 have extent 1, so their strides
             * take the natural row-major values (a dense head stays dense). */
            sv.nb[0] = a.st[0]; sv.nb[1] = a.st[1]; sv.nb[2] = sv.nb[3] = a.st[1] * ne1;
            dv.nb[0] = o.st[0]; dv.nb[1] = o.st[1]; dv.nb[2] = dv.nb[3] = o.st[1] * ne1;
            sv.ne[2] = sv.ne[3] = dv.ne[2] = dv.ne[3] = 1;
            orc_op_scale(&sv, &tv, scale);
            if (m) {
                const uint16_t *mp = m + ((i3 % mask->ne[3]) * mask->ne[2] + (i2 % mask->ne[2])) * plane;
                for (uint64_t k = 0; k < plane; k++) mf[k] = orc_fp16_to_f32(mp[k]);
                orc_op_binary(ORC_ADD, &tv, &mv, &tv2);
                orc_op_soft_max(&tv2, &dv);
            } else {
                orc_op_soft_max(&tv, &dv);
            }
        }
    free(tmp); free(tmp2); free(mf);
    return ORC_OK;
}

/* Per-row argmax: one OpArgmax (reductions.rs:715-730) per row view
 * ne=[ne0,1,1,1]; the f32 index is stored as i32 (exact below 2^24). */
int orc_argmax_rows(const orc_view *src, const orc_view *dst)
{
    if (orc_layout_validate(src, 0)) return ORC_INVALID_VIEW;
    if (dst->dtype != DT_I32) return ORC_INVALID_VIEW;
    rview a = resolve(src);
    uint64_t rows = a.count / a.ne[0];
    if (dst->ne[0] != 1 || dst->ne[1] != a.ne[1] || dst->ne[2] != a.ne[2] || dst->ne[3] != a.ne[3])
        return ORC_SHAPE_MISMATCH;
    if (dst->data_bytes < rows * 4) return ORC_INVALID_VIEW;
    int32_t *out = (int32_t *)dst->data;
    for (uint64_t r = 0; r < rows; r++) {
        float idx = (float)argmax_scan(&a, r * a.ne[0], a.ne[0]);
        out[r] = (int32_t)idx;
    }
    return ORC_OK;
}

/* 4-D broadcast binary: OpRepeat of src1 to dst's extents (generic.rs:
 * 1641-1665), then equal-count binary over src0 (binary.rs:411-424). */
int orc_binary_bcast(int op, const orc_view *src0, const orc_view *src1, const orc_view *dst)
{
    if (orc_layout_validate(src0, 1) || orc_layout_validate(src1, 0) || orc_layout_validate(dst, 1))
        return ORC_INVALID_VIEW;
    if (!same_ne(src0, dst)) return ORC_SHAPE_MISMATCH;
    uint64_t n = count_or_zero(dst);
    float *rep = malloc(sizeof(float) * n);
    if (!rep) return ORC_INVALID_PARAMETERS;
    orc_view rv = dense_f32(rep, dst->ne);
    int s = orc_op_repeat(src1, &rv);
    if (s == ORC_OK) s = orc_op_binary(op, src0, &rv, dst);
    free(rep);
    return s;
}

/* rms_norm then OpMulBroadcastRow by a weight row (normalization.rs:343-362,
 * broadcast.rs:372-390): two separate f32 roundings. */
int orc_rms_norm_mul(const orc_view *in, const orc_view *weight, const orc_view *out, float eps)
{
    /* Both guards are checked before anything is written, so a rejected
     * request leaves out untouched. */
    int s = norm_guard(in, out, eps);
    if (s == ORC_OK) s = broadcast_row_guard(out, weight, out);
    if (s) return s;
    orc_op_rms_norm(in, out, eps);
    return orc_op_broadcast_row(ORC_MUL, out, weight, out);
}

/* SwiGLU chain: OpSilu into a temporary, then equal-count OpMul. */
int orc_swiglu(const orc_view *gate, const orc_view *up, const orc_view *out)
{
    if (orc_layout_validate(gate, 0)) return ORC_INVALID_VIEW;
    uint64_t n = count_or_zero(gate);
    float *tmp = malloc(sizeof(float) * n);
    if (!tmp) return ORC_INVALID_PARAMETERS;
    orc_view tv = dense_f32(tmp, gate->ne);
    int s = orc_op_unary_event(SUB_SILU, gate, &tv);
    if (s == ORC_OK) s = orc_op_binary(ORC_MUL, &tv, up, out);
    free(tmp);
    return s;
}

/* ------------------------------------------------------------------ */
/* OpGlu (glu.rs:22-160, :243-282)                                     */
/* ------------------------------------------------------------------ */

/* Gate functions, glu.rs:103-129: relu = f32::max(x, 0) (rust_maxf),
 * silu = x / (1 + exp(-x)), gelu_tanh = 0.5 x (1 + tanh(0.7978846 x
 * (1 + 0.044715 x x))), gelu_quick = x (1 / (1 + exp(-1.702 x))), gelu_erf:
 * the Abramowitz-Stegun 7.1.26 polynomial with exp(-x x).  Every product
 * and sum rounds separately (no contraction). */
float orc_glu_gate(int subop, float g)
{
    switch (subop) {
    case ORC_REGLU: return rust_maxf(g, 0.0f);
    case ORC_GEGLU: return 0.5f * g * (1.0f + tanhf(0.7978846f * g * (1.0f + 0.044715f * g * g)));
    case ORC_SWIGLU: return orc_silu(g);
    case ORC_GEGLU_QUICK: return g * (1.0f / (1.0f + expf(-1.702f * g)));
    case ORC_GEGLU_ERF: {
        const float sign = g < 0.0f ? -1.0f : 1.0f;
        const float x = fabsf(g) / 1.41421356237309504880f; /* core::f32::consts::SQRT_2 */
        const float t = 1.0f / (1.0f + 0.3275911f * x);
        const float poly = (((((1.0614054f * t - 1.4531521f) * t) + 1.4214138f) * t - 0.28449672f) * t + 0.2548296f) * t;
        const float erf = sign * (1.0f - poly * expf(-x * x));
        return 0.5f * g * (1.0f + erf);
    }
    default: return 0.0f;
    }
}

/* split_len (glu.rs:85-91): input non-empty, even, output exactly half.
 * apply_split (:131-141): out[i] = values[i] * gate(gates[i]); SwiGluOai
 * (:258-270): gate and value clamped above by 7 (f32::min), then
 * silu(1.702 g) / 1.702 * (v + 1). */
int orc_op_glu(int subop, const float *input, uint64_t input_len, float *output, uint64_t output_len)
{
    if (subop < ORC_REGLU || subop > ORC_GEGLU_QUICK) return ORC_UNEXPECTED_EVENT;
    if (input_len == 0 || input_len % 2 != 0 || output_len != input_len / 2) return ORC_SHAPE_MISMATCH;
    const uint64_t n = input_len / 2;
    const float *values = input, *gates = input + n;
    for (uint64_t i = 0; i < n; i++) {
        if (subop == ORC_SWIGLU_OAI) {
            const float g = rust_minf(gates[i], 7.0f);
            const float v = rust_minf(values[i], 7.0f);
            output[i] = orc_silu(1.702f * g) / 1.702f * (v + 1.0f);
        } else {
            output[i] = values[i] * orc_glu_gate(subop, gates[i]);
        }
    }
    return ORC_OK;
}

/* ------------------------------------------------------------------ */
/* Dense-slice root events and power.rs                                */
/* ------------------------------------------------------------------ */

/* guard_dup_valid (actor.rs:2498-2501): input non-empty, lengths equal;
 * effect_dup_execute copies the slice. */
int orc_slice_dup(const float *in, uint64_t in_len, float *out, uint64_t out_len)
{
    if (in_len == 0 || in_len != out_len) return ORC_INVALID_SHAPE;
    memcpy(out, in, in_len * sizeof(float));
    return ORC_OK;
}

/* guard_{add,sub,mul,div}_valid (actor.rs:2522-2560) and the zip effects. */
int orc_slice_binary(int op, const float *lhs, uint64_t lhs_len, const float *rhs, uint64_t rhs_len, float *out,
                     uint64_t out_len)
{
    if (lhs_len == 0 || lhs_len != rhs_len || lhs_len != out_len) return ORC_INVALID_SHAPE;
    for (uint64_t i = 0; i < lhs_len; i++) out[i] = apply_binary(op, lhs[i], rhs[i]);
    return ORC_OK;
}

/* power.rs:266-273 and the v * v / sqrt(v) effects over logical ordinals. */
int orc_op_power(int sqrt_, const orc_view *in, const orc_view *out)
{
    if (orc_layout_validate(in, 0) || orc_layout_validate(out, 0)) return ORC_INVALID_VIEW;
    const uint64_t n = count_or_zero(in);
    if (n != count_or_zero(out)) return ORC_SHAPE_MISMATCH;
    rview a = resolve(in), o = resolve(out);
    for (uint64_t k = 0; k < n; k++) {
        const float v = rd(&a, k);
        wr(&o, k, sqrt_ ? sqrtf(v) : v * v);
    }
    return ORC_OK;
}

/* op_sqr / op_sqrt (actor.rs:1521-1555): slices as contiguous [len,1,1,1]
 * views (dense_power_layout :122-125), PowerError InvalidView and
 * ShapeMismatch both reported as InvalidShape (map_power_error :127-133). */
int orc_slice_power(int sqrt_, const float *in, uint64_t in_len, float *out, uint64_t out_len)
{
    const uint64_t ine[4] = {in_len, 1, 1, 1}, one[4] = {out_len, 1, 1, 1};
    orc_view iv = dense_f32((float *)in, ine), ov = dense_f32(out, one);
    const int s = orc_op_power(sqrt_, &iv, &ov);
    if (s == ORC_INVALID_VIEW || s == ORC_SHAPE_MISMATCH) return ORC_INVALID_SHAPE;
    return s;
}


/* ------------------------------------------------------------------ */
/* Typed events of activation.rs, elementwise.rs, diag.rs and          */
/* group_norm.rs                                                       */
/* ------------------------------------------------------------------ */

/* activation.rs views_valid + same_shape (:168-175). */
static int activation_guard(const orc_view *in, const orc_view *out)
{
    if (orc_layout_validate(in, 0) || orc_layout_validate(out, 0)) return ORC_INVALID_VIEW;
    if (!same_ne(in, out)) return ORC_SHAPE_MISMATCH;
    return ORC_OK;
}

/* effect_clamp_execute (activation.rs:403-421): std::clamp's comparisons. */
int orc_op_clamp(const orc_view *in, const orc_view *out, float min, float max)
{
    int s = activation_guard(in, out);
    if (s) return s;
    rview a = resolve(in), o = resolve(out);
    for (uint64_t k = 0; k < a.count; k++) {
        const float v = rd(&a, k);
        wr(&o, k, v < min ? min : (v > max ? max : v));
    }
    return ORC_OK;
}

/* effect_leaky_relu_execute (activation.rs:507-520). */
int orc_op_leaky_relu(const orc_view *in, const orc_view *out, float slope)
{
    int s = activation_guard(in, out);
    if (s) return s;
    rview a = resolve(in), o = resolve(out);
    for (uint64_t k = 0; k < a.count; k++) {
        const float v = rd(&a, k);
        wr(&o, k, v < 0.0f ? v * slope : v);
    }
    return ORC_OK;
}

/* guard_silu_back_* (activation.rs:435-465), effect (:467-480). */
int orc_op_silu_back(const orc_view *in, const orc_view *grad, const orc_view *out)
{
    if (orc_layout_validate(in, 0) || orc_layout_validate(grad, 0) || orc_layout_validate(out, 0))
        return ORC_INVALID_VIEW;
    if (!same_ne(in, grad) || !same_ne(in, out)) return ORC_SHAPE_MISMATCH;
    rview a = resolve(in), g = resolve(grad), o = resolve(out);
    for (uint64_t k = 0; k < a.count; k++) {
        const float x = rd(&a, k);
        const float sigmoid = 1.0f / (1.0f + expf(-x));
        const float derivative = sigmoid * (1.0f + x * (1.0f - sigmoid));
        wr(&o, k, rd(&g, k) * derivative);
    }
    return ORC_OK;
}

/* elementwise.rs guard_add1_* (:216-226), effect (:262-271). */
int orc_op_add1(const orc_view *src, float scalar, const orc_view *dst)
{
    if (orc_layout_validate(src, 0) || orc_layout_validate(dst, 0)) return ORC_INVALID_VIEW;
    if (!same_ne(src, dst)) return ORC_SHAPE_MISMATCH;
    rview a = resolve(src), o = resolve(dst);
    for (uint64_t k = 0; k < a.count; k++) wr(&o, k, rd(&a, k) + scalar);
    return ORC_OK;
}

/* Layout::is_dense_contiguous (tensor_view.rs:281-314). */
static int dense_contiguous(const orc_view *v)
{
    if (v->dtype != DT_F32) return 0;
    unsigned __int128 expect = 4;
    for (int d = 0; d < 4; d++) {
        if (v->nb[d] != expect) return 0;
        expect *= v->ne[d];
    }
    return 1;
}

/* OpAcc: the machine tries guard_acc_valid, _shape_invalid, _offset_invalid,
 * _view_invalid in that order (elementwise.rs:110-116, :227-243); effect
 * (:273-288). */
int orc_op_acc(const orc_view *base, const orc_view *update, const orc_view *dst, uint64_t offset)
{
    const int pair = !orc_layout_validate(base, 0) && !orc_layout_validate(dst, 0) && !orc_layout_validate(update, 0);
    const int views = pair && same_ne(base, dst) && dense_contiguous(base) && dense_contiguous(update) &&
                      dense_contiguous(dst);
    const uint64_t n = count_or_zero(dst), nu = count_or_zero(update);
    const int offset_ok = offset <= n && nu <= n - offset;
    if (views && offset_ok) {
        rview b = resolve(base), u = resolve(update), o = resolve(dst);
        for (uint64_t k = 0; k < b.count; k++) wr(&o, k, rd(&b, k));
        for (uint64_t k = 0; k < u.count; k++) wr(&o, offset + k, rd(&o, offset + k) + rd(&u, k));
        return ORC_OK;
    }
    if (pair && !same_ne(base, dst)) return ORC_SHAPE_MISMATCH;
    if (views && !offset_ok) return ORC_INVALID_OFFSET;
    return ORC_INVALID_VIEW;
}

/* diag.rs: square_side (:107-120), OpDiag::side (:57-64), apply_mask
 * (:144-160), effect_diag (:332-344).  Slices, lengths in floats. */
static int square_side(uint64_t len, uint64_t *side)
{
    if (len == 0) return 0;
    uint64_t s = 1;
    while (s * s < len) s++;
    if (s * s != len) return 0;
    *side = s;
    return 1;
}

int orc_op_diag(const float *in, uint64_t in_len, float *out, uint64_t out_len)
{
    if (in_len == 0 || (unsigned __int128)in_len * in_len != out_len) return ORC_INVALID_SHAPE;
    for (uint64_t k = 0; k < out_len; k++) out[k] = 0.0f;
    for (uint64_t i = 0; i < in_len; i++) out[i * in_len + i] = in[i];
    return ORC_OK;
}

int orc_op_diag_mask(int inf, const float *in, uint64_t in_len, float *out, uint64_t out_len, int32_t n_past)
{
    uint64_t side = 0;
    if (!(n_past >= 0 && in_len == out_len && square_side(in_len, &side))) return ORC_INVALID_SHAPE;
    const float masked = inf ? -INFINITY : 0.0f;
    for (uint64_t row = 0; row < side; row++)
        for (uint64_t col = 0; col < side; col++) {
            const uint64_t index = row * side + col;
            out[index] = col > row + (uint64_t)n_past ? masked : in[index];
        }
    return ORC_OK;
}

/* group_norm.rs: guards (:179-196), run_group_norm (:205-241). */
int orc_op_group_norm(const orc_view *in, const orc_view *out, uint64_t groups, float eps)
{
    if (!orc_normalization_view_valid(in) || !orc_normalization_view_valid(out)) return ORC_INVALID_VIEW;
    if (!same_ne(in, out)) return ORC_SHAPE_MISMATCH;
    if (!(groups != 0 && in->ne[2] != 0 && in->ne[2] % groups == 0 && isfinite(eps) && eps >= 0.0f))
        return ORC_INVALID_PARAMETERS;
    rview a = resolve(in), o = resolve(out);
    const uint64_t w = in->ne[0], h = in->ne[1], c = in->ne[2], b = in->ne[3], cpg = c / groups;
    const uint64_t count = w * h * cpg;
    for (uint64_t bt = 0; bt < b; bt++)
        for (uint64_t g = 0; g < groups; g++) {
            const uint64_t ch0 = g * cpg;
            double sum = 0.0;
            for (uint64_t ch = ch0; ch < ch0 + cpg; ch++)
                for (uint64_t r = 0; r < h; r++)
                    for (uint64_t col = 0; col < w; col++) sum += (double)rd(&a, col + w * (r + h * (ch + c * bt)));
            const float mean = (float)(sum / (double)count);
            double var = 0.0;
            for (uint64_t ch = ch0; ch < ch0 + cpg; ch++)
                for (uint64_t r = 0; r < h; r++)
                    for (uint64_t col = 0; col < w; col++) {
                        const float cen = rd(&a, col + w * (r + h * (ch + c * bt))) - mean;
                        var += (double)cen * (double)cen;
                    }
            const float scale = 1.0f / sqrtf((float)(var / (double)count) + eps);
            for (uint64_t ch = ch0; ch < ch0 + cpg; ch++)
                for (uint64_t r = 0; r < h; r++)
                    for (uint64_t col = 0; col < w; col++) {
                        const uint64_t k = col + w * (r + h * (ch + c * bt));
                        wr(&o, k, (rd(&a, k) - mean) * scale);
                    }
        }
    return ORC_OK;
}

/* OpL2Norm: guards (:252-260, :290-305), run_l2_norm (:262-268). */
int orc_op_l2_norm(const orc_view *in, const orc_view *out)
{
    if (!orc_normalization_view_valid(in) || !orc_normalization_view_valid(out)) return ORC_INVALID_VIEW;
    if (!same_ne(in, out)) return ORC_SHAPE_MISMATCH;
    rview a = resolve(in), o = resolve(out);
    float sum = 0.0f;
    for (uint64_t k = 0; k < a.count; k++) sum += rd(&a, k) * rd(&a, k);
    if (!(sum > 0.0f)) return ORC_ZERO_NORM;
    const float scale = 1.0f / sqrtf(sum);
    for (uint64_t k = 0; k < a.count; k++) wr(&o, k, rd(&a, k) * scale);
    return ORC_OK;
}
