/*
 * emel_oracle_generic.c -- CPU restatement of the generic wire envelope
 * (stateforward/emel.rs:crates/emel-kernels/src/any/generic.rs, routed by
 * sm.rs:318-426 with the guards of actor.rs:2448-2983).
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the product).  Every route is
 * restated as the reference's sequential loop, reading and writing through
 * byte offsets (coordinates_for_index / byte_offset, generic.rs:896-933),
 * with glibc expf/expm1f/tanhf/logf/sinf/cosf where Rust std calls them.
 *
 * Pinning:
 *   - the reference's known answers (tests/any/generic_envelope.rs):
 *     tests/test_oracle_generic.py::test_reference_known_answers;
 *   - guard classification (bad span, missing index_out, unknown opcode,
 *     unmaintained opcode, unrouted unary subop) against the same file;
 *   - closed forms and reductions to already-pinned ops: generic add/mul/
 *     div vs numpy IEEE f32, generic softmax vs the typed strided OpSoftMax
 *     (same f32 sum), cumsum vs numpy's sequential float32 cumsum,
 *     repeat_back(repeat(x)) == multiplicity * x, concat/diag/mask/fill/
 *     arange index formulas, mul_mat vs a float64 product within the fma
 *     chain's rounding bound, l2_norm's unit norm, count_equal's 2^24
 *     saturation, rms_norm(f64 scale) vs numpy float64: tests/test_oracle_generic.py.
 */
#include "emel_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

typedef unsigned __int128 u128;

#define DT_F32 0u
#define DT_F16 1u

enum {
    G_DUP = 0, G_ADD = 1, G_ADD1 = 3, G_SUB = 5, G_MUL = 6, G_DIV = 7, G_SQR = 8, G_SQRT = 9, G_LOG = 10,
    G_SIN = 11, G_COS = 12, G_SUM = 13, G_CUMSUM = 15, G_MEAN = 16, G_ARGMAX = 17, G_COUNT_EQUAL = 18,
    G_REPEAT = 19, G_REPEAT_BACK = 20, G_CONCAT = 21, G_SILU_BACK = 22, G_NORM = 23, G_RMS_NORM = 24,
    G_RMS_NORM_BACK = 25, G_L2_NORM = 27, G_MUL_MAT = 28, G_MUL_MAT_ARGMAX = 29, G_SCALE = 32, G_DIAG = 43,
    G_DIAG_MASK_INF = 44, G_DIAG_MASK_ZERO = 45, G_SOFT_MAX = 46, G_SOFT_MAX_BACK = 47, G_CLAMP = 50,
    G_ARANGE = 66, G_LEAKY_RELU = 70, G_FILL = 72, G_UNARY = 85, G_COUNT = 95
};

/* UnarySubOp wire codes the generic lane executes (actor.rs:2875-2905). */
enum { U_ABS = 0, U_NEG = 2, U_TANH = 4, U_ELU = 5, U_RELU = 6, U_GELU = 8, U_SILU = 10, U_EXP = 13 };

/* ---- views -------------------------------------------------------------------- */

/* Strides byte_offset uses: effective F32 strides for F32 (tensor_view.rs:
 * 262-277, None on overflow), nb as given otherwise. */
static int g_strides(const orc_view *v, uint64_t st[4])
{
    if (v->dtype != DT_F32) {
        memcpy(st, v->nb, sizeof(uint64_t) * 4);
        return 1;
    }
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

/* validate_span (generic.rs:849-894). */
static int g_span(const orc_view *v)
{
    uint64_t st[4];
    if (!g_strides(v, st)) return 0;
    u128 count = 1;
    for (int d = 0; d < 4; d++) {
        if (v->ne[d] == 0) return 0;
        count *= v->ne[d];
        if (count > (u128)UINT64_MAX) return 0;
        if (v->ne[d] > 1 && st[d] == 0) return 0;
    }
    u128 max_offset = 0;
    for (int d = 0; d < 4; d++) {
        u128 c = (u128)(v->ne[d] - 1) * st[d];
        if (max_offset > ~(u128)0 - c) return 0;
        max_offset += c;
    }
    return max_offset + 1 <= (u128)v->data_bytes;
}

/* f32_valid (generic.rs:471-476). */
static int g_f32(const orc_view *v)
{
    uint64_t st[4];
    if (!v || v->dtype != DT_F32 || !g_strides(v, st) || !g_span(v)) return 0;
    for (int d = 0; d < 4; d++)
        if (st[d] < 4) return 0;
    return 1;
}

/* f16_valid (generic.rs:489-493), dense contiguous F16 (tensor_view.rs:293-314). */
static int g_f16(const orc_view *v)
{
    if (!v || v->dtype != DT_F16 || !g_span(v)) return 0;
    u128 expect = 2;
    for (int d = 0; d < 4; d++) {
        if (v->nb[d] != expect) return 0;
        expect *= v->ne[d];
        if (expect > (u128)UINT64_MAX) return 0;
    }
    return 1;
}

static uint64_t g_count(const orc_view *v)
{
    uint64_t c = 1;
    for (int d = 0; d < 4; d++) c *= v->ne[d];
    return c;
}

static int g_same_ne(const orc_view *a, const orc_view *b)
{
    return memcmp(a->ne, b->ne, sizeof a->ne) == 0;
}

static int g_ne_is(const orc_view *v, uint64_t a, uint64_t b, uint64_t c, uint64_t e)
{
    return v->ne[0] == a && v->ne[1] == b && v->ne[2] == c && v->ne[3] == e;
}

static uint64_t g_off(const orc_view *v, uint64_t ordinal)
{
    uint64_t st[4], off = 0;
    g_strides(v, st);
    for (int d = 0; d < 4; d++) {
        off += (ordinal % v->ne[d]) * st[d];
        ordinal /= v->ne[d];
    }
    return off;
}

/* read_f32_index / write_f32_index (generic.rs:478-486, :556-566); the
 * caller has checked that every element lies inside data_bytes. */
static float g_rd(const orc_view *v, uint64_t ordinal)
{
    float x;
    memcpy(&x, (const unsigned char *)v->data + g_off(v, ordinal), 4);
    return x;
}

static void g_wr(const orc_view *v, uint64_t ordinal, float x)
{
    memcpy((unsigned char *)v->data + g_off(v, ordinal), &x, 4);
}

static uint16_t g_rd16(const orc_view *v, uint64_t ordinal)
{
    uint16_t h;
    memcpy(&h, (const unsigned char *)v->data + g_off(v, ordinal), 2);
    return h;
}

/* The whole last element inside data_bytes: where it is not, the
 * reference's guard passes (it checks one byte) and its read or write of
 * four bytes panics. */
static int g_whole(const orc_view *v)
{
    uint64_t st[4];
    if (!g_strides(v, st)) return 0;
    u128 max_offset = 0;
    for (int d = 0; d < 4; d++) max_offset += (u128)(v->ne[d] - 1) * st[d];
    return max_offset + (v->dtype == DT_F16 ? 2 : 4) <= (u128)v->data_bytes;
}

/* parameter_f32 / parameter_i32 (generic.rs:935-945). */
static int g_param(const orc_generic_request *r, int slot, void *out)
{
    if (r->op_params_size < 4u * (uint32_t)(slot + 1)) return 0;
    memcpy(out, r->op_params + 4 * slot, 4);
    return 1;
}

/* ---- predicates (generic.rs:947-1262) ---------------------------------------------- */

static int p_pair(const orc_generic_request *r)
{
    return g_f32(r->src0) && g_f32(r->dst) && g_count(r->src0) == g_count(r->dst);
}

static int p_triplet(const orc_generic_request *r)
{
    return g_f32(r->src0) && g_f32(r->src1) && g_f32(r->dst) && g_same_ne(r->src0, r->src1) &&
           g_same_ne(r->src0, r->dst);
}

static int p_scalar(const orc_generic_request *r)
{
    float s;
    return p_pair(r) && g_param(r, 0, &s) && isfinite(s);
}

static int p_clamp(const orc_generic_request *r)
{
    float lo, hi;
    if (!p_pair(r) || !g_param(r, 0, &lo) || !g_param(r, 1, &hi)) return 0;
    return isfinite(lo) && isfinite(hi) && lo <= hi;
}

static int p_cumsum(const orc_generic_request *r)
{
    return g_f32(r->src0) && g_f32(r->dst) && g_same_ne(r->src0, r->dst);
}

static int p_repeat_shape(const orc_view *src, const orc_view *dst)
{
    for (int d = 0; d < 4; d++)
        if (src->ne[d] == 0 || dst->ne[d] == 0 || dst->ne[d] % src->ne[d] != 0) return 0;
    return 1;
}

static int p_repeat(const orc_generic_request *r)
{
    return g_f32(r->src0) && g_f32(r->dst) && p_repeat_shape(r->src0, r->dst);
}

static int p_repeat_back(const orc_generic_request *r)
{
    return g_f32(r->src0) && g_f32(r->dst) && p_repeat_shape(r->dst, r->src0);
}

static int p_concat(const orc_generic_request *r, int axis)
{
    int32_t p;
    if (!g_f32(r->src0) || !g_f32(r->src1) || !g_f32(r->dst) || !g_param(r, 0, &p) || p != axis) return 0;
    for (int d = 0; d < 4; d++) {
        if (d == axis) {
            if ((u128)r->src0->ne[d] + r->src1->ne[d] != (u128)r->dst->ne[d]) return 0;
        } else if (r->src0->ne[d] != r->src1->ne[d] || r->src0->ne[d] != r->dst->ne[d]) {
            return 0;
        }
    }
    return 1;
}

static int p_fill(const orc_generic_request *r)
{
    float v;
    return !r->src0 && g_f32(r->dst) && g_param(r, 0, &v) && isfinite(v);
}

static int p_arange(const orc_generic_request *r)
{
    float a, b;
    return !r->src0 && g_f32(r->dst) && g_param(r, 0, &a) && isfinite(a) && g_param(r, 1, &b) && isfinite(b);
}

static int p_diag(const orc_generic_request *r)
{
    if (!r->src0 || !r->dst) return 0;
    const uint64_t n = r->src0->ne[0];
    const u128 side = (u128)n * n;
    if (side > (u128)UINT64_MAX) return 0;
    return g_f32(r->src0) && g_f32(r->dst) && r->src0->ne[1] == 1 && r->src0->ne[2] == 1 && r->src0->ne[3] == 1 &&
           g_ne_is(r->dst, n, n, 1, 1) && g_count(r->dst) == (uint64_t)side;
}

static int p_mask(const orc_generic_request *r)
{
    int32_t n_past;
    if (!r->src0 || !r->dst || !g_param(r, 0, &n_past)) return 0;
    const uint64_t *s = r->src0->ne;
    return n_past >= 0 && g_f32(r->src0) && g_f32(r->dst) && g_same_ne(r->src0, r->dst) && s[0] > 0 && s[1] == s[0] &&
           s[2] == 1 && s[3] == 1;
}

static int p_l2(const orc_generic_request *r)
{
    return g_f32(r->src0) && g_f32(r->dst) && g_same_ne(r->src0, r->dst) && g_count(r->src0) > 0;
}

static int p_softmax_back(const orc_generic_request *r)
{
    int32_t row;
    if (!p_triplet(r) || !g_param(r, 0, &row)) return 0;
    return row > 0 && g_count(r->src0) % (uint64_t)row == 0;
}

static int p_rms_norm_back(const orc_generic_request *r)
{
    float eps;
    if (!p_triplet(r) || !g_param(r, 0, &eps)) return 0;
    return isfinite(eps) && eps >= 0.0f && r->src0->ne[0] > 0;
}

static int p_count_equal(const orc_generic_request *r)
{
    return g_f32(r->src0) && g_f32(r->src1) && g_f32(r->dst) && g_count(r->src0) == g_count(r->src1) &&
           g_count(r->dst) == 1;
}

static int p_binary(const orc_generic_request *r)
{
    return g_f32(r->src0) && g_f32(r->src1) && g_f32(r->dst) && g_count(r->src0) == g_count(r->src1) &&
           g_count(r->src0) == g_count(r->dst);
}

static int p_reduce(const orc_generic_request *r)
{
    return g_f32(r->src0) && g_f32(r->dst) && g_count(r->dst) == 1;
}

static int p_norm(const orc_generic_request *r)
{
    float eps;
    return g_f32(r->src0) && g_f32(r->dst) && g_same_ne(r->src0, r->dst) && g_param(r, 0, &eps) && isfinite(eps) &&
           eps >= 0.0f;
}

static int p_matmul(const orc_generic_request *r)
{
    if (!g_f32(r->src0) || !g_f32(r->src1) || !g_f32(r->dst)) return 0;
    const uint64_t *l = r->src0->ne, *m = r->src1->ne, *o = r->dst->ne;
    return l[0] > 0 && l[1] > 0 && m[0] > 0 && m[1] == l[0] && o[0] == m[0] && o[1] == l[1] && l[2] == 1 &&
           l[3] == 1 && m[2] == 1 && m[3] == 1 && o[2] == 1 && o[3] == 1;
}

static int p_matmul_argmax(const orc_generic_request *r)
{
    if (!r->index_out || !g_f32(r->src0) || !g_f32(r->src1) || !g_f32(r->dst)) return 0;
    const uint64_t *l = r->src0->ne;
    return l[0] > 0 && l[1] > 0 && g_ne_is(r->src1, l[0], 1, 1, 1) && g_ne_is(r->dst, 1, 1, 1, 1) && l[2] == 1 &&
           l[3] == 1;
}

static int p_matmul_f16(const orc_generic_request *r)
{
    if (!g_f16(r->src0) || !g_f16(r->src1) || !g_f32(r->dst)) return 0;
    const uint64_t *l = r->src0->ne, *m = r->src1->ne, *o = r->dst->ne;
    return l[0] > 0 && l[1] > 0 && m[0] == l[0] && m[1] > 0 && o[0] == l[1] && o[1] == m[1] && l[2] == 1 &&
           l[3] == 1 && m[2] == 1 && m[3] == 1 && o[2] == 1 && o[3] == 1;
}

static int unary_routed(uint32_t s)
{
    return s == U_ABS || s == U_NEG || s == U_TANH || s == U_ELU || s == U_RELU || s == U_GELU || s == U_SILU ||
           s == U_EXP;
}

/* ---- executors (generic.rs:1264-2055) ---------------------------------------------- */

static float g_param_f32(const orc_generic_request *r, int slot)
{
    float v = 0.0f;
    g_param(r, slot, &v);
    return v;
}

static int32_t g_param_i32(const orc_generic_request *r, int slot)
{
    int32_t v = 0;
    g_param(r, slot, &v);
    return v;
}

static void x_copy(const orc_generic_request *r)
{
    const uint64_t n = g_count(r->src0);
    for (uint64_t i = 0; i < n; i++) g_wr(r->dst, i, g_rd(r->src0, i));
}

static void x_binary(const orc_generic_request *r)
{
    const uint64_t n = g_count(r->src0);
    for (uint64_t i = 0; i < n; i++) {
        const float a = g_rd(r->src0, i), b = g_rd(r->src1, i);
        float v;
        switch (r->operation) {
        case G_ADD: v = a + b; break;
        case G_SUB: v = a - b; break;
        case G_MUL: v = a * b; break;
        default: v = a / b; break;
        }
        g_wr(r->dst, i, v);
    }
}

/* execute_generic_unary (generic.rs:1307-1350); code is the local selector. */
static float unary_value(int code, float v)
{
    switch (code) {
    case U_ABS: return fabsf(v);
    case U_NEG: return -v;
    case U_TANH: return tanhf(v);
    case U_ELU: return v > 0.0f ? v : expm1f(v);
    case U_RELU: return rust_maxf(v, 0.0f); /* f32::max, as the typed OpUnary */
    case U_GELU: return 0.5f * v * (1.0f + tanhf(0.7978846f * fmaf(0.044715f * v * v, v, v)));
    case U_SILU: return v / (1.0f + expf(-v));
    case U_EXP: return expf(v);
    case 100 + G_SQR: return v * v;
    case 100 + G_SQRT: return sqrtf(v);
    case 100 + G_LOG: return logf(v);
    case 100 + G_SIN: return sinf(v);
    default: return cosf(v);
    }
}

static void x_unary(const orc_generic_request *r, int code)
{
    const uint64_t n = g_count(r->src0);
    for (uint64_t i = 0; i < n; i++) g_wr(r->dst, i, unary_value(code, g_rd(r->src0, i)));
}

static void x_scalar(const orc_generic_request *r)
{
    const float s = g_param_f32(r, 0);
    const uint64_t n = g_count(r->src0);
    for (uint64_t i = 0; i < n; i++) {
        const float v = g_rd(r->src0, i);
        float o;
        if (r->operation == G_ADD1) o = v + s;
        else if (r->operation == G_SCALE) o = v * s;
        else o = v < 0.0f ? v * s : v;
        g_wr(r->dst, i, o);
    }
}

static void x_clamp(const orc_generic_request *r)
{
    const float lo = g_param_f32(r, 0), hi = g_param_f32(r, 1);
    const uint64_t n = g_count(r->src0);
    for (uint64_t i = 0; i < n; i++) {
        float v = g_rd(r->src0, i); /* f32::clamp */
        if (v < lo) v = lo;
        if (v > hi) v = hi;
        g_wr(r->dst, i, v);
    }
}

static void x_silu_back(const orc_generic_request *r)
{
    const uint64_t n = g_count(r->src0);
    for (uint64_t i = 0; i < n; i++) {
        const float x = g_rd(r->src0, i);
        const float sg = 1.0f / (1.0f + expf(-x));
        const float deriv = sg * (1.0f + x * (1.0f - sg));
        g_wr(r->dst, i, g_rd(r->src1, i) * deriv);
    }
}

static void x_reduce(const orc_generic_request *r)
{
    const uint64_t n = g_count(r->src0);
    if (r->operation == G_ARGMAX) {
        uint64_t best_i = 0;
        float best = g_rd(r->src0, 0);
        for (uint64_t i = 1; i < n; i++) {
            const float v = g_rd(r->src0, i);
            if (v > best) {
                best = v;
                best_i = i;
            }
        }
        g_wr(r->dst, 0, (float)best_i);
        return;
    }
    double sum = 0.0;
    for (uint64_t i = 0; i < n; i++) sum += (double)g_rd(r->src0, i);
    g_wr(r->dst, 0, r->operation == G_SUM ? (float)sum : (float)(sum / (double)n));
}

static void x_cumsum(const orc_generic_request *r)
{
    const uint64_t w = r->src0->ne[0], rows = g_count(r->src0) / w;
    for (uint64_t row = 0; row < rows; row++) {
        float sum = 0.0f;
        for (uint64_t c = 0; c < w; c++) {
            sum += g_rd(r->src0, row * w + c);
            g_wr(r->dst, row * w + c, sum);
        }
    }
}

static void decode(uint64_t ordinal, const uint64_t ne[4], uint64_t c[4])
{
    for (int d = 0; d < 4; d++) {
        c[d] = ordinal % ne[d];
        ordinal /= ne[d];
    }
}

static uint64_t encode(const uint64_t c[4], const uint64_t ne[4])
{
    uint64_t o = 0, s = 1;
    for (int d = 0; d < 4; d++) {
        o += c[d] * s;
        s *= ne[d];
    }
    return o;
}

static void x_repeat(const orc_generic_request *r)
{
    const uint64_t n = g_count(r->dst);
    for (uint64_t k = 0; k < n; k++) {
        uint64_t c[4];
        decode(k, r->dst->ne, c);
        for (int d = 0; d < 4; d++) c[d] %= r->src0->ne[d];
        g_wr(r->dst, k, g_rd(r->src0, encode(c, r->src0->ne)));
    }
}

static void x_repeat_back(const orc_generic_request *r)
{
    const uint64_t nt = g_count(r->dst), ns = g_count(r->src0);
    for (uint64_t k = 0; k < nt; k++) g_wr(r->dst, k, 0.0f);
    for (uint64_t k = 0; k < ns; k++) {
        uint64_t c[4];
        decode(k, r->src0->ne, c);
        for (int d = 0; d < 4; d++) c[d] %= r->dst->ne[d];
        const uint64_t t = encode(c, r->dst->ne);
        g_wr(r->dst, t, g_rd(r->dst, t) + g_rd(r->src0, k));
    }
}

static void x_concat(const orc_generic_request *r, int axis)
{
    const uint64_t nl = g_count(r->src0), nr = g_count(r->src1);
    for (uint64_t k = 0; k < nl; k++) {
        uint64_t c[4];
        decode(k, r->src0->ne, c);
        g_wr(r->dst, encode(c, r->dst->ne), g_rd(r->src0, k));
    }
    for (uint64_t k = 0; k < nr; k++) {
        uint64_t c[4];
        decode(k, r->src1->ne, c);
        c[axis] += r->src0->ne[axis];
        g_wr(r->dst, encode(c, r->dst->ne), g_rd(r->src1, k));
    }
}

static void x_fill(const orc_generic_request *r)
{
    const float v = g_param_f32(r, 0);
    const uint64_t n = g_count(r->dst);
    for (uint64_t k = 0; k < n; k++) g_wr(r->dst, k, v);
}

static void x_arange(const orc_generic_request *r)
{
    const float start = g_param_f32(r, 0), step = g_param_f32(r, 1);
    const uint64_t n = g_count(r->dst);
    for (uint64_t k = 0; k < n; k++) g_wr(r->dst, k, fmaf((float)k, step, start));
}

static void x_diag(const orc_generic_request *r)
{
    const uint64_t side = r->src0->ne[0];
    for (uint64_t row = 0; row < side; row++)
        for (uint64_t col = 0; col < side; col++)
            g_wr(r->dst, row * side + col, row == col ? g_rd(r->src0, row) : 0.0f);
}

static void x_diag_mask(const orc_generic_request *r)
{
    const uint64_t side = r->src0->ne[0], n_past = (uint64_t)g_param_i32(r, 0);
    for (uint64_t row = 0; row < side; row++)
        for (uint64_t col = 0; col < side; col++) {
            const uint64_t i = row * side + col;
            float v;
            if (col > row + n_past) v = r->operation == G_DIAG_MASK_INF ? -INFINITY : 0.0f;
            else v = g_rd(r->src0, i);
            g_wr(r->dst, i, v);
        }
}

static void x_l2(const orc_generic_request *r)
{
    const uint64_t n = g_count(r->src0);
    float sum = 0.0f;
    for (uint64_t i = 0; i < n; i++) {
        const float v = g_rd(r->src0, i);
        sum += v * v;
    }
    const float scale = 1.0f / sqrtf(sum);
    for (uint64_t i = 0; i < n; i++) g_wr(r->dst, i, g_rd(r->src0, i) * scale);
}

static void x_softmax_back(const orc_generic_request *r)
{
    const uint64_t w = (uint64_t)g_param_i32(r, 0), rows = g_count(r->src0) / w;
    for (uint64_t row = 0; row < rows; row++) {
        const uint64_t s = row * w;
        float dot = 0.0f;
        for (uint64_t c = 0; c < w; c++) dot = fmaf(g_rd(r->src0, s + c), g_rd(r->src1, s + c), dot);
        for (uint64_t c = 0; c < w; c++)
            g_wr(r->dst, s + c, g_rd(r->src0, s + c) * (g_rd(r->src1, s + c) - dot));
    }
}

static void x_rms_norm_back(const orc_generic_request *r)
{
    const float eps = g_param_f32(r, 0);
    const uint64_t w = r->src0->ne[0], rows = g_count(r->src0) / w;
    const double wd = (double)w;
    for (uint64_t row = 0; row < rows; row++) {
        const uint64_t s = row * w;
        double sum = 0.0;
        for (uint64_t c = 0; c < w; c++) {
            const float v = g_rd(r->src0, s + c);
            sum += (double)(v * v);
        }
        const double inv = 1.0 / sqrt(sum / wd + (double)eps);
        double dot = 0.0;
        for (uint64_t c = 0; c < w; c++) dot += (double)(g_rd(r->src1, s + c) * g_rd(r->src0, s + c));
        for (uint64_t c = 0; c < w; c++) {
            const double x = (double)g_rd(r->src0, s + c), dy = (double)g_rd(r->src1, s + c);
            g_wr(r->dst, s + c, (float)(dy * inv - x * inv * inv * inv * dot / wd));
        }
    }
}

static void x_count_equal(const orc_generic_request *r)
{
    const uint64_t n = g_count(r->src0);
    float equal = 0.0f;
    for (uint64_t i = 0; i < n; i++) {
        const float a = g_rd(r->src0, i), b = g_rd(r->src1, i);
        uint32_t ua, ub;
        memcpy(&ua, &a, 4);
        memcpy(&ub, &b, 4);
        if (ua == ub) equal += 1.0f;
    }
    g_wr(r->dst, 0, equal);
}

static void x_softmax(const orc_generic_request *r)
{
    const uint64_t w = r->src0->ne[0], rows = g_count(r->src0) / w;
    for (uint64_t row = 0; row < rows; row++) {
        float mx = -INFINITY;
        for (uint64_t c = 0; c < w; c++) mx = rust_maxf(mx, g_rd(r->src0, row * w + c)); /* generic.rs:1970 */
        float sum = 0.0f;
        for (uint64_t c = 0; c < w; c++) {
            const float e = expf(g_rd(r->src0, row * w + c) - mx);
            g_wr(r->dst, row * w + c, e);
            sum += e;
        }
        for (uint64_t c = 0; c < w; c++) g_wr(r->dst, row * w + c, g_rd(r->dst, row * w + c) / sum);
    }
}

static void x_norm(const orc_generic_request *r, int rms)
{
    const float eps = g_param_f32(r, 0);
    const uint64_t w = r->src0->ne[0], rows = g_count(r->src0) / w;
    for (uint64_t row = 0; row < rows; row++) {
        double sum = 0.0;
        for (uint64_t c = 0; c < w; c++) {
            const float v = g_rd(r->src0, row * w + c);
            sum += rms ? (double)(v * v) : (double)v;
        }
        const float mean = (float)(sum / (double)w);
        double var = 0.0;
        if (!rms) {
            for (uint64_t c = 0; c < w; c++) {
                const float centered = g_rd(r->src0, row * w + c) - mean;
                var += (double)(centered * centered);
            }
            var /= (double)w;
        }
        const float scale = (float)(1.0 / sqrt((rms ? (double)mean : var) + (double)eps));
        for (uint64_t c = 0; c < w; c++) {
            const float v = g_rd(r->src0, row * w + c);
            g_wr(r->dst, row * w + c, rms ? v * scale : (v - mean) * scale);
        }
    }
}

static void x_matmul(const orc_generic_request *r)
{
    const uint64_t k = r->src0->ne[0], m = r->src0->ne[1], n = r->src1->ne[0];
    for (uint64_t row = 0; row < m; row++)
        for (uint64_t col = 0; col < n; col++) {
            float v = 0.0f;
            for (uint64_t i = 0; i < k; i++) v = fmaf(g_rd(r->src0, row * k + i), g_rd(r->src1, i * n + col), v);
            g_wr(r->dst, row * n + col, v);
        }
}

static void x_matmul_argmax(const orc_generic_request *r)
{
    const uint64_t k = r->src0->ne[0], rows = r->src0->ne[1];
    uint64_t best_i = 0;
    float best = -INFINITY;
    for (uint64_t row = 0; row < rows; row++) {
        float v = 0.0f;
        for (uint64_t i = 0; i < k; i++) v = fmaf(g_rd(r->src0, row * k + i), g_rd(r->src1, i), v);
        if (row == 0 || v > best) {
            best = v;
            best_i = row;
        }
    }
    g_wr(r->dst, 0, best);
    *r->index_out = (int32_t)best_i;
}

static void x_matmul_f16(const orc_generic_request *r)
{
    const uint64_t k = r->src0->ne[0], m = r->src0->ne[1], n = r->src1->ne[1];
    for (uint64_t col = 0; col < n; col++)
        for (uint64_t row = 0; row < m; row++) {
            double sum = 0.0;
            for (uint64_t i = 0; i < k; i++) {
                const float a = orc_fp16_to_f32(g_rd16(r->src0, row * k + i));
                const float b = orc_fp16_to_f32(g_rd16(r->src1, col * k + i));
                sum += (double)(a * b);
            }
            g_wr(r->dst, row + col * m, (float)sum);
        }
}

/* ---- dispatch (sm.rs:318-426) ------------------------------------------------------ */

enum {
    R_NONE = 0, R_DUP, R_BINARY, R_SCALAR, R_CLAMP, R_SILU_BACK, R_CUMSUM, R_REPEAT, R_REPEAT_BACK, R_CONCAT,
    R_DIAG, R_MASK, R_SOFTMAX_BACK, R_RMS_NORM_BACK, R_L2, R_COUNT_EQUAL, R_FILL, R_ARANGE, R_MATMUL,
    R_MATMUL_F16, R_MATMUL_ARGMAX, R_UNARY_OP, R_REDUCE, R_SOFTMAX, R_NORM, R_UNARY
};

static int route(const orc_generic_request *r, int *axis)
{
    switch (r->operation) {
    case G_DUP: return p_pair(r) ? R_DUP : R_NONE;
    case G_ADD: case G_SUB: case G_MUL: case G_DIV: return p_binary(r) ? R_BINARY : R_NONE;
    case G_ADD1: case G_SCALE: case G_LEAKY_RELU: return p_scalar(r) ? R_SCALAR : R_NONE;
    case G_CLAMP: return p_clamp(r) ? R_CLAMP : R_NONE;
    case G_SILU_BACK: return p_triplet(r) ? R_SILU_BACK : R_NONE;
    case G_CUMSUM: return p_cumsum(r) ? R_CUMSUM : R_NONE;
    case G_REPEAT: return p_repeat(r) ? R_REPEAT : R_NONE;
    case G_REPEAT_BACK: return p_repeat_back(r) ? R_REPEAT_BACK : R_NONE;
    case G_CONCAT:
        for (int a = 0; a < 4; a++)
            if (p_concat(r, a)) {
                *axis = a;
                return R_CONCAT;
            }
        return R_NONE;
    case G_DIAG: return p_diag(r) ? R_DIAG : R_NONE;
    case G_DIAG_MASK_INF: case G_DIAG_MASK_ZERO: return p_mask(r) ? R_MASK : R_NONE;
    case G_SOFT_MAX_BACK: return p_softmax_back(r) ? R_SOFTMAX_BACK : R_NONE;
    case G_RMS_NORM_BACK: return p_rms_norm_back(r) ? R_RMS_NORM_BACK : R_NONE;
    case G_L2_NORM: return p_l2(r) ? R_L2 : R_NONE;
    case G_COUNT_EQUAL: return p_count_equal(r) ? R_COUNT_EQUAL : R_NONE;
    case G_FILL: return p_fill(r) ? R_FILL : R_NONE;
    case G_ARANGE: return p_arange(r) ? R_ARANGE : R_NONE;
    case G_MUL_MAT:
        if (p_matmul(r)) return R_MATMUL;
        return p_matmul_f16(r) ? R_MATMUL_F16 : R_NONE;
    case G_MUL_MAT_ARGMAX: return p_matmul_argmax(r) ? R_MATMUL_ARGMAX : R_NONE;
    case G_SQR: case G_SQRT: case G_LOG: case G_SIN: case G_COS: return p_pair(r) ? R_UNARY_OP : R_NONE;
    case G_SUM: case G_MEAN: case G_ARGMAX: return p_reduce(r) ? R_REDUCE : R_NONE;
    case G_SOFT_MAX: return p_pair(r) ? R_SOFTMAX : R_NONE;
    case G_NORM: case G_RMS_NORM: return p_norm(r) ? R_NORM : R_NONE;
    case G_UNARY: return unary_routed(r->unary_subop) && p_pair(r) ? R_UNARY : R_NONE;
    default: return R_NONE;
    }
}

static int maintained(uint32_t op)
{
    switch (op) {
    case G_DUP: case G_ADD: case G_SUB: case G_MUL: case G_DIV: case G_ADD1: case G_SCALE: case G_LEAKY_RELU:
    case G_CLAMP: case G_SILU_BACK: case G_CUMSUM: case G_REPEAT: case G_REPEAT_BACK: case G_CONCAT: case G_DIAG:
    case G_DIAG_MASK_INF: case G_DIAG_MASK_ZERO: case G_SOFT_MAX_BACK: case G_RMS_NORM_BACK: case G_L2_NORM:
    case G_COUNT_EQUAL: case G_FILL: case G_ARANGE: case G_MUL_MAT: case G_MUL_MAT_ARGMAX: case G_SQR: case G_SQRT:
    case G_LOG: case G_SIN: case G_COS: case G_SUM: case G_MEAN: case G_ARGMAX: case G_SOFT_MAX: case G_NORM:
    case G_RMS_NORM: case G_UNARY:
        return 1;
    default:
        return 0;
    }
}

/* GenericRequest::validate (generic.rs:769-789). */
static int request_valid(const orc_generic_request *r)
{
    const orc_view *vs[4] = {r->src0, r->src1, r->src2, r->dst};
    for (int i = 0; i < 4; i++)
        if (vs[i] && !g_span(vs[i])) return 0;
    return !(r->operation == G_MUL_MAT_ARGMAX && !r->index_out);
}

int orc_generic(const orc_generic_request *r)
{
    if (r->operation >= G_COUNT || r->op_params_size > 64) return ORC_INVALID_ARGUMENT;
    int axis = 0;
    const int rt = route(r, &axis);
    if (rt == R_NONE) {
        const int valid = request_valid(r);
        if (valid && maintained(r->operation)) return ORC_INVALID_SHAPE;
        return valid ? ORC_UNSUPPORTED_OPERATION : ORC_INVALID_SHAPE;
    }
    /* The views the route reads and writes; a partial last element would
     * panic the reference mid-loop. */
    const orc_view *used[3] = {r->dst, NULL, NULL};
    if (rt != R_FILL && rt != R_ARANGE) used[1] = r->src0;
    if (rt == R_BINARY || rt == R_SILU_BACK || rt == R_CONCAT || rt == R_SOFTMAX_BACK || rt == R_RMS_NORM_BACK ||
        rt == R_COUNT_EQUAL || rt == R_MATMUL || rt == R_MATMUL_F16 || rt == R_MATMUL_ARGMAX)
        used[2] = r->src1;
    for (int i = 0; i < 3; i++)
        if (used[i] && !g_whole(used[i])) return ORC_PANIC;
    switch (rt) {
    case R_DUP: x_copy(r); break;
    case R_BINARY: x_binary(r); break;
    case R_SCALAR: x_scalar(r); break;
    case R_CLAMP: x_clamp(r); break;
    case R_SILU_BACK: x_silu_back(r); break;
    case R_CUMSUM: x_cumsum(r); break;
    case R_REPEAT: x_repeat(r); break;
    case R_REPEAT_BACK: x_repeat_back(r); break;
    case R_CONCAT: x_concat(r, axis); break;
    case R_DIAG: x_diag(r); break;
    case R_MASK: x_diag_mask(r); break;
    case R_SOFTMAX_BACK: x_softmax_back(r); break;
    case R_RMS_NORM_BACK: x_rms_norm_back(r); break;
    case R_L2: x_l2(r); break;
    case R_COUNT_EQUAL: x_count_equal(r); break;
    case R_FILL: x_fill(r); break;
    case R_ARANGE: x_arange(r); break;
    case R_MATMUL: x_matmul(r); break;
    case R_MATMUL_F16: x_matmul_f16(r); break;
    case R_MATMUL_ARGMAX: x_matmul_argmax(r); break;
    case R_UNARY_OP: x_unary(r, 100 + (int)r->operation); break;
    case R_REDUCE: x_reduce(r); break;
    case R_SOFTMAX: x_softmax(r); break;
    case R_NORM: x_norm(r, r->operation == G_RMS_NORM); break;
    case R_UNARY: x_unary(r, (int)r->unary_subop); break;
    default: return ORC_INVALID_SHAPE;
    }
    return ORC_OK;
}
