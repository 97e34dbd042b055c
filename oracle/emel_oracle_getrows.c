/*
 * emel_oracle_getrows.c -- CPU restatement of the row gather
 * (stateforward/emel.rs:crates/emel-kernels/src/any/get_rows.rs).
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the product).  Restates the
 * IndexView contract (:42-216), each event's guards in the transition order
 * of the machine (:664-719, predicates :855-1262) and the actions' i2 / i1 /
 * i0 loops (:1453-2003) with the block decoders of quant.rs:106-205 and
 * quant_more.rs:438-468, 952-961.
 *
 * Pinning: tests/test_oracle_getrows.py checks every fixture of
 * snapshots/parity/kernel-get-rows/manifest.txt and the known answers of
 * tests/any/get_rows_ops.rs (row/batch order, strided and implicit indices,
 * Q4_0/Q8_0/Q4_K rows incl. the upper scale/min groups, rejections), plus
 * closed forms (numpy fancy indexing, f16/bf16 widening, block decoders
 * against independent numpy formulas).
 */
#include "emel_oracle.h"

#include <math.h>
#include <string.h>

typedef unsigned __int128 u128;

#define DT_F32 0u
#define DT_F16 1u
#define DT_BF16 30u

/* ---- IndexView (get_rows.rs:54-196) ----------------------------------------------- */

typedef struct {
    const orc_index_view *v;
    uint64_t bstride[3]; /* byte strides used */
    uint64_t count;
    int shape_valid, strides_valid, span_valid;
} ix_t;

static int contiguous_byte_strides(const uint64_t ne[3], uint64_t out[3])
{
    int ok = 1;
    out[0] = 4;
    for (int d = 1; d < 3; d++) {
        u128 s = (u128)out[d - 1] * ne[d - 1];
        if (s > (u128)UINT64_MAX) {
            ok = 0;
            out[d] = 0;
        } else {
            out[d] = (uint64_t)s;
        }
    }
    return ok;
}

static ix_t ix_make(const orc_index_view *v)
{
    ix_t x;
    x.v = v;
    int inferred_valid, allow_implicit;
    if (!v->explicit_strides) { /* IndexView::new */
        inferred_valid = contiguous_byte_strides(v->ne, x.bstride);
        allow_implicit = 0;
    } else if (v->nb[0] == 0) { /* with_strides, implicit sentinel */
        inferred_valid = contiguous_byte_strides(v->ne, x.bstride);
        allow_implicit = 1;
    } else {
        memcpy(x.bstride, v->nb, sizeof x.bstride);
        inferred_valid = 1;
        allow_implicit = 0;
    }
    uint64_t count = 1;
    int zero = 0;
    x.shape_valid = 1;
    x.strides_valid = inferred_valid;
    for (int d = 0; d < 3; d++) {
        const uint64_t extent = v->ne[d], stride = x.bstride[d];
        if (extent > 1 && stride == 0 && !allow_implicit) x.strides_valid = 0;
        if (stride != 0 && (stride < 4 || stride % 4 != 0)) x.strides_valid = 0;
        if (extent == 0) {
            zero = 1;
        } else if (!zero) {
            u128 c = (u128)count * extent;
            if (c > (u128)UINT64_MAX) {
                x.shape_valid = 0;
                count = 0;
            } else {
                count = (uint64_t)c;
            }
        }
    }
    if (zero) count = 0;
    x.count = count;
    x.span_valid = 0;
    if (x.strides_valid && x.shape_valid) {
        if (zero) {
            x.span_valid = 1;
        } else { /* span_fits (:198-216) */
            u128 max_offset = 0;
            int ok = 1;
            for (int d = 0; d < 3 && ok; d++) {
                u128 c = (u128)(v->ne[d] - 1) * x.bstride[d];
                if (max_offset > ~(u128)0 - c) ok = 0;
                else max_offset += c;
            }
            x.span_valid = ok && max_offset + 4 <= (u128)v->len * 4;
        }
    }
    return x;
}

static int ix_validate(const ix_t *x) { return x->shape_valid && x->strides_valid && x->span_valid; }

static int32_t ix_read(const ix_t *x, uint64_t ordinal)
{
    const uint64_t *ne = x->v->ne;
    const uint64_t i0 = ordinal % ne[0], rem = ordinal / ne[0];
    const uint64_t i1 = rem % ne[1], i2 = rem / ne[1];
    return x->v->data[i0 * (x->bstride[0] / 4) + i1 * (x->bstride[1] / 4) + i2 * (x->bstride[2] / 4)];
}

/* ---- views --------------------------------------------------------------------- */

static int count_of(const orc_view *v, uint64_t *count)
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

static int f32_strides(const orc_view *v, uint64_t st[4])
{
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

static int half_strides(const orc_view *v, uint64_t st[4])
{
    if (v->nb[0] != 0) {
        memcpy(st, v->nb, sizeof(uint64_t) * 4);
        return 1;
    }
    u128 s = 2;
    st[0] = 2;
    for (int d = 1; d < 4; d++) {
        s *= v->ne[d - 1];
        if (s > (u128)UINT64_MAX) return 0;
        st[d] = (uint64_t)s;
    }
    return 1;
}

/* Layout::validate / validate_binary for F32 (tensor_view.rs:365-447). */
static int f32_validate(const orc_view *v, int allow_singleton_zero)
{
    uint64_t count, st[4];
    if (v->dtype != DT_F32 || !count_of(v, &count) || !f32_strides(v, st)) return 0;
    for (int d = 0; d < 4; d++) {
        const int sz = allow_singleton_zero && v->ne[d] == 1 && st[d] == 0;
        if (!sz && (st[d] < 4 || st[d] % 4 != 0)) return 0;
    }
    u128 max_offset = 0;
    for (int d = 0; d < 4; d++) max_offset += (u128)(v->ne[d] - 1) * st[d];
    return max_offset + 4 <= (u128)(v->data_bytes / 4) * 4;
}

/* is_dense_contiguous_for (tensor_view.rs:297-314). */
static int dense_f32(const orc_view *v)
{
    if (v->dtype != DT_F32) return 0;
    u128 expect = 4;
    for (int d = 0; d < 4; d++) {
        if (v->nb[d] != expect) return 0;
        expect *= v->ne[d];
        if (expect > (u128)UINT64_MAX) return 0;
    }
    return 1;
}

/* ByteTensorView::validate (tensor_view.rs:588-645). */
static int bytes_validate(const orc_view *v)
{
    uint64_t count, st[4];
    if (v->dtype != DT_F32 || !count_of(v, &count)) return 0;
    if (v->nb[0] != 0) {
        if (v->nb[0] < 4 || v->nb[0] % 4 != 0) return 0;
        for (int d = 0; d < 4; d++)
            if (v->ne[d] > 1 && v->nb[d] == 0) return 0;
    }
    if (!f32_strides(v, st)) return 0;
    u128 max_offset = 0;
    for (int d = 1; d < 4; d++) max_offset += (u128)(v->ne[d] - 1) * st[d];
    return max_offset + (u128)v->ne[0] * 4 <= (u128)v->data_bytes;
}

static int half_span(const orc_view *v, const uint64_t st[4])
{
    u128 max_offset = 0;
    for (int d = 0; d < 4; d++) {
        u128 c = (u128)(v->ne[d] - 1) * st[d];
        if (max_offset > ~(u128)0 - c) return 0;
        max_offset += c;
    }
    return max_offset + 2 <= (u128)(v->data_bytes / 2) * 2;
}

/* F16View::validate (f16_matmul.rs:49-90). */
static int f16_validate(const orc_view *v)
{
    uint64_t st[4], count;
    if (!half_strides(v, st)) return 0;
    if (v->dtype != DT_F16 || !count_of(v, &count)) return 0;
    for (int d = 0; d < 4; d++)
        if (v->ne[d] > 1 && (st[d] < 2 || st[d] % 2 != 0)) return 0;
    return half_span(v, st);
}

/* Bf16View::validate (get_rows.rs:302-343). */
static int bf16_validate(const orc_view *v)
{
    uint64_t st[4], count;
    if (v->dtype != DT_BF16 || !count_of(v, &count)) return 0;
    if (!half_strides(v, st)) return 0;
    if (v->nb[0] != 0)
        for (int d = 0; d < 4; d++)
            if ((v->ne[d] > 1 && v->nb[d] == 0) || (v->nb[d] != 0 && (v->nb[d] < 2 || v->nb[d] % 2 != 0))) return 0;
    return half_span(v, st);
}

/* PackedRowView::validate (tensor_view.rs:487-532). */
static int packed_validate(const orc_view *v, uint32_t code, uint64_t bv, uint64_t bb)
{
    if (v->dtype != code || bv == 0) return 0;
    for (int d = 0; d < 4; d++)
        if (v->ne[d] == 0) return 0;
    if (v->ne[0] % bv != 0 || v->nb[0] != 1) return 0;
    u128 row = (u128)(v->ne[0] / bv) * bb;
    u128 rs2 = row * v->ne[1];
    u128 rs3 = rs2 * v->ne[2];
    if (row > (u128)UINT64_MAX || rs2 > (u128)UINT64_MAX || rs3 > (u128)UINT64_MAX) return 0;
    if (row == 0 || v->nb[1] != row || v->nb[2] != rs2 || v->nb[3] != rs3) return 0;
    u128 max_offset = 0;
    for (int d = 1; d < 4; d++) max_offset += (u128)(v->ne[d] - 1) * v->nb[d];
    return max_offset + row <= (u128)v->data_bytes;
}

/* empty_index_source_valid / empty_f32_bytes_source_valid /
 * empty_bf16_source_valid (get_rows.rs:883-943, :1076-1097). */
static int empty_source(const orc_view *v, uint32_t dtype, uint64_t elem, int any_multiple)
{
    if (v->dtype != dtype || v->ne[0] == 0 || v->ne[1] == 0) return 0;
    if (any_multiple) {
        if (v->nb[0] != 0 && (v->nb[0] < 4 || v->nb[0] % 4 != 0)) return 0;
    } else if (v->nb[0] != 0 && v->nb[0] != elem) {
        return 0;
    }
    if (v->nb[0] != 0)
        for (int d = 0; d < 4; d++)
            if (v->ne[d] > 1 && v->nb[d] == 0) return 0;
    return 1;
}

/* ---- reads ----------------------------------------------------------------------- */

static float rd_f32_bytes(const orc_view *v, uint64_t byte_offset)
{
    float x;
    memcpy(&x, (const unsigned char *)v->data + byte_offset, 4);
    return x;
}

/* f16_to_f32 (f16_matmul.rs:508-531). */
static float f16_exact(uint16_t bits)
{
    const uint32_t sign = (uint32_t)(bits & 0x8000u) << 16;
    const uint32_t exponent = (bits >> 10) & 0x1fu;
    const uint32_t fraction = bits & 0x3ffu;
    uint32_t value;
    if (exponent == 0) {
        if (fraction == 0) {
            value = sign;
        } else {
            uint32_t normalized = fraction, shift = 0;
            while ((normalized & 0x400u) == 0) {
                normalized <<= 1;
                shift++;
            }
            value = sign | ((127u - (14u + shift)) << 23) | ((normalized & 0x3ffu) << 13);
        }
    } else if (exponent == 0x1f) {
        value = sign | 0x7f800000u | (fraction << 13);
    } else {
        value = sign | ((exponent + 112u) << 23) | (fraction << 13);
    }
    float f;
    memcpy(&f, &value, 4);
    return f;
}

static float half_read(const orc_view *v, uint64_t ordinal, int bf16)
{
    uint64_t st[4], off = 0;
    half_strides(v, st);
    for (int d = 0; d < 4; d++) {
        off += (ordinal % v->ne[d]) * st[d];
        ordinal /= v->ne[d];
    }
    uint16_t h;
    memcpy(&h, (const unsigned char *)v->data + (off / 2) * 2, 2);
    if (bf16) {
        uint32_t bits = (uint32_t)h << 16;
        float f;
        memcpy(&f, &bits, 4);
        return f;
    }
    return f16_exact(h);
}

/* ---- block decoders (quant.rs:106-205, quant_more.rs:438-468) --------------------- */

static void decode_q4_0(const unsigned char *b, float out[32])
{
    const float scale = orc_fp16_to_f32((uint16_t)(b[0] | (b[1] << 8)));
    for (int i = 0; i < 16; i++) {
        const unsigned char p = b[i + 2];
        out[i] = ((float)(p & 0x0f) - 8.0f) * scale;
        out[i + 16] = ((float)(p >> 4) - 8.0f) * scale;
    }
}

static void decode_q8_0(const unsigned char *b, float out[32])
{
    const float scale = orc_fp16_to_f32((uint16_t)(b[0] | (b[1] << 8)));
    for (int i = 0; i < 32; i++) out[i] = (float)(int8_t)b[i + 2] * scale;
}

static void q4k_scale_min(int j, const unsigned char *s, unsigned *sc, unsigned *mn)
{
    if (j < 4) {
        *sc = s[j] & 0x3f;
        *mn = s[j + 4] & 0x3f;
    } else {
        *sc = (s[j + 4] & 0x0f) | ((s[j - 4] >> 6) << 4);
        *mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

static void decode_q4_k(const unsigned char *b, float out[256])
{
    const float scale = orc_fp16_to_f32((uint16_t)(b[0] | (b[1] << 8)));
    const float minimum = orc_fp16_to_f32((uint16_t)(b[2] | (b[3] << 8)));
    int si = 0;
    for (int off = 0; off < 256; off += 64, si += 2) {
        unsigned sa, ma, sb, mb;
        q4k_scale_min(si, b + 4, &sa, &ma);
        q4k_scale_min(si + 1, b + 4, &sb, &mb);
        const float d0 = scale * (float)sa, d1 = scale * (float)sb;
        const float m0 = minimum * (float)ma, m1 = minimum * (float)mb;
        const unsigned char *q = b + 16 + off / 2;
        for (int l = 0; l < 32; l++) {
            out[off + l] = d0 * (float)(q[l] & 0x0f) - m0;
            out[off + l + 32] = d1 * (float)(q[l] >> 4) - m1;
        }
    }
}

/* ---- the event ------------------------------------------------------------------------ */

int orc_get_rows(int kind, const orc_view *src, const orc_index_view *idx, const orc_view *dst)
{
    const ix_t x = ix_make(idx);
    const uint64_t n = ix_validate(&x) ? x.count : 0;
    /* views_valid* */
    int dst_ok, src_ok;
    if (n == 0 && kind != ORC_GR_F16) dst_ok = dense_f32(dst);
    else dst_ok = f32_validate(dst, 0) && dense_f32(dst);
    switch (kind) {
    case ORC_GR_F32: src_ok = n == 0 ? empty_source(src, DT_F32, 4, 0) : f32_validate(src, 1); break;
    case ORC_GR_F32_BYTES: src_ok = n == 0 ? empty_source(src, DT_F32, 4, 1) : bytes_validate(src); break;
    case ORC_GR_F16: src_ok = f16_validate(src); break;
    case ORC_GR_BF16: src_ok = n == 0 ? empty_source(src, DT_BF16, 2, 0) : bf16_validate(src); break;
    case ORC_GR_Q4_0: src_ok = packed_validate(src, 2, 32, 18); break;
    case ORC_GR_Q8_0: src_ok = packed_validate(src, 8, 32, 34); break;
    default: src_ok = packed_validate(src, 12, 256, 144); break;
    }
    if (!ix_validate(&x) || !src_ok || !dst_ok) return ORC_INVALID_VIEW;
    /* shape_valid */
    const uint64_t *s = src->ne, *i = idx->ne, *o = dst->ne;
    if (!(s[0] > 0 && s[1] > 0 && o[0] == s[0] && o[1] == i[0] && o[2] == i[1] && o[3] == i[2] && s[2] == i[1] &&
          s[3] == i[2]))
        return ORC_SHAPE_MISMATCH;
    /* source_stride_valid (F32 route only) */
    if (kind == ORC_GR_F32 && !(src->nb[0] == 0 || (src->nb[0] >= 4 && src->nb[0] % 4 == 0)))
        return ORC_UNSUPPORTED_SOURCE_STRIDE;
    /* indices_valid */
    for (uint64_t k = 0; k < n; k++) {
        const int32_t r = ix_read(&x, k);
        if (r < 0 || (uint64_t)r >= s[1]) return ORC_INDEX_OUT_OF_BOUNDS;
    }
    /* the action */
    const uint64_t cols = s[0];
    float *out = (float *)dst->data;
    uint64_t dst_row = 0;
    for (uint64_t i2 = 0; i2 < i[2]; i2++)
        for (uint64_t i1 = 0; i1 < i[1]; i1++)
            for (uint64_t i0 = 0; i0 < i[0]; i0++, dst_row++) {
                const uint64_t index = (uint64_t)ix_read(&x, dst_row);
                if (kind == ORC_GR_F32 || kind == ORC_GR_F32_BYTES) { /* read_row_contiguous */
                    uint64_t st[4];
                    f32_strides(src, st);
                    const uint64_t base = index * st[1] + i1 * st[2] + i2 * st[3];
                    for (uint64_t c = 0; c < cols; c++) out[dst_row * cols + c] = rd_f32_bytes(src, base + c * 4);
                } else if (kind == ORC_GR_F16 || kind == ORC_GR_BF16) {
                    const uint64_t source_row = i2 * s[2] * s[1] * cols + i1 * s[1] * cols + index * cols;
                    for (uint64_t c = 0; c < cols; c++)
                        out[dst_row * cols + c] = half_read(src, source_row + c, kind == ORC_GR_BF16);
                } else {
                    const uint64_t bv = kind == ORC_GR_Q4_K ? 256 : 32;
                    const uint64_t bb = kind == ORC_GR_Q4_0 ? 18 : kind == ORC_GR_Q8_0 ? 34 : 144;
                    const uint64_t row_bytes = (cols / bv) * bb;
                    const uint64_t source_row = (i2 * s[2] + i1) * s[1] + index;
                    const unsigned char *row = (const unsigned char *)src->data + source_row * row_bytes;
                    float decoded[256];
                    for (uint64_t b = 0; b < cols / bv; b++) {
                        if (kind == ORC_GR_Q4_0) decode_q4_0(row + b * bb, decoded);
                        else if (kind == ORC_GR_Q8_0) decode_q8_0(row + b * bb, decoded);
                        else decode_q4_k(row + b * bb, decoded);
                        for (uint64_t c = 0; c < bv; c++) out[dst_row * cols + b * bv + c] = decoded[c];
                    }
                }
            }
    return ORC_OK;
}
