/*
 * c_caller.c -- a plain C99 caller of the emel-hip C ABI, standing in for
 * the Rust FFI crate (or a cgo / JNI binding): include/emel_hip.h compiles
 * as C, libemel_hip.so links and runs without C++, Python or torch, and
 * every buffer is device memory the library itself allocates.
 *
 *   c_caller cpu   host-only entry points and guards; on a machine without
 *                  a gfx950 device an accepted op must report
 *                  EMEL_ERR_KERNEL_UNAVAILABLE (there is no CPU fallback)
 *   c_caller gpu   the above plus ops run on device 0 and checked here:
 *                  broadcast add (exact), scaled + masked soft_max (within
 *                  1e-6 of a sequential double-sum softmax), per-row argmax
 *                  (exact), the logits validator (exact) and the sampler
 *                  (ranking, Park-Miller state and the race's invariants)
 *
 * Prints one line per check and "c_caller <mode>: ok" at the end; exits 1
 * on the first failure.  Built by __graft_entry__.build() with
 * gcc -std=c99 -Wall -Wextra -Werror -pedantic.
 */
#include "emel_hip.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static int g_failed = 0;

#define CHECK(cond, ...)                                                                            \
    do {                                                                                            \
        if (!(cond)) {                                                                              \
            printf("FAIL %s:%d: ", __FILE__, __LINE__);                                              \
            printf(__VA_ARGS__);                                                                    \
            printf(" [%s]\n", emel_last_error());                                                   \
            g_failed = 1;                                                                           \
            return 1;                                                                               \
        }                                                                                           \
    } while (0)

#define STATUS(call, want)                                                                          \
    do {                                                                                            \
        const emel_status st_ = (call);                                                             \
        CHECK(st_ == (want), "%s returned %d (%s), expected %d", #call, (int)st_,                   \
              emel_status_string(st_), (int)(want));                                                \
    } while (0)

static emel_tensor_view view_f32(const void *data, uint64_t bytes, uint64_t n0, uint64_t n1, uint64_t n2,
                                 uint64_t n3)
{
    emel_tensor_view v;
    memset(&v, 0, sizeof v);
    v.data = data;
    v.data_bytes = bytes;
    v.dtype = EMEL_DTYPE_F32;
    v.ne[0] = n0; v.ne[1] = n1; v.ne[2] = n2; v.ne[3] = n3;
    v.nb[0] = 4; v.nb[1] = 4 * n0; v.nb[2] = 4 * n0 * n1; v.nb[3] = 4 * n0 * n1 * n2;
    return v;
}

static emel_tensor_view_mut view_mut(void *data, uint64_t bytes, uint32_t dtype, uint64_t n0, uint64_t n1,
                                     uint64_t n2, uint64_t n3)
{
    const uint64_t es = 4;
    emel_tensor_view_mut v;
    memset(&v, 0, sizeof v);
    v.data = data;
    v.data_bytes = bytes;
    v.dtype = dtype;
    v.ne[0] = n0; v.ne[1] = n1; v.ne[2] = n2; v.ne[3] = n3;
    v.nb[0] = es; v.nb[1] = es * n0; v.nb[2] = es * n0 * n1; v.nb[3] = es * n0 * n1 * n2;
    return v;
}

/* x * 16807 mod (2^31 - 1), the Park-Miller minimal standard step */
static uint32_t park_miller(uint32_t s) { return (uint32_t)(((uint64_t)s * 16807u) % 2147483647u); }

/* deterministic inputs: a 32-bit LCG mapped to [-4, 4) */
static uint32_t g_lcg = 2463534242u;
static float uniform_pm4(void)
{
    g_lcg = g_lcg * 1664525u + 1013904223u;
    return (float)(g_lcg >> 8) / 16777216.0f * 8.0f - 4.0f;
}

static int check_host(int have_gpu)
{
    float host[16] = {0};
    emel_tensor_view v;
    int32_t tok = -1, count = -1;

    CHECK(emel_abi_version() == EMEL_HIP_ABI_VERSION, "abi version %u", emel_abi_version());
    for (int s = 0; s <= 13; ++s) CHECK(emel_status_string((emel_status)s) != NULL, "status string %d", s);
    STATUS(emel_device_count(&count), EMEL_OK);
    printf("devices: %d\n", count);
    CHECK(have_gpu ? count > 0 : count == 0, "device count %d", count);

    /* Layout::validate: the span must fit the allocation */
    v = view_f32(host, 16, 4, 1, 1, 1);
    STATUS(emel_validate_view(&v, 0), EMEL_OK);
    v.data_bytes = 12;
    STATUS(emel_validate_view(&v, 0), EMEL_ERR_INVALID_VIEW);

    /* sample_preselected: host only, token must be inside the vocabulary */
    STATUS(emel_sample_preselected(10, 3, &tok), EMEL_OK);
    CHECK(tok == 3, "preselected token %d", tok);
    STATUS(emel_sample_preselected(10, 10, &tok), EMEL_ERR_INVALID_REQUEST);
    STATUS(emel_sample_preselected(10, -1, &tok), EMEL_ERR_INVALID_REQUEST);

    if (!have_gpu) {
        /* an accepted request with no device: reported, never run on the CPU */
        emel_tensor_view in = view_f32(host, sizeof host, 16, 1, 1, 1);
        emel_tensor_view_mut out = view_mut(host, sizeof host, EMEL_DTYPE_F32, 16, 1, 1, 1);
        STATUS(emel_op_silu(&in, &out, NULL), EMEL_ERR_KERNEL_UNAVAILABLE);
    }
    printf("host checks: ok\n");
    return 0;
}

#define NE0 1000
#define NE1 6
#define NE2 2
#define CARD 1000
#define TOPK 10

static int check_gpu(void)
{
    const uint64_t n = (uint64_t)NE0 * NE1 * NE2, rows = (uint64_t)NE1 * NE2;
    float *hx = malloc(n * 4), *hy = malloc(n * 4), *hrow = malloc(NE0 * 4);
    uint16_t *hmask = malloc((uint64_t)NE0 * NE1 * 2);
    int32_t *hidx = malloc(rows * 4);
    void *dx = NULL, *dy = NULL, *drow = NULL, *dmask = NULL, *didx = NULL;
    emel_stream stream = NULL;
    uint64_t i, r;

    CHECK(hx && hy && hrow && hmask && hidx, "host allocation");
    for (i = 0; i < n; ++i) hx[i] = uniform_pm4();
    for (i = 0; i < NE0; ++i) hrow[i] = uniform_pm4();
    for (r = 0; r < rows; ++r) hx[r * NE0 + (r * 97) % NE0] = 9.0f + (float)r; /* planted row maxima */
    for (r = 0; r < NE1; ++r)
        for (i = 0; i < NE0; ++i) hmask[r * NE0 + i] = (i <= 900 + r * 10) ? 0x0000 : 0xfc00; /* 0 / -inf */

    STATUS(emel_set_device(0), EMEL_OK);
    STATUS(emel_stream_create(&stream), EMEL_OK);
    {   /* scratch reserved and tables built up front (no counterpart in the reference) */
        uint64_t work = 1, counters = 1;
        STATUS(emel_stream_workspace(stream, &work, &counters), EMEL_OK);
        CHECK(work == 0 && counters == 0, "fresh stream holds %llu / %llu bytes", (unsigned long long)work,
              (unsigned long long)counters);
        STATUS(emel_stream_reserve(stream, 3u << 20, 1u << 20), EMEL_OK);
        STATUS(emel_stream_workspace(stream, &work, &counters), EMEL_OK);
        CHECK(work >= (3u << 20) && counters >= (1u << 20), "reserved %llu / %llu bytes", (unsigned long long)work,
              (unsigned long long)counters);
        STATUS(emel_stream_workspace(stream, NULL, &counters), EMEL_ERR_INVALID_ARGUMENT);
        STATUS(emel_device_prepare(stream), EMEL_OK);
        printf("stream_reserve / device_prepare: ok\n");
    }
    STATUS(emel_malloc(&dx, n * 4), EMEL_OK);
    STATUS(emel_malloc(&dy, n * 4), EMEL_OK);
    STATUS(emel_malloc(&drow, NE0 * 4), EMEL_OK);
    STATUS(emel_malloc(&dmask, (uint64_t)NE0 * NE1 * 2), EMEL_OK);
    STATUS(emel_malloc(&didx, rows * 4), EMEL_OK);
    STATUS(emel_memcpy_htod(dx, hx, n * 4, stream), EMEL_OK);
    STATUS(emel_memcpy_htod(drow, hrow, NE0 * 4, stream), EMEL_OK);
    STATUS(emel_memcpy_htod(dmask, hmask, (uint64_t)NE0 * NE1 * 2, stream), EMEL_OK);

    {   /* broadcast row add: bit-exact IEEE f32 */
        emel_tensor_view a = view_f32(dx, n * 4, NE0, NE1, NE2, 1);
        emel_tensor_view b = view_f32(drow, NE0 * 4, NE0, 1, 1, 1);
        emel_tensor_view bad = view_f32(drow, NE0 * 4, NE0 - 1, 1, 1, 1);
        emel_tensor_view_mut o = view_mut(dy, n * 4, EMEL_DTYPE_F32, NE0, NE1, NE2, 1);
        STATUS(emel_op_add_broadcast_row(&a, &b, &o, stream), EMEL_OK);
        STATUS(emel_memcpy_dtoh(hy, dy, n * 4, stream), EMEL_OK);
        STATUS(emel_stream_synchronize(stream), EMEL_OK);
        for (i = 0; i < n; ++i) CHECK(hy[i] == hx[i] + hrow[i % NE0], "add_broadcast_row at %llu", (unsigned long long)i);
        STATUS(emel_op_add_broadcast_row(&a, &bad, &o, stream), EMEL_ERR_SHAPE_MISMATCH);
        printf("add_broadcast_row: exact\n");
    }

    {   /* scaled + masked soft_max, per row against a sequential double sum */
        const float scale = 0.5f;
        emel_tensor_view a = view_f32(dx, n * 4, NE0, NE1, NE2, 1);
        emel_tensor_view m;
        emel_tensor_view_mut o = view_mut(dy, n * 4, EMEL_DTYPE_F32, NE0, NE1, NE2, 1);
        double worst = 0.0;
        memset(&m, 0, sizeof m);
        m.data = dmask; m.data_bytes = (uint64_t)NE0 * NE1 * 2; m.dtype = EMEL_DTYPE_F16;
        m.ne[0] = NE0; m.ne[1] = NE1; m.ne[2] = 1; m.ne[3] = 1;
        m.nb[0] = 2; m.nb[1] = 2 * NE0; m.nb[2] = 2 * NE0 * NE1; m.nb[3] = m.nb[2];
        STATUS(emel_op_soft_max_ext(&a, &m, scale, &o, stream), EMEL_OK);
        STATUS(emel_memcpy_dtoh(hy, dy, n * 4, stream), EMEL_OK);
        STATUS(emel_stream_synchronize(stream), EMEL_OK);
        for (r = 0; r < rows; ++r) {
            const float *x = hx + r * NE0;
            const uint16_t *mk = hmask + (r % NE1) * NE0;
            float v[NE0], mx = -INFINITY;
            double sum = 0.0;
            for (i = 0; i < NE0; ++i) {
                v[i] = x[i] * scale + (mk[i] ? -INFINITY : 0.0f);
                if (v[i] > mx) mx = v[i];
            }
            for (i = 0; i < NE0; ++i) {
                v[i] = expf(v[i] - mx);
                sum += (double)v[i];
            }
            for (i = 0; i < NE0; ++i) {
                const float want = v[i] / (float)sum, got = hy[r * NE0 + i];
                const double err = fabs((double)got - (double)want);
                CHECK(err <= 1e-6 * fabs((double)want), "soft_max_ext row %llu col %llu: %.9g vs %.9g",
                      (unsigned long long)r, (unsigned long long)i, (double)got, (double)want);
                if (want > 0.0f && err / want > worst) worst = err / want;
            }
        }
        printf("soft_max_ext: max relative difference %.3g\n", worst);
    }

    {   /* per-row argmax: the planted maxima, exactly */
        emel_tensor_view a = view_f32(dx, n * 4, NE0, NE1, NE2, 1);
        emel_tensor_view_mut o = view_mut(didx, rows * 4, EMEL_DTYPE_I32, 1, NE1, NE2, 1);
        STATUS(emel_op_argmax_rows(&a, &o, stream), EMEL_OK);
        STATUS(emel_memcpy_dtoh(hidx, didx, rows * 4, stream), EMEL_OK);
        STATUS(emel_stream_synchronize(stream), EMEL_OK);
        for (r = 0; r < rows; ++r) CHECK(hidx[r] == (int32_t)((r * 97) % NE0), "argmax row %llu: %d", (unsigned long long)r, hidx[r]);
        printf("argmax_rows: exact\n");
    }

    {   /* logits validator: ids 0..n-1, scores logits - max (max from column 0, strict >) */
        int32_t count = -1, err = -1;
        float mx = hx[0];
        STATUS(emel_logits_validator_build((const float *)dx, CARD, CARD, (int32_t *)didx, 0, (float *)dy, CARD, CARD,
                                           &count, &err, stream),
               EMEL_ERR_INVALID_REQUEST);
        CHECK(count == 0 && err == EMEL_VALIDATOR_INVALID_REQUEST, "validator guard: count %d error %d", count, err);
        {
            void *dids = NULL;
            int32_t *hids = malloc(CARD * 4);
            CHECK(hids != NULL, "host allocation");
            STATUS(emel_malloc(&dids, CARD * 4), EMEL_OK);
            STATUS(emel_logits_validator_build((const float *)dx, CARD, CARD, (int32_t *)dids, CARD, (float *)dy, CARD,
                                               CARD, &count, &err, stream),
                   EMEL_OK);
            STATUS(emel_memcpy_dtoh(hids, dids, CARD * 4, stream), EMEL_OK);
            STATUS(emel_memcpy_dtoh(hy, dy, CARD * 4, stream), EMEL_OK);
            STATUS(emel_stream_synchronize(stream), EMEL_OK);
            CHECK(count == CARD && err == EMEL_VALIDATOR_NONE, "validator: count %d error %d", count, err);
            for (i = 1; i < CARD; ++i)
                if (hx[i] > mx) mx = hx[i];
            for (i = 0; i < CARD; ++i) {
                CHECK(hids[i] == (int32_t)i, "validator id %llu", (unsigned long long)i);
                CHECK(hy[i] == hx[i] - mx, "validator score %llu", (unsigned long long)i);
            }
            STATUS(emel_free(dids), EMEL_OK);
            free(hids);
        }
        printf("logits_validator_build: exact\n");
    }

    {   /* temperature / top-k sampling over one row of well-separated logits */
        float logits[CARD], topp[TOPK], score = 0.0f;
        int32_t topi[TOPK], token = -1, status = -1, order[TOPK];
        uint32_t state = 12345u, want_state = 12345u;
        void *dl = NULL, *ds = NULL, *dtp = NULL, *dti = NULL, *dtok = NULL, *dsc = NULL, *dst = NULL;
        emel_sample_temperature_top_k_request q;
        int k;
        for (i = 0; i < CARD; ++i) logits[i] = (float)((i * 389) % CARD) * 0.01f; /* a permutation of 0.00 .. 9.99 */
        for (k = 0; k < TOPK; ++k) {
            /* rank k holds value 9.99 - 0.01 k, at the index i with i*389 % CARD == 999 - k */
            for (i = 0; i < CARD; ++i)
                if ((i * 389) % CARD == (uint64_t)(CARD - 1 - k)) order[k] = (int32_t)i;
            want_state = park_miller(want_state);
        }
        STATUS(emel_malloc(&dl, CARD * 4), EMEL_OK);
        STATUS(emel_malloc(&ds, CARD * 4), EMEL_OK);
        STATUS(emel_malloc(&dtp, TOPK * 4), EMEL_OK);
        STATUS(emel_malloc(&dti, TOPK * 4), EMEL_OK);
        STATUS(emel_malloc(&dtok, 4), EMEL_OK);
        STATUS(emel_malloc(&dsc, 4), EMEL_OK);
        STATUS(emel_malloc(&dst, 4), EMEL_OK);
        STATUS(emel_memcpy_htod(dl, logits, CARD * 4, stream), EMEL_OK);
        memset(&q, 0, sizeof q);
        q.card = CARD; q.temperature = 0.7f; q.top_k = 0;
        q.logits = (float *)dl; q.logits_len = CARD;
        q.sorted_indices = (int32_t *)ds; q.sorted_indices_len = CARD;
        q.top_probabilities = (float *)dtp; q.top_probabilities_len = TOPK;
        q.top_indices = (int32_t *)dti; q.top_indices_len = TOPK;
        q.random_state = &state;
        q.selected_token_out = (int32_t *)dtok; q.selected_score_out = (float *)dsc; q.status_out = (int32_t *)dst;
        STATUS(emel_sample_temperature_top_k(&q, stream), EMEL_ERR_INVALID_REQUEST); /* top_k == 0 */
        CHECK(state == 12345u, "state changed by a rejected request");
        q.top_k = TOPK;
        STATUS(emel_sample_temperature_top_k(&q, stream), EMEL_OK);
        STATUS(emel_memcpy_dtoh(topp, dtp, TOPK * 4, stream), EMEL_OK);
        STATUS(emel_memcpy_dtoh(topi, dti, TOPK * 4, stream), EMEL_OK);
        STATUS(emel_memcpy_dtoh(&token, dtok, 4, stream), EMEL_OK);
        STATUS(emel_memcpy_dtoh(&score, dsc, 4, stream), EMEL_OK);
        STATUS(emel_memcpy_dtoh(&status, dst, 4, stream), EMEL_OK);
        STATUS(emel_stream_synchronize(stream), EMEL_OK);
        CHECK(state == want_state, "random_state %u, expected %u after %d draws", state, want_state, TOPK);
        CHECK(status == EMEL_OK, "device result guard %d", status);
        for (k = 0; k < TOPK; ++k) {
            CHECK(topi[k] == order[k], "rank %d: index %d, expected %d", k, topi[k], order[k]);
            CHECK(k == 0 || topp[k] < topp[k - 1], "probabilities not descending at rank %d", k);
        }
        {
            int found = 0;
            for (k = 0; k < TOPK; ++k) found |= token == topi[k];
            CHECK(found && isfinite(score) && score > 0.0f, "selected %d score %g", token, (double)score);
        }
        printf("sample_temperature_top_k: token %d score %.6g, state %u\n", token, (double)score, state);
        STATUS(emel_free(dl), EMEL_OK); STATUS(emel_free(ds), EMEL_OK); STATUS(emel_free(dtp), EMEL_OK);
        STATUS(emel_free(dti), EMEL_OK); STATUS(emel_free(dtok), EMEL_OK); STATUS(emel_free(dsc), EMEL_OK);
        STATUS(emel_free(dst), EMEL_OK);
    }

    STATUS(emel_free(dx), EMEL_OK);
    STATUS(emel_free(dy), EMEL_OK);
    STATUS(emel_free(drow), EMEL_OK);
    STATUS(emel_free(dmask), EMEL_OK);
    STATUS(emel_free(didx), EMEL_OK);
    STATUS(emel_release_workspaces(), EMEL_OK);
    STATUS(emel_stream_destroy(stream), EMEL_OK);
    free(hx); free(hy); free(hrow); free(hmask); free(hidx);
    return 0;
}

int main(int argc, char **argv)
{
    const int gpu = argc > 1 && strcmp(argv[1], "gpu") == 0;
    if (argc < 2 || (!gpu && strcmp(argv[1], "cpu") != 0)) {
        fprintf(stderr, "usage: %s cpu|gpu\n", argv[0]);
        return 2;
    }
    setvbuf(stdout, NULL, _IOLBF, 0);
    if (check_host(gpu) || (gpu && check_gpu())) return 1;
    printf("c_caller %s: ok\n", gpu ? "gpu" : "cpu");
    return g_failed;
}
