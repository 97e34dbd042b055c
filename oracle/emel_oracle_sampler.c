/*
 * emel_oracle_sampler.c -- CPU restatement of emel-logits' native sampler
 * and candidate validator.
 *
 * TEST INFRASTRUCTURE ONLY (the checker, never the product).  See
 * emel_oracle.h.  Build: oracle/Makefile (gcc -O2 -ffp-contract=off).
 *
 * Reference file:line citations are relative to
 * stateforward/emel.rs:crates/emel-logits/src/.
 *
 * Rust's f32 arithmetic maps one to one onto C float arithmetic here
 * (no contraction), f32::exp and f32::ln onto glibc expf / logf, and
 * f32::max onto "keep the non-NaN operand".
 *
 * Pinning (tests/test_oracle_sampler.py): the reference's unit tests
 * (sampler/sm.rs:896-1055, tests/validator.rs); the Park-Miller minimal
 * standard generator's published check value (seed 1, 10,000 steps ->
 * 1043618065); the sequential f32 sum against a numpy float32 loop; the
 * softmax against float64; the ranking against numpy's stable argsort of
 * -p; the race selection against a float64 evaluation away from near-ties.
 */
#include "emel_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define RANDOM_MODULUS 2147483647u /* sampler/sm.rs:22 */
#define RANDOM_MULTIPLIER 16807u   /* sampler/sm.rs:23 */

static inline uint32_t bits_of(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

/* f32::total_cmp as an unsigned key: flip the magnitude bits of negative
 * values, set the sign bit of positive ones. */
static inline uint32_t total_key(float f)
{
    const uint32_t b = bits_of(f);
    return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}

/* sort_unstable_by(|a, b| v[b].total_cmp(&v[a])) (sampler/sm.rs:810): a
 * descending total order.  The reference leaves the order of equal values
 * unspecified; the oracle breaks ties by ascending index. */
static const float *g_rank_values;
static int rank_cmp(const void *pa, const void *pb)
{
    const int32_t a = *(const int32_t *)pa, b = *(const int32_t *)pb;
    const uint32_t ka = total_key(g_rank_values[a]), kb = total_key(g_rank_values[b]);
    if (ka != kb) return ka > kb ? -1 : 1;
    return a < b ? -1 : (a > b);
}

uint32_t orc_park_miller_next(uint32_t state)
{
    /* sampler/sm.rs:834 */
    return (uint32_t)(((uint64_t)state * RANDOM_MULTIPLIER) % RANDOM_MODULUS);
}

/* The softmax of sampler/sm.rs:773-795: f32::max fold from -inf, expf of
 * the difference written in place, a sequential f32 sum, then a division.
 * Returns the sum. */
float orc_sampler_softmax(float *values, uint64_t card)
{
    float maximum = -INFINITY;
    for (uint64_t i = 0; i < card; i++) {
        const float v = values[i];
        /* f32::max: a NaN operand yields the other one */
        if (isnan(maximum) || v > maximum) maximum = isnan(v) ? maximum : v;
    }
    float total = 0.0f;
    for (uint64_t i = 0; i < card; i++) {
        values[i] = expf(values[i] - maximum);
        total += values[i];
    }
    for (uint64_t i = 0; i < card; i++) values[i] /= total;
    return total;
}

/* Sampler::sample_temperature_top_k (sampler/sm.rs:380-392): guard
 * (:729-747), scale (:759-771), softmax (:773-795), rank (:797-819),
 * select (:821-847), result guard (:849-858).  Returns ORC_OK or
 * ORC_INVALID_REQUEST; on a failed request guard nothing is written, on a
 * failed result guard the outputs are written (as the reference's select
 * step does before its guard runs). */
int orc_sample_temperature_top_k(uint64_t card, float temperature, uint64_t top_k, float *logits,
                                 uint64_t logits_len, int32_t *sorted_indices, uint64_t sorted_len,
                                 float *top_probabilities, uint64_t top_probabilities_len, int32_t *top_indices,
                                 uint64_t top_indices_len, uint32_t *random_state, int32_t *selected_token_out,
                                 float *selected_score_out)
{
    if (!(card > 0 && top_k > 0 && top_k <= card && isfinite(temperature) && temperature > 0.0f &&
          logits_len >= card && sorted_len >= card && top_probabilities_len >= top_k && top_indices_len >= top_k &&
          *random_state % RANDOM_MODULUS != 0))
        return ORC_INVALID_REQUEST;

    const float scale = 1.0f / temperature;
    for (uint64_t i = 0; i < card; i++) logits[i] *= scale;

    orc_sampler_softmax(logits, card);

    for (uint64_t i = 0; i < card; i++) sorted_indices[i] = (int32_t)i;
    g_rank_values = logits;
    qsort(sorted_indices, card, sizeof(int32_t), rank_cmp);
    for (uint64_t slot = 0; slot < top_k; slot++) {
        const int32_t index = sorted_indices[slot];
        top_probabilities[slot] = logits[index];
        top_indices[slot] = index;
    }

    uint32_t state = *random_state;
    int32_t selected = -1;
    float score = -INFINITY;
    for (uint64_t slot = 0; slot < top_k; slot++) {
        state = orc_park_miller_next(state);
        const float uniform = (float)state / (float)RANDOM_MODULUS;
        const float race = top_probabilities[slot] / -logf(uniform);
        if (race > score) {
            score = race;
            selected = top_indices[slot];
        }
    }
    *random_state = state;
    *selected_token_out = selected;
    *selected_score_out = score;
    if (!(selected >= 0 && (uint64_t)selected < card && isfinite(score))) return ORC_INVALID_REQUEST;
    return ORC_OK;
}

/* Validator::process_event(Build) (validator/sm.rs): begin_build resets the
 * count and error, valid_request checks the sizes, execute_build writes ids
 * and logits - max (max from logits[0] by strict >), publish_error resets
 * the count.  error_out takes ValidatorError's discriminant
 * (None = 0, InvalidRequest = 1). */
int orc_validator_build(const float *logits, uint64_t logits_len, int32_t vocab_size, int32_t *candidate_ids,
                        uint64_t ids_len, float *candidate_scores, uint64_t scores_len, int32_t candidate_capacity,
                        int32_t *candidate_count_out, int32_t *error_out)
{
    *candidate_count_out = 0;
    *error_out = 0;
    const int valid = vocab_size > 0 && candidate_capacity >= vocab_size && logits_len <= INT32_MAX &&
                      (int64_t)logits_len >= vocab_size && ids_len <= INT32_MAX && (int64_t)ids_len >= vocab_size &&
                      scores_len <= INT32_MAX && (int64_t)scores_len >= vocab_size;
    if (!valid) {
        *candidate_count_out = 0;
        *error_out = 1;
        return ORC_INVALID_REQUEST;
    }
    float maximum = logits[0];
    for (int32_t i = 0; i < vocab_size; i++) {
        const float score = logits[i];
        candidate_ids[i] = i;
        candidate_scores[i] = score;
        if (score > maximum) maximum = score;
    }
    for (int32_t i = 0; i < vocab_size; i++) candidate_scores[i] = candidate_scores[i] - maximum;
    *candidate_count_out = vocab_size;
    return ORC_OK;
}
