/*
 * kq_sample.c — CPU restatement of the reference's token sampler.
 *
 * TEST INFRASTRUCTURE ONLY (the checker). Never linked into libkq_hip.so.
 *
 * Follows src/kq_sampling.c: the PCG-XSH-RR 64/32 stream (M. O'Neill's
 * published generator; seeding :121-134, step :110-119), the RNG state
 * record's integrity word (:83-96), and kq_sampling_select_f32 (:576-772):
 *   scores = logits / temperature (when temperature != 1);
 *   ids sorted by (score, id) ascending (:276-331, a stable merge sort);
 *   top-k keeps every id whose score reaches the k-th largest (ties kept);
 *   weights expf(score - max) summed in ascending-score order;
 *   top-p drops ids from the low end while the running sum of p = w / sum
 *   stays at or below 1 - top_p (:676-690);
 *   the kept weights are summed again in id order, normalised in id order;
 *   the categorical draw maps the next word to uniform = word / 2^32 and
 *   walks the binary64 running sum in id order (:400-447).
 * Pinned by the reference's calibration, holdout and RNG vectors
 * (tests/golden/sampling_vectors.json) and by the reference's own
 * kq_sampling_select_f32 (oracle/_ref) on seeded cases.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "kq_oracle.h"

#define PCG_MULT 6364136223846793005ULL
#define FNV_OFFSET 1469598103934665603ULL
#define FNV_PRIME 1099511628211ULL

static uint32_t pcg_step(uint64_t *state, uint64_t inc) {
    const uint64_t old = *state;
    *state = old * PCG_MULT + inc;
    const uint32_t xs = (uint32_t)(((old >> 18U) ^ old) >> 27U);
    const uint32_t rot = (uint32_t)(old >> 59U);
    return (xs >> rot) | (xs << ((0U - rot) & 31U));
}

static uint64_t integrity(const kqo_rng_state *s) {
    const uint64_t f[7] = {s->version, s->reserved, s->seed, s->stream,
                           s->state, s->increment, s->draws};
    uint64_t h = FNV_OFFSET;
    for (int i = 0; i < 7; ++i) {
        h ^= f[i];
        h *= FNV_PRIME;
    }
    return h;
}

void kqo_rng_seed(uint64_t seed, uint64_t stream, kqo_rng_state *out) {
    const uint64_t inc = (stream << 1U) | 1U;
    uint64_t st = 0U;
    (void)pcg_step(&st, inc);
    st += seed;
    (void)pcg_step(&st, inc);
    out->version = 1U;
    out->reserved = 0U;
    out->seed = seed;
    out->stream = stream;
    out->state = st;
    out->increment = inc;
    out->draws = 0U;
    out->integrity = integrity(out);
}

uint32_t kqo_rng_next(kqo_rng_state *s) {
    const uint32_t w = pcg_step(&s->state, s->increment);
    s->draws += 1U;
    s->integrity = integrity(s);
    return w;
}

/* (score, id) ascending */
static const float *g_scores;
static int by_score_id(const void *a, const void *b) {
    const uint32_t x = *(const uint32_t *)a, y = *(const uint32_t *)b;
    if (g_scores[x] < g_scores[y]) return -1;
    if (g_scores[y] < g_scores[x]) return 1;
    return x < y ? -1 : (x > y ? 1 : 0);
}

int kqo_sample_f32(float temperature, float top_p, uint32_t top_k, uint32_t canonical_count,
                   const float *logits, uint32_t count, uint32_t word, kqo_sample_result *r,
                   float *scores_out, float *probs_out) {
    float *scores = (float *)malloc(sizeof(float) * count);
    float *prob = (float *)calloc(count, sizeof(float));
    uint32_t *order = (uint32_t *)malloc(sizeof(uint32_t) * count);
    int st = KQO_OK;
    uint32_t i, top_start = 0U, keep_start;
    float maximum, sum, norm_sum, maxp;
    double total = 0.0, cum = 0.0, uniform, thr;
    uint32_t last = UINT32_MAX, sel = UINT32_MAX;
    memset(r, 0, sizeof(*r));
    if (scores == NULL || prob == NULL || order == NULL || count == 0U) {
        st = KQO_INVALID_ARGUMENT;
        goto done;
    }
    for (i = 0U; i < count; ++i) {
        float v = logits[i];
        if (!isfinite(v)) { st = KQO_NUMERIC_DOMAIN; goto done; }
        if (temperature != 1.0f) {
            v = v / temperature;
            if (!isfinite(v)) { st = KQO_NUMERIC_DOMAIN; goto done; }
        }
        scores[i] = v;
        order[i] = i;
    }
    g_scores = scores;
    qsort(order, count, sizeof(uint32_t), by_score_id);
    if (top_k != 0U) {
        const float t = scores[order[count - top_k]];
        while (top_start < count && scores[order[top_start]] < t) ++top_start;
    }
    if (top_start >= count) { st = KQO_NUMERIC_DOMAIN; goto done; }
    r->top_k_retained_count = count - top_start;
    maximum = scores[order[count - 1U]];
    sum = 0.0f;
    for (i = top_start; i < count; ++i) {
        const float w = kqo_expf(scores[order[i]] - maximum);
        if (!isfinite(w) || w < 0.0f) { st = KQO_NUMERIC_DOMAIN; goto done; }
        prob[order[i]] = w;
        sum = sum + w;
    }
    if (!isfinite(sum) || sum <= 0.0f) { st = KQO_NUMERIC_DOMAIN; goto done; }
    keep_start = top_start;
    if (top_p < 1.0f) {
        const float cutoff = 1.0f - top_p;
        float c = 0.0f;
        for (i = top_start; i < count; ++i) {
            const float p = prob[order[i]] / sum;
            c = c + p;
            if (i == count - 1U || c > cutoff) {
                keep_start = i;
                break;
            }
            prob[order[i]] = 0.0f;
            keep_start = i + 1U;
        }
    }
    if (keep_start >= count) { st = KQO_NUMERIC_DOMAIN; goto done; }
    for (i = top_start; i < keep_start; ++i) prob[order[i]] = 0.0f;
    r->retained_count = count - keep_start;
    sum = 0.0f;
    for (i = 0U; i < count; ++i)
        if (prob[i] > 0.0f) {
            const float w = kqo_expf(scores[i] - maximum);
            prob[i] = w;
            sum = sum + w;
        }
    if (!isfinite(sum) || sum <= 0.0f) { st = KQO_NUMERIC_DOMAIN; goto done; }
    norm_sum = 0.0f;
    maxp = 0.0f;
    for (i = 0U; i < count; ++i)
        if (prob[i] > 0.0f) {
            const float p = prob[i] / sum;
            if (!isfinite(p) || p < 0.0f) { st = KQO_NUMERIC_DOMAIN; goto done; }
            prob[i] = p;
            norm_sum = norm_sum + p;
            if (p > maxp) maxp = p;
        }
    if (!isfinite(norm_sum) || norm_sum <= 0.0f) { st = KQO_NUMERIC_DOMAIN; goto done; }
    r->maximum_probability = maxp;
    r->normalized_sum_f32 = norm_sum;
    /* the categorical draw (src/kq_sampling.c:400-447) */
    for (i = 0U; i < count; ++i)
        if (prob[i] > 0.0f) {
            total += (double)prob[i];
            last = i;
        }
    uniform = (double)word / 4294967296.0;
    thr = uniform * total;
    for (i = 0U; i < count; ++i) {
        cum += (double)prob[i];
        if (prob[i] > 0.0f && thr < cum) {
            sel = i;
            break;
        }
    }
    if (sel == UINT32_MAX) {
        if (thr < total) sel = last;
        else { st = KQO_NUMERIC_DOMAIN; goto done; }
    }
    r->selected_token_id = sel; /* also reported with INVALID_TOKEN_ID */
    if (sel >= canonical_count) { st = KQO_INVALID_TOKEN_ID; goto done; }
    r->rng_word = word;
    r->selected_probability = prob[sel];
    r->uniform_value = uniform;
done:
    if (st == KQO_OK || st == KQO_INVALID_TOKEN_ID) {
        if (scores_out) memcpy(scores_out, scores, sizeof(float) * count);
        if (probs_out) memcpy(probs_out, prob, sizeof(float) * count);
    }
    free(scores);
    free(prob);
    free(order);
    return st;
}
