/*
 * kq_hip_sampling.c — host side of the device token sampler
 * (include/kq_hip.h, "Token sampling on the device").
 *
 * C17. The policy and RNG functions restate src/kq_sampling.c:83-322 on
 * the host: PCG-XSH-RR 64/32 (M. O'Neill's published generator; the
 * increment is (stream << 1) | 1, seeding steps once, adds the seed and
 * steps again) and an FNV-1a-style integrity word over the record's seven
 * fields. Selection validates in the reference's order
 * (src/kq_sampling.c:601-640), draws the next word on the host, runs the
 * kernels of csrc/kq_sample.hip on the context's stream and commits the new
 * RNG state only when the device reports success.
 */
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "kq_hip.h"
#include "kq_hip_internal.h"
#include "kq_launch.h"
#include "kq_status_internal.h"

#define KQ_SAMPLING_CONFIG_MAGIC UINT64_C(0x4b51485341435331) /* "KQHSACS1" */
#define PCG_MULTIPLIER UINT64_C(6364136223846793005)
#define INTEGRITY_OFFSET UINT64_C(1469598103934665603)
#define INTEGRITY_PRIME UINT64_C(1099511628211)
#define MAX_VOCABULARY (UINT32_C(1) << 24)
#define PREP_THREADS 256u

struct kq_hip_sampling_config {
    uint64_t magic;
    kq_hip_sampling_policy policy;
    uint32_t vocabulary_size;
    uint32_t canonical_token_count;
    uint64_t sort_bytes;
    uint64_t scratch_bytes;
};

/* device scratch, carved from a 256-byte aligned start */
typedef struct scratch_layout {
    kq_launch_sample_out *out;
    float *scores;
    uint32_t *keys, *ids, *sorted_keys, *sorted_ids;
    float *probs;
    uint32_t *bad, *bmax;
    void *sort_temp;
} scratch_layout;

static uint64_t round256(uint64_t n) { return (n + 255u) & ~(uint64_t)255u; }

static uint64_t layout_bytes(uint32_t v, uint64_t sort_bytes) {
    const uint64_t arr = round256((uint64_t)v * 4u);
    const uint64_t bad = round256((((uint64_t)v + PREP_THREADS - 1u) / PREP_THREADS) * 4u);
    return 256u + 6u * arr + 2u * bad + round256(sort_bytes);
}

static void carve(const kq_hip_sampling_config *cfg, void *scratch, scratch_layout *l) {
    const uint64_t arr = round256((uint64_t)cfg->vocabulary_size * 4u);
    const uint64_t bad =
        round256((((uint64_t)cfg->vocabulary_size + PREP_THREADS - 1u) / PREP_THREADS) * 4u);
    unsigned char *p = (unsigned char *)(((uintptr_t)scratch + 255u) & ~(uintptr_t)255u);
    l->out = (kq_launch_sample_out *)p;
    p += 256u;
    l->scores = (float *)p;
    p += arr;
    l->keys = (uint32_t *)p;
    p += arr;
    l->ids = (uint32_t *)p;
    p += arr;
    l->sorted_keys = (uint32_t *)p;
    p += arr;
    l->sorted_ids = (uint32_t *)p;
    p += arr;
    l->probs = (float *)p;
    p += arr;
    l->bad = (uint32_t *)p;
    p += bad;
    l->bmax = (uint32_t *)p;
    p += bad;
    l->sort_temp = p;
}

static int overlap(const void *a, uint64_t an, const void *b, uint64_t bn) {
    uintptr_t a0 = (uintptr_t)a, b0 = (uintptr_t)b;
    if (a == NULL || b == NULL || an == 0u || bn == 0u) return 0;
    if (a0 > UINTPTR_MAX - an || b0 > UINTPTR_MAX - bn) return 1;
    return a0 < b0 + bn && b0 < a0 + an;
}

static int is_finite(float v) {
    uint32_t u;
    memcpy(&u, &v, sizeof u);
    return (u & 0x7f800000u) != 0x7f800000u;
}

/* ------------------------------------------------------------------ */
/* RNG (src/kq_sampling.c:83-159) */

static uint64_t mix(uint64_t h, uint64_t v) {
    h ^= v;
    return h * INTEGRITY_PRIME;
}

static uint64_t integrity(const kq_hip_sampling_rng_state *s) {
    uint64_t h = INTEGRITY_OFFSET;
    h = mix(h, s->version);
    h = mix(h, s->reserved);
    h = mix(h, s->seed);
    h = mix(h, s->stream);
    h = mix(h, s->state);
    h = mix(h, s->increment);
    return mix(h, s->draws);
}

static int rng_valid(const kq_hip_sampling_rng_state *s) {
    return s != NULL && s->version == KQ_HIP_SAMPLING_RNG_STATE_VERSION && s->reserved == 0u &&
           s->stream <= KQ_HIP_SAMPLING_MAX_STREAM &&
           s->increment == ((s->stream << 1u) | 1u) && s->integrity == integrity(s);
}

static uint32_t pcg_step(uint64_t *state, uint64_t inc) {
    const uint64_t old = *state;
    const uint32_t xs = (uint32_t)(((old >> 18u) ^ old) >> 27u);
    const uint32_t rot = (uint32_t)(old >> 59u);
    *state = old * PCG_MULTIPLIER + inc;
    return (xs >> rot) | (xs << ((0u - rot) & 31u));
}

static void rng_seed_value(uint64_t seed, uint64_t stream, kq_hip_sampling_rng_state *o) {
    uint64_t st = 0u;
    const uint64_t inc = (stream << 1u) | 1u;
    (void)pcg_step(&st, inc);
    st += seed;
    (void)pcg_step(&st, inc);
    o->version = KQ_HIP_SAMPLING_RNG_STATE_VERSION;
    o->reserved = 0u;
    o->seed = seed;
    o->stream = stream;
    o->state = st;
    o->increment = inc;
    o->draws = 0u;
    o->integrity = integrity(o);
}

kq_status kq_hip_sampling_rng_seed(uint64_t seed, uint64_t stream,
                                   kq_hip_sampling_rng_state *out, kq_diagnostic *diag) {
    kq_hip_sampling_rng_state local;
    kq_diagnostic_clear(diag);
    if (out == NULL)
        return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT, "sampling RNG output is null");
    if (stream > KQ_HIP_SAMPLING_MAX_STREAM)
        return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT, "sampling RNG stream exceeds 63 bits");
    rng_seed_value(seed, stream, &local);
    *out = local;
    return KQ_STATUS_OK;
}

kq_status kq_hip_sampling_rng_reset(kq_hip_sampling_rng_state *state, kq_diagnostic *diag) {
    kq_hip_sampling_rng_state local;
    kq_diagnostic_clear(diag);
    if (!rng_valid(state))
        return kq_fail(diag, KQ_STATUS_INVALID_RNG_STATE, "sampling RNG reset state is invalid");
    rng_seed_value(state->seed, state->stream, &local);
    *state = local;
    return KQ_STATUS_OK;
}

kq_status kq_hip_sampling_rng_snapshot(const kq_hip_sampling_rng_state *state,
                                       kq_hip_sampling_rng_state *out, kq_diagnostic *diag) {
    kq_hip_sampling_rng_state local;
    kq_diagnostic_clear(diag);
    if (out == NULL)
        return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT, "sampling RNG snapshot output is null");
    if (!rng_valid(state))
        return kq_fail(diag, KQ_STATUS_INVALID_RNG_STATE, "sampling RNG snapshot source is invalid");
    local = *state;
    *out = local;
    return KQ_STATUS_OK;
}

kq_status kq_hip_sampling_rng_import(const kq_hip_sampling_rng_state *snapshot,
                                     kq_hip_sampling_rng_state *out, kq_diagnostic *diag) {
    return kq_hip_sampling_rng_snapshot(snapshot, out, diag);
}

kq_status kq_hip_sampling_rng_next_u32(kq_hip_sampling_rng_state *state, uint32_t *word,
                                       kq_diagnostic *diag) {
    kq_hip_sampling_rng_state local;
    kq_diagnostic_clear(diag);
    if (word == NULL)
        return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT, "sampling RNG word output is null");
    if (!rng_valid(state))
        return kq_fail(diag, KQ_STATUS_INVALID_RNG_STATE, "sampling RNG state is invalid");
    if (state->draws == UINT64_MAX)
        return kq_fail(diag, KQ_STATUS_ARITHMETIC_OVERFLOW, "sampling RNG draw count overflowed");
    local = *state;
    *word = pcg_step(&local.state, local.increment);
    local.draws += 1u;
    local.integrity = integrity(&local);
    *state = local;
    return KQ_STATUS_OK;
}

/* ------------------------------------------------------------------ */
/* policy and config (src/kq_sampling.c:161-244) */

void kq_hip_sampling_policy_qwen38_default(kq_hip_sampling_policy *policy) {
    if (policy == NULL) return;
    memset(policy, 0, sizeof(*policy));
    policy->version = KQ_HIP_SAMPLING_POLICY_VERSION;
    policy->temperature = 1.0f;
    policy->top_p = 0.95f;
    policy->top_k = 20u;
}

kq_status kq_hip_sampling_config_open(const kq_hip_sampling_policy *policy, uint32_t vocab,
                                      uint32_t canonical, kq_hip_sampling_config **out,
                                      kq_diagnostic *diag) {
    kq_hip_sampling_config *cfg;
    size_t sort_bytes = 0;
    int e;
    kq_diagnostic_clear(diag);
    if (out == NULL)
        return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT, "sampling config output is null");
    if (policy != NULL && overlap(policy, sizeof(*policy), out, sizeof(*out)))
        return kq_fail(diag, KQ_STATUS_ALIASING_VIOLATION,
                       "sampling policy and config output overlap");
    *out = NULL;
    if (policy == NULL || policy->version != KQ_HIP_SAMPLING_POLICY_VERSION || policy->flags != 0u)
        return kq_fail(diag, KQ_STATUS_INCOMPATIBLE_SAMPLING,
                       "sampling policy version or flags are unsupported");
    for (int i = 0; i < 3; ++i)
        if (policy->reserved[i] != 0u)
            return kq_fail(diag, KQ_STATUS_INCOMPATIBLE_SAMPLING,
                           "sampling policy reserved fields are nonzero");
    if (vocab == 0u || canonical == 0u || canonical > vocab)
        return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT,
                       "vocabulary and canonical token counts must satisfy 1 <= canonical <= "
                       "vocabulary");
    if (vocab > MAX_VOCABULARY)
        return kq_fail(diag, KQ_STATUS_LIMIT_EXCEEDED, "vocabulary exceeds 2^24 ids");
    if (!is_finite(policy->temperature) || policy->temperature <= 0.0f ||
        !is_finite(policy->top_p) || policy->top_p < 0.0f || policy->top_p > 1.0f ||
        policy->top_k > vocab)
        return kq_fail(diag, KQ_STATUS_INCOMPATIBLE_SAMPLING,
                       "sampling temperature, top-k, or top-p is invalid");
    e = (int)kq_launch_sample_sort_bytes(vocab, &sort_bytes);
    if (e != 0) return kqi_hip_fail(diag, e, "sampling sort work-size query");
    cfg = (kq_hip_sampling_config *)calloc(1u, sizeof(*cfg));
    if (cfg == NULL)
        return kq_fail(diag, KQ_STATUS_OUT_OF_MEMORY, "sampling config allocation failed");
    cfg->magic = KQ_SAMPLING_CONFIG_MAGIC;
    cfg->policy = *policy;
    cfg->vocabulary_size = vocab;
    cfg->canonical_token_count = canonical;
    cfg->sort_bytes = (uint64_t)sort_bytes;
    cfg->scratch_bytes = 255u + layout_bytes(vocab, cfg->sort_bytes);
    *out = cfg;
    return KQ_STATUS_OK;
}

kq_status kq_hip_sampling_config_open_qwen38(const kq_hip_sampling_policy *policy,
                                             kq_hip_sampling_config **out,
                                             kq_diagnostic *diag) {
    return kq_hip_sampling_config_open(policy, KQ_HIP_SAMPLING_QWEN38_VOCAB_SIZE,
                                       KQ_HIP_SAMPLING_QWEN38_CANONICAL_TOKEN_COUNT, out, diag);
}

static int config_valid(const kq_hip_sampling_config *c) {
    return c != NULL && c->magic == KQ_SAMPLING_CONFIG_MAGIC && c->vocabulary_size != 0u;
}

void kq_hip_sampling_config_close(kq_hip_sampling_config *c) {
    if (c == NULL) return;
    if (c->magic == KQ_SAMPLING_CONFIG_MAGIC) c->magic = 0u;
    free(c);
}

uint64_t kq_hip_sampling_config_owned_bytes(const kq_hip_sampling_config *c) {
    return config_valid(c) ? (uint64_t)sizeof(*c) : 0u;
}

uint32_t kq_hip_sampling_config_vocabulary_size(const kq_hip_sampling_config *c) {
    return config_valid(c) ? c->vocabulary_size : 0u;
}

uint64_t kq_hip_sampling_required_scratch_bytes(const kq_hip_sampling_config *c) {
    return config_valid(c) ? c->scratch_bytes : 0u;
}

/* ------------------------------------------------------------------ */
/* selection (src/kq_sampling.c:576-772) */

/* checks before any device work, in the reference's order */
static kq_status select_checks(kq_hip_context *ctx, const kq_hip_sampling_config *cfg,
                               const kq_hip_sampling_rng_state *state, const float *logits,
                               uint64_t count, const void *scratch, uint64_t scratch_bytes,
                               const kq_hip_sampling_result *result, kq_diagnostic *diag) {
    uint64_t lb;
    if (!config_valid(cfg))
        return kq_fail(diag, KQ_STATUS_INCOMPATIBLE_SAMPLING, "sampling config is invalid");
    if (state == NULL || logits == NULL || result == NULL || count != cfg->vocabulary_size)
        return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT,
                       "sampling input or target vocabulary count is invalid");
    if (!rng_valid(state))
        return kq_fail(diag, KQ_STATUS_INVALID_RNG_STATE, "sampling RNG state is invalid");
    lb = count * 4u;
    if (overlap(logits, lb, scratch, scratch_bytes) ||
        overlap(state, sizeof(*state), scratch, scratch_bytes) ||
        overlap(result, sizeof(*result), scratch, scratch_bytes) ||
        overlap(logits, lb, state, sizeof(*state)) ||
        overlap(logits, lb, result, sizeof(*result)) ||
        overlap(state, sizeof(*state), result, sizeof(*result)) ||
        overlap(cfg, sizeof(*cfg), logits, lb) ||
        overlap(cfg, sizeof(*cfg), scratch, scratch_bytes) ||
        overlap(cfg, sizeof(*cfg), state, sizeof(*state)) ||
        overlap(cfg, sizeof(*cfg), result, sizeof(*result)))
        return kq_fail(diag, KQ_STATUS_ALIASING_VIOLATION, "sampling buffers overlap");
    if (scratch == NULL || scratch_bytes < cfg->scratch_bytes)
        return kq_fail(diag, KQ_STATUS_BUFFER_TOO_SMALL, "sampling scratch buffer is too small");
    if (((uintptr_t)logits & 3u) != 0u)
        return kq_fail(diag, KQ_STATUS_INVALID_ALIGNMENT, "logits must be 4-byte aligned");
    return kqi_context_begin(ctx, diag);
}

/* enqueue the sampler on the context's stream (logits already enqueued
 * before it when fused), wait, and translate the device record */
static kq_status run_select(kq_hip_context *ctx, const kq_hip_sampling_config *cfg,
                            kq_hip_sampling_rng_state *state, const float *logits,
                            void *scratch, kq_hip_sampling_result *result,
                            kq_diagnostic *diag) {
    kq_hip_sampling_rng_state next = *state;
    kq_launch_sample_out rec;
    kq_launch_sample_args a;
    scratch_layout l;
    uint32_t word = 0u;
    const int overflow = state->draws == UINT64_MAX;
    kq_status st;
    int e;
    if (!overflow) {
        word = pcg_step(&next.state, next.increment);
        next.draws += 1u;
        next.integrity = integrity(&next);
    }
    carve(cfg, scratch, &l);
    memset(&a, 0, sizeof(a));
    a.logits = logits;
    a.count = cfg->vocabulary_size;
    a.canonical = cfg->canonical_token_count;
    a.top_k = cfg->policy.top_k;
    a.temperature = cfg->policy.temperature;
    a.top_p = cfg->policy.top_p;
    a.word = word;
    a.scores = l.scores;
    a.keys = l.keys;
    a.ids = l.ids;
    a.sorted_keys = l.sorted_keys;
    a.sorted_ids = l.sorted_ids;
    a.probs = l.probs;
    a.bad_per_block = l.bad;
    a.max_per_block = l.bmax;
    a.sort_temp = l.sort_temp;
    a.sort_bytes = (size_t)cfg->sort_bytes;
    a.out = l.out;
    /* KQ_HIP_SAMPLE_SEQUENTIAL=1: every draw over many kept ids takes the
     * sequential binary64 walk rather than the parallel prefix sums that
     * are certified to select the same id (a diagnostic: the tests run the
     * two and compare them with the oracle) */
    {
        const char *seq = getenv("KQ_HIP_SAMPLE_SEQUENTIAL");
        a.sequential_draw = seq != NULL && seq[0] == '1' ? 1u : 0u;
    }
    e = (int)kq_launch_sample(&a, (hipStream_t)kqi_context_stream_ptr(ctx));
    if (e == 0)
        e = (int)hipMemcpyAsync(&rec, l.out, sizeof(rec), hipMemcpyDeviceToHost,
                                (hipStream_t)kqi_context_stream_ptr(ctx));
    if (e != 0) {
        (void)kqi_context_drain(ctx, NULL);
        return kqi_hip_fail(diag, e, "sampler launch");
    }
    st = kqi_context_drain(ctx, diag); /* the LM head's flags, when fused */
    if (st != KQ_STATUS_OK) return st;
    if (rec.status == KQ_SAMPLE_FULL_SORT) {
        /* the fast path's top did not fit (ties): sort everything */
        e = (int)kq_launch_sample_full(&a, (hipStream_t)kqi_context_stream_ptr(ctx));
        if (e == 0)
            e = (int)hipMemcpyAsync(&rec, l.out, sizeof(rec), hipMemcpyDeviceToHost,
                                    (hipStream_t)kqi_context_stream_ptr(ctx));
        if (e != 0) {
            (void)kqi_context_drain(ctx, NULL);
            return kqi_hip_fail(diag, e, "sampler launch");
        }
        st = kqi_context_drain(ctx, diag);
        if (st != KQ_STATUS_OK) return st;
    }
    switch (rec.status) {
    case KQ_SAMPLE_OK:
    case KQ_SAMPLE_INVALID_TOKEN:
        break;
    case KQ_SAMPLE_NUMERIC_BEFORE_DRAW:
        return kq_fail(diag, KQ_STATUS_NUMERIC_DOMAIN,
                       "sampling logits, scores or softmax mass are not finite and positive");
    case KQ_SAMPLE_NUMERIC_IN_DRAW:
        if (overflow) break;
        return kq_fail(diag, KQ_STATUS_NUMERIC_DOMAIN, "categorical threshold is outside mass");
    default:
        return kq_fail(diag, KQ_STATUS_DEVICE_FAILURE, "sampler returned status %u", rec.status);
    }
    if (overflow)
        return kq_fail(diag, KQ_STATUS_ARITHMETIC_OVERFLOW, "sampling RNG draw count overflowed");
    if (rec.status == KQ_SAMPLE_INVALID_TOKEN)
        return kq_fail(diag, KQ_STATUS_INVALID_TOKEN_ID, "sampled model-capacity padding token ID");
    memset(result, 0, sizeof(*result));
    result->selected_token_id = rec.selected;
    result->top_k_retained_count = rec.top_k_retained;
    result->retained_count = rec.retained;
    result->rng_word = word;
    result->selected_probability = rec.selected_probability;
    result->maximum_probability = rec.maximum_probability;
    result->normalized_sum_f32 = rec.normalized_sum;
    result->uniform_value = rec.uniform;
    result->rng_draws_before = state->draws;
    result->rng_draws_after = next.draws;
    *state = next;
    return KQ_STATUS_OK;
}

kq_status kq_hip_sampling_select_f32(kq_hip_context *ctx, const kq_hip_sampling_config *cfg,
                                     kq_hip_sampling_rng_state *state, const float *logits,
                                     uint64_t count, void *scratch, uint64_t scratch_bytes,
                                     kq_hip_sampling_result *result, kq_diagnostic *diag) {
    kq_status st;
    kq_diagnostic_clear(diag);
    st = select_checks(ctx, cfg, state, logits, count, scratch, scratch_bytes, result, diag);
    if (st != KQ_STATUS_OK) return st;
    return run_select(ctx, cfg, state, logits, scratch, result, diag);
}

kq_status kq_hip_lm_head_sample_f32(kq_hip_context *ctx, const kq_hip_sampling_config *cfg,
                                    kq_hip_sampling_rng_state *state, uint32_t type_id,
                                    const void *w, uint64_t vocab, uint64_t cols,
                                    const float *h, float *logits, void *scratch,
                                    uint64_t scratch_bytes, kq_hip_sampling_result *result,
                                    kq_diagnostic *diag) {
    kq_status st;
    kq_diagnostic_clear(diag);
    st = select_checks(ctx, cfg, state, logits, vocab, scratch, scratch_bytes, result, diag);
    if (st != KQ_STATUS_OK) return st;
    if (w == NULL || h == NULL)
        return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT, "LM-head weights and hidden are required");
    if (overlap(h, cols * 4u, scratch, scratch_bytes))
        return kq_fail(diag, KQ_STATUS_ALIASING_VIOLATION, "hidden state overlaps the scratch");
    st = kqi_enqueue_logits(ctx, type_id, w, vocab, cols, h, logits, diag);
    if (st != KQ_STATUS_OK) return st;
    return run_select(ctx, cfg, state, logits, scratch, result, diag);
}

kq_status kq_hip_sampling_copy_work(kq_hip_context *ctx, const kq_hip_sampling_config *cfg,
                                    const void *scratch, uint64_t scratch_bytes, float *scores,
                                    float *probs, uint64_t capacity, kq_diagnostic *diag) {
    scratch_layout l;
    uint64_t bytes;
    kq_status st;
    int e;
    kq_diagnostic_clear(diag);
    if (!config_valid(cfg) || scratch == NULL || scores == NULL || probs == NULL ||
        capacity < cfg->vocabulary_size)
        return kq_fail(diag, KQ_STATUS_INVALID_ARGUMENT, "sampling work request is invalid");
    bytes = (uint64_t)cfg->vocabulary_size * 4u;
    if (overlap(scores, bytes, probs, bytes) || overlap(scores, bytes, scratch, scratch_bytes) ||
        overlap(probs, bytes, scratch, scratch_bytes))
        return kq_fail(diag, KQ_STATUS_ALIASING_VIOLATION, "sampling work buffers overlap");
    if (scratch_bytes < cfg->scratch_bytes)
        return kq_fail(diag, KQ_STATUS_BUFFER_TOO_SMALL, "sampling scratch buffer is too small");
    st = kqi_context_begin(ctx, diag);
    if (st != KQ_STATUS_OK) return st;
    carve(cfg, (void *)scratch, &l);
    e = (int)hipMemcpyAsync(scores, l.scores, (size_t)bytes, hipMemcpyDeviceToHost,
                            (hipStream_t)kqi_context_stream_ptr(ctx));
    if (e == 0)
        e = (int)hipMemcpyAsync(probs, l.probs, (size_t)bytes, hipMemcpyDeviceToHost,
                                (hipStream_t)kqi_context_stream_ptr(ctx));
    if (e != 0) {
        (void)kqi_context_drain(ctx, NULL);
        return kqi_hip_fail(diag, e, "sampling work copy");
    }
    return kqi_context_drain(ctx, diag);
}
