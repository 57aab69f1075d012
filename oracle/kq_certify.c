/*
 * kq_certify.c — CPU restatement of the device's certified one-token
 * routing, and a campaign that checks it against the oracle's exact route.
 *
 * TEST INFRASTRUCTURE ONLY (the checker). Never linked into libkq_hip.so.
 *
 * The device (kestrel-q_amd/csrc/kq_moe.hip: router_bounds, route_certify)
 * skips the reference's 2048-step binary32 chains for one token when it can
 * prove which experts the chains would select:
 *   - a_e = S_n, the binary64 sum of the rounded products fl(w_i * x_i) of
 *     row e, and b_e = 1.001 * 2^-24 * sum_i |S_i| over its prefix sums
 *     S_i, bound |l_e - a_e| for the CPU's left-to-right binary32 sum l_e
 *     (src/kq_numeric.c:474-496 via kq_f32_dot; infinite when a product is
 *     not finite or the prefix sums approach the binary32 range);
 *   - the top k by a (larger first, lower id among equals) is certified if
 *     each adjacent pair of it, and its last member against the largest
 *     a + b outside it, are separated by more than both bounds plus
 *     2^-20 * (4 + |hi - max a| + |lo - max a|), and the higher member of
 *     each pair has hi - b - max a > -75 (its probability a normal binary32
 *     number: two probabilities that underflow tie, and the CPU orders
 *     ties by id). Then the CPU's softmax
 *     probabilities are strictly ordered the same way, and its partial
 *     selection (src/kq_moe_qwen38.c:211-274) returns exactly these ids in
 *     this order.
 * kqo_route_certify restates that decision step by step, including how the
 * device gathers its candidates (waves of 64 experts, each wave's per-th
 * largest key, at most 128 candidates) so the cases it certifies are the
 * device's. kqo_certify_campaign generates routers and activations from a
 * SplitMix64 stream, optionally plants near ties at gaps around the bound,
 * and counts certified selections whose ids differ from the oracle's exact
 * route: the soundness claim is that there are none.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "kq_oracle.h"

#ifdef _OPENMP
#include <omp.h>
#endif

/* router_bounds: a = S_n, b = 1.001 u sum |S_i| (infinite when unsafe). */
static void row_bound(const float *w, const float *x, uint32_t n, double *a, double *b) {
    double s = 0.0, sab = 0.0;
    int bad = 0;
    for (uint32_t i = 0; i < n; ++i) {
        const float p = w[i] * x[i];
        if (!isfinite(p)) bad = 1;
        s += (double)p;
        sab += fabs(s);
    }
    *a = s;
    *b = bad || !(sab < 0x1p126) ? INFINITY : 1.001 * 0x1p-24 * sab;
}

/* slack < 0: |slack| as below, without the normal-probability rule (a
 * planted unsound certification for scaled activations) */
static int certify_sep(double hi, double bhi, double lo, double blo, double m, double slack) {
    const double margin = fabs(slack) * 0x1p-20 * (4.0 + fabs(hi - m) + fabs(lo - m));
    return (slack < 0.0 || (hi - bhi) - m > -75.0) && (hi - bhi) - (lo + blo) > margin;
}

typedef struct cand {
    double a, b;
    uint32_t id;
} cand;

/* (larger a first, lower id among equals) */
static int cand_before(const cand *p, const cand *q) {
    return p->a > q->a || (p->a == q->a && p->id < q->id);
}

/* route_certify. a[], b[] per expert; writes ids[k] and returns 1 when
 * certified, 0 otherwise. At most 1024 experts, k <= 64. slack scales the
 * margin (1 as on the device). */
static int certify(const double *ar, const double *b, uint32_t E, uint32_t k, uint32_t *ids,
                   double slack) {
    enum { kCand = 128 };
    double a[1024];
    float key[1024];
    cand list[kCand];
    uint32_t total = 0;
    double rest = -INFINITY;
    if (E == 0 || E > 1024 || k == 0 || k > E || k > kCand) return 0;
    for (uint32_t e = 0; e < E; ++e) {
        a[e] = ar[e] == ar[e] ? ar[e] : -INFINITY;
        key[e] = (float)a[e];
        if (!(b[e] < INFINITY)) return 0;
    }
    /* 1-2. per-th largest key of each full wave; t = their least */
    const uint32_t need = k + 1 < E ? k + 1 : E;
    const uint32_t ns = E >= 64 ? E / 64 : 1;
    const uint32_t per = (need + ns - 1) / ns;
    float t = INFINITY;
    for (uint32_t w = 0; w < ns; ++w) {
        float v[64];
        uint32_t lanes = 0;
        for (uint32_t l = 0; l < 64; ++l) {
            const uint32_t e = 64 * w + l;
            v[l] = e < E ? key[e] : -INFINITY;
            if (e < E) lanes = l + 1;
        }
        (void)lanes;
        float m = INFINITY;
        for (uint32_t r = 0; r < per; ++r) {
            /* the largest remaining key; the lowest lane holding it drops out */
            uint32_t at = 0;
            m = v[0];
            for (uint32_t l = 1; l < 64; ++l)
                if (v[l] > m) { m = v[l]; at = l; }
            v[at] = -INFINITY;
        }
        if (m < t) t = m;
    }
    /* 3. candidates: key >= t; the rest keep their largest a + b */
    for (uint32_t e = 0; e < E; ++e) {
        if (key[e] >= t) {
            if (total < kCand) list[total] = (cand){a[e], b[e], e};
            ++total;
        } else if (a[e] + b[e] > rest) {
            rest = a[e] + b[e];
        }
    }
    if (total > kCand) return 0;
    /* 4. rank the candidates */
    for (uint32_t i = 1; i < total; ++i) {
        cand c = list[i];
        uint32_t j = i;
        while (j > 0 && cand_before(&c, &list[j - 1])) {
            list[j] = list[j - 1];
            --j;
        }
        list[j] = c;
    }
    for (uint32_t r = k; r < total; ++r)
        if (list[r].a + list[r].b > rest) rest = list[r].a + list[r].b;
    /* 5. adjacent selected pairs, then the last selected against the rest */
    const double m = list[0].a;
    for (uint32_t r = 0; r + 1 < k; ++r)
        if (!certify_sep(list[r].a, list[r].b, list[r + 1].a, list[r + 1].b, m, slack))
            return 0;
    if (rest > -INFINITY && !certify_sep(list[k - 1].a, list[k - 1].b, rest, 0.0, m, slack))
        return 0;
    for (uint32_t r = 0; r < k; ++r) ids[r] = list[r].id;
    return 1;
}

int kqo_route_certify(uint32_t experts, uint32_t hidden, uint32_t top_k, const float *router,
                      const float *x, uint32_t *ids, int *certified) {
    double *a, *b;
    if (router == NULL || x == NULL || ids == NULL || certified == NULL || experts == 0 ||
        experts > 1024 || hidden == 0 || top_k == 0 || top_k > experts || top_k > 64)
        return KQO_INVALID_ARGUMENT;
    a = (double *)malloc(2 * sizeof(double) * experts);
    if (a == NULL) return KQO_INVALID_ARGUMENT;
    b = a + experts;
    for (uint32_t e = 0; e < experts; ++e)
        row_bound(router + (uint64_t)e * hidden, x, hidden, &a[e], &b[e]);
    *certified = certify(a, b, experts, top_k, ids, 1.0);
    free(a);
    return KQO_OK;
}

/* ------------------------------------------------------------------ */
/* campaign */

static uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

typedef struct rng {
    uint64_t s;
} rng;

static uint64_t next64(rng *r) {
    r->s += 0x9E3779B97F4A7C15ULL;
    return mix64(r->s);
}

static double unif(rng *r) { return ((next64(r) >> 11) + 0.5) * 0x1p-53; }

static float normal(rng *r, float sigma) {
    const double u1 = unif(r), u2 = unif(r);
    return (float)(sigma * sqrt(-2.0 * log(u1)) * cos(6.283185307179586 * u2));
}

/*
 * Plants a near tie: expert `lo` becomes expert `hi`'s row plus a small
 * independent perturbation (so the two chains round differently), then one
 * column moves its binary64 logit to a_hi - gap.
 */
static void plant_tie(float *router, const float *x, uint32_t H, uint32_t hi, uint32_t lo,
                      double gap, rng *r) {
    float *wl = router + (uint64_t)lo * H;
    const float *wh = router + (uint64_t)hi * H;
    uint32_t col = 0;
    double ah = 0.0, al = 0.0;
    for (uint32_t i = 0; i < H; ++i) {
        wl[i] = wh[i] * (1.0f + 1e-3f * normal(r, 1.0f));
        if (fabsf(x[i]) > fabsf(x[col])) col = i;
    }
    for (uint32_t i = 0; i < H; ++i) {
        ah += (double)wh[i] * (double)x[i];
        al += (double)wl[i] * (double)x[i];
    }
    wl[col] = (float)((double)wl[col] + (ah - gap - al) / (double)x[col]);
}

/*
 * stats[0] trials, [1] certified, [2] certified with ids different from the
 * oracle's exact route (must stay 0), [3] trials whose exact ids differ from
 * the top k of the binary64 sums (rounding decided the selection: these
 * must not certify), [4] index of the first certified mismatch + 1 (0 when
 * none), [5] exact-route failures (non-finite values; none expected).
 *
 * mode 0: router ~N(0, sigma), x ~N(0, 1), a new x every trial and a new
 *         router every 64 trials;
 * mode 1: as 0, plus a near tie between the k-th and (k+1)-th experts by
 *         binary64 logit, gap = c * (b_k + b_k+1) with c log-uniform in
 *         [2^-6, 2^6];
 * mode 2: as 1 for a pair inside the selection (positions j, j+1 < k);
 * mode 3: as 1 with c log-uniform in [2^-16, 2^-2]: ties far below the
 *         bound, where the chains' rounding decides;
 * mode 4: as 0 with x scaled by 2^s, s uniform in [0, 28]: logits so far
 *         apart that the lower selected probabilities underflow and tie.
 * slack multiplies every bound and the margin: 1 restates the device; a
 * smaller value plants an unsound certification, which the campaign must
 * catch (certified selections that differ from the exact route); a
 * negative one also drops the rule that a pair's higher probability be a
 * normal number.
 */
int kqo_certify_campaign(uint64_t seed, uint64_t trials, uint32_t E, uint32_t H, uint32_t K,
                         int mode, float sigma, double slack, int threads,
                         uint64_t *stats) {
    if (stats == NULL || E == 0 || E > 1024 || H == 0 || K == 0 || K >= E || K > 64 || mode < 0 ||
        mode > 4)
        return KQO_INVALID_ARGUMENT;
    memset(stats, 0, 6 * sizeof(uint64_t));
    const uint64_t per_router = 64;
    const int64_t groups = (int64_t)((trials + per_router - 1) / per_router);
    uint64_t first_bad = UINT64_MAX;
    uint64_t t_cert = 0, t_bad = 0, t_flip = 0, t_fail = 0;
#ifdef _OPENMP
#pragma omp parallel for schedule(dynamic, 1) num_threads(threads > 0 ? threads : 1) \
    reduction(+ : t_cert, t_bad, t_flip, t_fail) reduction(min : first_bad)
#endif
    for (int64_t g = 0; g < groups; ++g) {
        rng r = {mix64(seed ^ (0x9E3779B97F4A7C15ULL * (uint64_t)(g + 1)))};
        float *router = (float *)malloc(sizeof(float) * ((uint64_t)E * H + 3u * H));
        float *x = router + (uint64_t)E * H;
        float *saved = x + H;
        double *a = (double *)malloc(sizeof(double) * 2u * E);
        double *b = a + E;
        float *logits = (float *)malloc(sizeof(float) * 2u * E + sizeof(float) * K);
        float *probs = logits + E;
        float *wts = probs + E;
        uint32_t *ids = (uint32_t *)malloc(sizeof(uint32_t) * (3u * K + E));
        uint32_t *cids = ids + K;
        uint32_t *top = cids + K;
        uint32_t *ord = top + K;
        for (uint64_t i = 0; i < (uint64_t)E * H; ++i) router[i] = normal(&r, sigma);
        for (uint64_t tt = 0; tt < per_router; ++tt) {
            const uint64_t trial = (uint64_t)g * per_router + tt;
            if (trial >= trials) break;
            for (uint32_t i = 0; i < H; ++i) x[i] = normal(&r, 1.0f);
            if (mode == 4) {
                const float sc = ldexpf(1.0f, (int)(next64(&r) % 29u));
                for (uint32_t i = 0; i < H; ++i) x[i] *= sc;
            }
            uint32_t planted = UINT32_MAX;
            if (mode != 0 && mode != 4) {
                /* rank by binary64 logit, then plant the tie */
                for (uint32_t e = 0; e < E; ++e) row_bound(router + (uint64_t)e * H, x, H, &a[e], &b[e]);
                for (uint32_t e = 0; e < E; ++e) ord[e] = e;
                for (uint32_t i = 1; i < E; ++i) {
                    uint32_t v = ord[i], j = i;
                    while (j > 0 && (a[ord[j - 1]] < a[v] || (a[ord[j - 1]] == a[v] && ord[j - 1] > v))) {
                        ord[j] = ord[j - 1];
                        --j;
                    }
                    ord[j] = v;
                }
                uint32_t pos = K - 1;
                if (mode == 2 && K >= 2) pos = (uint32_t)(next64(&r) % (K - 1));
                const uint32_t hi = ord[pos], lo = ord[pos + 1];
                const double lc = mode == 3 ? -16.0 + 14.0 * unif(&r) : -6.0 + 12.0 * unif(&r);
                const double gap = exp2(lc) * (b[hi] + b[lo]);
                memcpy(saved, router + (uint64_t)lo * H, sizeof(float) * H);
                plant_tie(router, x, H, hi, lo, gap, &r);
                planted = lo;
            }
            /* the exact route and the certification */
            kqo_moe_dims d = {H, E, K, 1, 1};
            kqo_tensor rt = {KQO_F32, router};
            if (kqo_moe_route_f32(&d, &rt, x, logits, probs, ids, wts, 1) != KQO_OK) {
                ++t_fail;
            } else {
                /* the top k of the binary64 sums, and the certification */
                for (uint32_t e = 0; e < E; ++e) {
                    row_bound(router + (uint64_t)e * H, x, H, &a[e], &b[e]);
                    b[e] *= slack;
                }
                const int cert = certify(a, b, E, K, cids, slack);
                for (uint32_t j = 0; j < K; ++j) {
                    uint32_t best = UINT32_MAX;
                    for (uint32_t e = 0; e < E; ++e) {
                        int used = 0;
                        for (uint32_t q = 0; q < j; ++q) used |= top[q] == e;
                        if (used) continue;
                        if (best == UINT32_MAX || a[e] > a[best]) best = e;
                    }
                    top[j] = best;
                }
                int flip = memcmp(top, ids, sizeof(uint32_t) * K) != 0;
                t_flip += (uint64_t)flip;
                if (cert) {
                    ++t_cert;
                    if (memcmp(cids, ids, sizeof(uint32_t) * K) != 0) {
                        ++t_bad;
                        if (trial < first_bad) first_bad = trial;
                    }
                }
            }
            if (planted != UINT32_MAX)
                memcpy(router + (uint64_t)planted * H, saved, sizeof(float) * H);
        }
        free(router);
        free(a);
        free(logits);
        free(ids);
    }
    stats[0] = trials;
    stats[1] = t_cert;
    stats[2] = t_bad;
    stats[3] = t_flip;
    stats[4] = first_bad == UINT64_MAX ? 0 : first_bad + 1;
    stats[5] = t_fail;
    return KQO_OK;
}
