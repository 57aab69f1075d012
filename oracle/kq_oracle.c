/*
 * kq_oracle.c — CPU restatement of the Kestrel-Q quantized-weight path.
 *
 * TEST INFRASTRUCTURE ONLY (the checker). Never linked into libkq_hip.so.
 * Compile flags follow CMakeLists.txt:104-117 of the reference:
 *   -std=c17 -O2 -fno-fast-math -ffp-contract=off   (no intrinsics)
 *
 * What pins each part (tests/test_oracle_*.py):
 *   kqo_f16_to_f32      exhaustive over all 65536 patterns vs an independent
 *                       conversion (numpy float16) + EXACT_BITS golden cases
 *   Q8_0 / Q4_K decode  research/numerics/.../dequant-vectors.json (EXACT_BITS,
 *                       llama.cpp 90c26fcd) — also F32/BF16/Q5_1/Q5_K/IQ4_NL
 *   Q6_K decode         no reference vector exists (the reference has no
 *                       Q6_K); pinned by closed-form checks: single-bit
 *                       toggles of ql/qh/sc/d, all-zero block, pack->decode
 *                       round trip and an f64 closed form rounded per step
 *   row dot             dequant-vectors.json row_dot_cases (EXACT_BITS) and a
 *                       brute-force sequential sum
 *   primitives          primitive-calibration/holdout.json (ULP contracts)
 *   kqo_expf            bit-equal to glibc 2.35 expf on all 2^32 inputs
 *   top-k / route       moe-routing-vectors.json (512 experts, top-10,
 *                       EXACT_DISCRETE) and primitive topk cases
 *   MoE execute         moe-calibration/holdout.json (Tier A, per-checkpoint
 *                       calibrated contracts from moe-native-validation.json)
 *   argmax              brute force (first maximum, strict >)
 *   permutation         brute force (definition of a stable counting sort)
 */
#include "kq_oracle.h"

#include <math.h>
#include <stddef.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

static const int8_t kqo_iq4_nl_values[16] = {
    -127, -104, -83, -65, -49, -35, -22, -10,
    1, 13, 25, 38, 53, 69, 89, 113};

int kqo_geometry(uint32_t type_id, uint32_t *block_elements,
                 uint32_t *bytes_per_block) {
    /* src/kq_gguf.c:57-65 type table, plus Q6_K (256, 210) from GGML. */
    uint32_t e = 0U, b = 0U;
    switch (type_id) {
    case KQO_F32: e = 1U; b = 4U; break;
    case KQO_Q5_1: e = 32U; b = 24U; break;
    case KQO_Q8_0: e = 32U; b = 34U; break;
    case KQO_Q4_K: e = 256U; b = 144U; break;
    case KQO_Q5_K: e = 256U; b = 176U; break;
    case KQO_Q6_K: e = 256U; b = 210U; break;
    case KQO_IQ4_NL: e = 32U; b = 18U; break;
    case KQO_BF16: e = 1U; b = 2U; break;
    default: return KQO_UNSUPPORTED_TENSOR_TYPE;
    }
    if (block_elements) *block_elements = e;
    if (bytes_per_block) *bytes_per_block = b;
    return KQO_OK;
}

static uint16_t rd16(const unsigned char *p) {
    return (uint16_t)((uint16_t)p[0] | ((uint16_t)p[1] << 8U));
}

static uint32_t rd32(const unsigned char *p) {
    return (uint32_t)p[0] | ((uint32_t)p[1] << 8U) |
           ((uint32_t)p[2] << 16U) | ((uint32_t)p[3] << 24U);
}

static float bits_f32(uint32_t u) {
    float f;
    memcpy(&f, &u, sizeof f);
    return f;
}

/* src/kq_numeric.c:58-82: exact binary16 -> binary32 including subnormals
 * (normalised by shifting) and Inf/NaN payloads. */
float kqo_f16_to_f32(uint16_t value) {
    uint32_t sign = ((uint32_t)value & 0x8000U) << 16U;
    uint32_t exponent = ((uint32_t)value >> 10U) & 0x1fU;
    uint32_t fraction = (uint32_t)value & 0x03ffU;
    uint32_t bits;
    if (exponent == 0U) {
        if (fraction == 0U) {
            bits = sign;
        } else {
            uint32_t e = 113U;
            while ((fraction & 0x0400U) == 0U) {
                fraction <<= 1U;
                e -= 1U;
            }
            fraction &= 0x03ffU;
            bits = sign | (e << 23U) | (fraction << 13U);
        }
    } else if (exponent == 31U) {
        bits = sign | 0x7f800000U | (fraction << 13U);
    } else {
        bits = sign | ((exponent + 112U) << 23U) | (fraction << 13U);
    }
    return bits_f32(bits);
}

/*
 * expf as the reference calls it: src/kq_numeric.c:628-638 and :776-813 call
 * libm expf. On this Linux image libm is glibc 2.35, whose x86-64 expf is the
 * ARM optimized-routines method (Szabolcs Nagy): x*32/ln2 = k + r, 2^(k/32)
 * from a 32-entry table, a cubic in r, all in binary64 with fused
 * multiply-adds, one final rounding to binary32. Restated here (and in the
 * device header) so CPU and GPU give identical bits on every host; the CPU
 * test suite checks equality with libm expf over all 2^32 inputs.
 * Table entry i = bits(2^(i/32)) - (i << 47), 2^(i/32) correctly rounded.
 */
static const uint64_t kqo_exp2_table[32] = {
    0x3ff0000000000000ULL, 0x3fefd9b0d3158574ULL, 0x3fefb5586cf9890fULL,
    0x3fef9301d0125b51ULL, 0x3fef72b83c7d517bULL, 0x3fef54873168b9aaULL,
    0x3fef387a6e756238ULL, 0x3fef1e9df51fdee1ULL, 0x3fef06fe0a31b715ULL,
    0x3feef1a7373aa9cbULL, 0x3feedea64c123422ULL, 0x3feece086061892dULL,
    0x3feebfdad5362a27ULL, 0x3feeb42b569d4f82ULL, 0x3feeab07dd485429ULL,
    0x3feea47eb03a5585ULL, 0x3feea09e667f3bcdULL, 0x3fee9f75e8ec5f74ULL,
    0x3feea11473eb0187ULL, 0x3feea589994cce13ULL, 0x3feeace5422aa0dbULL,
    0x3feeb737b0cdc5e5ULL, 0x3feec49182a3f090ULL, 0x3feed503b23e255dULL,
    0x3feee89f995ad3adULL, 0x3feeff76f2fb5e47ULL, 0x3fef199bdd85529cULL,
    0x3fef3720dcef9069ULL, 0x3fef5818dcfba487ULL, 0x3fef7c97337b9b5fULL,
    0x3fefa4afa2a490daULL, 0x3fefd0765b6e4540ULL};

float kqo_expf(float x) {
    uint32_t ux;
    uint64_t ki, t;
    double xd, z, kd, r, s, p, r2, y;
    memcpy(&ux, &x, sizeof ux);
    if (((ux >> 20U) & 0x7ffU) >= 0x42bU) { /* |x| >= 88 (or Inf/NaN) */
        if (ux == 0xff800000U) return 0.0f;
        if (((ux >> 20U) & 0x7ffU) >= 0x7f8U) return x + x;
        if (x > 0x1.62e42ep6f) return HUGE_VALF;
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    xd = (double)x;
    z = 0x1.71547652b82fep+0 * 32.0 * xd;
    kd = z + 0x1.8p+52;
    memcpy(&ki, &kd, sizeof ki);
    kd -= 0x1.8p+52;
    r = fma(0x1.71547652b82fep+0 * 32.0, xd, -kd);
    t = kqo_exp2_table[ki % 32U] + (ki << 47U);
    memcpy(&s, &t, sizeof s);
    p = fma(0x1.c6af84b912394p-5 / 32768.0, r, 0x1.ebfce50fac4f3p-3 / 1024.0);
    r2 = r * r;
    y = fma(0x1.62e42ff0c52d6p-1 / 32.0, r, 1.0);
    y = fma(p, r2, y);
    y = y * s;
    return (float)y;
}

void kqo_f16_to_f32_array(const uint16_t *in, uint64_t n, float *out) {
    uint64_t i;
    for (i = 0U; i < n; ++i) out[i] = kqo_f16_to_f32(in[i]);
}

void kqo_expf_array(const float *in, uint64_t n, float *out, int threads) {
    int64_t i;
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(threads > 0 ? threads : 1) if (threads > 1)
#else
    (void)threads;
#endif
    for (i = 0; i < (int64_t)n; ++i) out[i] = kqo_expf(in[i]);
}

/* Checker for the restatement itself: how many bit patterns in
 * [start, start+count) give a different result from this process's libm expf
 * (NaN results compare equal to NaN). */
uint64_t kqo_expf_libm_mismatches(uint64_t start, uint64_t count,
                                  int threads) {
    uint64_t bad = 0U;
    int64_t i;
#ifdef _OPENMP
#pragma omp parallel for schedule(static, 1 << 16) reduction(+ : bad) num_threads(threads > 0 ? threads : 1)
#else
    (void)threads;
#endif
    for (i = 0; i < (int64_t)count; ++i) {
        uint32_t u = (uint32_t)(start + (uint64_t)i);
        float x, a, b;
        uint32_t ab, bb;
        memcpy(&x, &u, sizeof x);
        a = kqo_expf(x);
        b = expf(x);
        memcpy(&ab, &a, sizeof ab);
        memcpy(&bb, &b, sizeof bb);
        if (ab != bb && !(isnan(a) && isnan(b))) bad += 1U;
    }
    return bad;
}

/* src/kq_numeric.c:161-174 */
static void unpack_k_scale(uint32_t j, const unsigned char *q, uint8_t *sc,
                           uint8_t *mn) {
    if (j < 4U) {
        *sc = (uint8_t)(q[j] & 63U);
        *mn = (uint8_t)(q[j + 4U] & 63U);
    } else {
        *sc = (uint8_t)((q[j + 4U] & 15U) | ((q[j - 4U] >> 6U) << 4U));
        *mn = (uint8_t)((q[j + 4U] >> 4U) | ((q[j] >> 6U) << 4U));
    }
}

/* src/kq_numeric.c:176-295, plus the GGML Q6_K layout. */
static int decode_one_block(uint32_t type_id, const unsigned char *b,
                            float *y) {
    uint32_t i;
    if (type_id == KQO_F32) {
        y[0] = bits_f32(rd32(b));
        return KQO_OK;
    }
    if (type_id == KQO_BF16) {
        y[0] = bits_f32((uint32_t)rd16(b) << 16U);
        return KQO_OK;
    }
    if (type_id == KQO_Q5_1) {
        float d = kqo_f16_to_f32(rd16(b));
        float m = kqo_f16_to_f32(rd16(b + 2U));
        uint32_t high = rd32(b + 4U);
        if (!isfinite(d) || !isfinite(m)) return KQO_MALFORMED_QUANTIZED_DATA;
        for (i = 0U; i < 16U; ++i) {
            uint8_t byte = b[8U + i];
            uint32_t lo = (uint32_t)(byte & 15U) | (((high >> i) & 1U) << 4U);
            uint32_t hi = (uint32_t)(byte >> 4U) |
                          (((high >> (i + 16U)) & 1U) << 4U);
            y[i] = (float)lo * d + m;
            y[i + 16U] = (float)hi * d + m;
        }
        return KQO_OK;
    }
    if (type_id == KQO_Q8_0) {
        float d = kqo_f16_to_f32(rd16(b));
        if (!isfinite(d)) return KQO_MALFORMED_QUANTIZED_DATA;
        for (i = 0U; i < 32U; ++i) y[i] = (float)(int8_t)b[2U + i] * d;
        return KQO_OK;
    }
    if (type_id == KQO_Q4_K || type_id == KQO_Q5_K) {
        float d = kqo_f16_to_f32(rd16(b));
        float dmin = kqo_f16_to_f32(rd16(b + 2U));
        const unsigned char *scales = b + 4U;
        const unsigned char *high = type_id == KQO_Q5_K ? b + 16U : NULL;
        const unsigned char *qs = type_id == KQO_Q5_K ? b + 48U : b + 16U;
        uint32_t g;
        if (!isfinite(d) || !isfinite(dmin)) return KQO_MALFORMED_QUANTIZED_DATA;
        for (g = 0U; g < 4U; ++g) {
            uint8_t s0, m0, s1, m1;
            float dl, ml, dh, mh;
            uint8_t mask_lo = (uint8_t)(1U << (2U * g));
            uint8_t mask_hi = (uint8_t)(2U << (2U * g));
            unpack_k_scale(2U * g, scales, &s0, &m0);
            unpack_k_scale(2U * g + 1U, scales, &s1, &m1);
            dl = d * (float)s0;
            ml = dmin * (float)m0;
            dh = d * (float)s1;
            mh = dmin * (float)m1;
            for (i = 0U; i < 32U; ++i) {
                uint8_t byte = qs[g * 32U + i];
                uint32_t lo = (uint32_t)(byte & 15U);
                uint32_t hi = (uint32_t)(byte >> 4U);
                if (high != NULL) {
                    if ((high[i] & mask_lo) != 0U) lo += 16U;
                    if ((high[i] & mask_hi) != 0U) hi += 16U;
                }
                y[g * 64U + i] = dl * (float)lo - ml;
                y[g * 64U + 32U + i] = dh * (float)hi - mh;
            }
        }
        return KQO_OK;
    }
    if (type_id == KQO_Q6_K) {
        /* GGML block_q6_K: ql[128] @0, qh[64] @128, int8 sc[16] @192,
         * f16 d @208. Weight = (d * sc) * (q - 32), q = 4 low bits from ql
         * and 2 high bits from qh. */
        float d = kqo_f16_to_f32(rd16(b + 208U));
        uint32_t n, l;
        if (!isfinite(d)) return KQO_MALFORMED_QUANTIZED_DATA;
        for (n = 0U; n < 2U; ++n) {
            const unsigned char *ql = b + 64U * n;
            const unsigned char *qh = b + 128U + 32U * n;
            const int8_t *sc = (const int8_t *)(b + 192U + 8U * n);
            float *yy = y + 128U * n;
            for (l = 0U; l < 32U; ++l) {
                uint32_t is = l / 16U;
                int q1 = (int)((ql[l] & 15U) | (((qh[l] >> 0U) & 3U) << 4U)) - 32;
                int q2 = (int)((ql[l + 32U] & 15U) | (((qh[l] >> 2U) & 3U) << 4U)) - 32;
                int q3 = (int)((ql[l] >> 4U) | (((qh[l] >> 4U) & 3U) << 4U)) - 32;
                int q4 = (int)((ql[l + 32U] >> 4U) | (((qh[l] >> 6U) & 3U) << 4U)) - 32;
                yy[l] = d * (float)sc[is] * (float)q1;
                yy[l + 32U] = d * (float)sc[is + 2U] * (float)q2;
                yy[l + 64U] = d * (float)sc[is + 4U] * (float)q3;
                yy[l + 96U] = d * (float)sc[is + 6U] * (float)q4;
            }
        }
        return KQO_OK;
    }
    if (type_id == KQO_IQ4_NL) {
        float d = kqo_f16_to_f32(rd16(b));
        if (!isfinite(d)) return KQO_MALFORMED_QUANTIZED_DATA;
        for (i = 0U; i < 16U; ++i) {
            uint8_t byte = b[2U + i];
            y[i] = d * (float)kqo_iq4_nl_values[byte & 15U];
            y[i + 16U] = d * (float)kqo_iq4_nl_values[byte >> 4U];
        }
        return KQO_OK;
    }
    return KQO_UNSUPPORTED_TENSOR_TYPE;
}

/* src/kq_numeric.c:297-359 */
int kqo_dequantize_blocks_f32(uint32_t type_id, const void *packed,
                              uint64_t packed_bytes, float *output,
                              uint64_t output_capacity,
                              uint64_t *output_count) {
    uint32_t be, bb;
    uint64_t blocks, need, k;
    int st;
    if (output_count == NULL || packed == NULL || packed_bytes == 0U)
        return KQO_INVALID_ARGUMENT;
    *output_count = 0U;
    st = kqo_geometry(type_id, &be, &bb);
    if (st != KQO_OK) return st;
    if (packed_bytes % bb != 0U) return KQO_MALFORMED_QUANTIZED_DATA;
    blocks = packed_bytes / bb;
    need = blocks * be;
    *output_count = need;
    if (output == NULL || output_capacity < need) return KQO_BUFFER_TOO_SMALL;
    for (k = 0U; k < blocks; ++k) {
        st = decode_one_block(type_id, (const unsigned char *)packed + k * bb,
                              output + k * be);
        if (st != KQO_OK) return st;
    }
    return KQO_OK;
}

static int finite_vec(const float *x, uint64_t n) {
    uint64_t i;
    for (i = 0U; i < n; ++i)
        if (!isfinite(x[i])) return 0;
    return 1;
}

/* src/kq_numeric.c:420-503: decode one block into a scratch, then a single
 * left-to-right accumulator over the whole row: acc = acc + (w * x). */
int kqo_row_dot_f32(uint32_t type_id, const void *packed,
                    uint64_t packed_bytes, const float *x, uint64_t count,
                    float *output) {
    float scratch[256];
    float acc = 0.0f;
    uint32_t be, bb;
    uint64_t blocks, k, i;
    int st;
    if (packed == NULL || x == NULL || output == NULL || packed_bytes == 0U ||
        count == 0U)
        return KQO_INVALID_ARGUMENT;
    st = kqo_geometry(type_id, &be, &bb);
    if (st != KQO_OK) return st;
    if (packed_bytes % bb != 0U) return KQO_MALFORMED_QUANTIZED_DATA;
    blocks = packed_bytes / bb;
    if (blocks * be != count) return KQO_DIMENSION_MISMATCH;
    if (!finite_vec(x, count)) return KQO_NUMERIC_DOMAIN;
    for (k = 0U; k < blocks; ++k) {
        st = decode_one_block(type_id, (const unsigned char *)packed + k * bb,
                              scratch);
        if (st != KQO_OK) return st;
        for (i = 0U; i < be; ++i) {
            float product = scratch[i] * x[k * be + i];
            acc = acc + product;
        }
    }
    if (!isfinite(acc)) return KQO_NUMERIC_DOMAIN;
    *output = acc;
    return KQO_OK;
}

/* src/kq_weight_provider.c:378-509 (linear_f32): one row-dot per output row
 * over rows of cols/QK blocks; the output is committed only on success. */
int kqo_matvec_f32(uint32_t type_id, const void *w, uint64_t rows,
                   uint64_t cols, const float *x, uint32_t batch, float *y,
                   int threads) {
    uint32_t be, bb;
    uint64_t row_bytes;
    int st = kqo_geometry(type_id, &be, &bb);
    int failed = KQO_OK;
    int64_t r;
    if (st != KQO_OK) return st;
    if (w == NULL || x == NULL || y == NULL || rows == 0U || cols == 0U ||
        batch == 0U)
        return KQO_INVALID_ARGUMENT;
    if (cols % be != 0U) return KQO_DIMENSION_MISMATCH;
    row_bytes = cols / be * bb;
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(threads > 0 ? threads : 1) if (threads > 1)
#else
    (void)threads;
#endif
    for (r = 0; r < (int64_t)rows; ++r) {
        uint32_t b;
        for (b = 0U; b < batch; ++b) {
            float v = 0.0f;
            int s = kqo_row_dot_f32(type_id,
                                    (const unsigned char *)w + (uint64_t)r * row_bytes,
                                    row_bytes, x + (uint64_t)b * cols, cols, &v);
            if (s != KQO_OK) {
#ifdef _OPENMP
#pragma omp critical
#endif
                failed = s;
            }
            y[(uint64_t)b * rows + (uint64_t)r] = v;
        }
    }
    return failed;
}

/* GDN layouts (src/kq_weight_provider.c:17-20, :205-248, :438-451): the
 * model's value-head features are stored tiled by repeat while the
 * canonical order groups them by key head. grouped_to_tiled maps a
 * canonical index to its physical one with 16 key heads and 3 repeats. */
#define KQO_GDN_KEY_HEADS 16U
#define KQO_GDN_HEAD_WIDTH 128U
#define KQO_GDN_VALUE_REPEAT 3U

static uint64_t grouped_to_tiled(uint64_t canonical, uint64_t width) {
    uint64_t group = canonical / (KQO_GDN_VALUE_REPEAT * width);
    uint64_t within = canonical % (KQO_GDN_VALUE_REPEAT * width);
    uint64_t repeat = within / width;
    uint64_t feature = within % width;
    return (repeat * KQO_GDN_KEY_HEADS + group) * width + feature;
}

/* physical_row_for (src/kq_weight_provider.c:231-248) */
uint64_t kqo_gdn_physical_row(uint32_t transform, uint64_t canonical_row) {
    const uint64_t qk = 2ULL * KQO_GDN_KEY_HEADS * KQO_GDN_HEAD_WIDTH;
    switch (transform) {
    case KQO_GDN_QKV:
    case KQO_GDN_CONV:
        return canonical_row < qk ? canonical_row
                                  : qk + grouped_to_tiled(canonical_row - qk, KQO_GDN_HEAD_WIDTH);
    case KQO_GDN_ALPHA:
    case KQO_GDN_BETA:
        return grouped_to_tiled(canonical_row, 1U);
    case KQO_GDN_GATE:
        return grouped_to_tiled(canonical_row, KQO_GDN_HEAD_WIDTH);
    default:
        return canonical_row;
    }
}

uint64_t kqo_gdn_physical_column(uint32_t transform, uint64_t canonical_column) {
    return transform == KQO_GDN_OUT ? grouped_to_tiled(canonical_column, KQO_GDN_HEAD_WIDTH)
                                    : canonical_column;
}

/* The provider's linear for a GDN role (src/kq_weight_provider.c:438-475):
 * GDN_OUT scatters the activation into physical column order first; every
 * role dots canonical row r with physical row physical_row_for(r). A
 * transform that leaves the geometry fails with DIMENSION_MISMATCH (the
 * reference's TENSOR_LAYOUT_MISMATCH). */
int kqo_gdn_linear_f32(uint32_t transform, uint32_t type_id, const void *w, uint64_t rows,
                       uint64_t cols, const float *x, float *y, int threads) {
    uint32_t be, bb;
    uint64_t row_bytes;
    float *permuted = NULL;
    const float *act = x;
    int failed = KQO_OK;
    int64_t r;
    int st = kqo_geometry(type_id, &be, &bb);
    if (st != KQO_OK) return st;
    if (w == NULL || x == NULL || y == NULL || rows == 0U || cols == 0U)
        return KQO_INVALID_ARGUMENT;
    if (cols % be != 0U) return KQO_DIMENSION_MISMATCH;
    row_bytes = cols / be * bb;
    if (transform == KQO_GDN_OUT) {
        uint64_t i;
        permuted = (float *)calloc(cols, sizeof(float));
        if (permuted == NULL) return KQO_INVALID_ARGUMENT;
        for (i = 0U; i < cols; ++i) {
            uint64_t pc = kqo_gdn_physical_column(transform, i);
            if (pc >= cols) {
                free(permuted);
                return KQO_DIMENSION_MISMATCH;
            }
            permuted[pc] = x[i];
        }
        act = permuted;
    }
    for (r = 0; r < (int64_t)rows; ++r)
        if (kqo_gdn_physical_row(transform, (uint64_t)r) >= rows) {
            free(permuted);
            return KQO_DIMENSION_MISMATCH;
        }
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(threads > 0 ? threads : 1) if (threads > 1)
#else
    (void)threads;
#endif
    for (r = 0; r < (int64_t)rows; ++r) {
        const uint64_t pr = kqo_gdn_physical_row(transform, (uint64_t)r);
        float v = 0.0f;
        int s = kqo_row_dot_f32(type_id, (const unsigned char *)w + pr * row_bytes, row_bytes,
                                act, cols, &v);
        if (s != KQO_OK) {
#ifdef _OPENMP
#pragma omp critical
#endif
            failed = s;
        }
        y[r] = v;
    }
    free(permuted);
    return failed;
}

/* src/kq_model_exec.c:566-584: first maximum (strict >), ties -> lowest id. */
int kqo_argmax_f32(const float *logits, uint64_t count, uint32_t *id) {
    uint64_t i;
    uint32_t sel = 0U;
    if (logits == NULL || id == NULL || count == 0U || count > UINT32_MAX)
        return KQO_INVALID_ARGUMENT;
    for (i = 0U; i < count; ++i) {
        if (!isfinite(logits[i])) return KQO_NUMERIC_DOMAIN;
        if (i != 0U && logits[i] > logits[sel]) sel = (uint32_t)i;
    }
    *id = sel;
    return KQO_OK;
}

/* --- F32 primitives: src/kq_numeric.c:505-911 --- */
int kqo_f32_add(const float *a, const float *b, uint64_t n, float *out) {
    uint64_t i;
    if (!finite_vec(a, n) || !finite_vec(b, n)) return KQO_NUMERIC_DOMAIN;
    for (i = 0U; i < n; ++i) {
        float v = a[i] + b[i];
        if (!isfinite(v)) return KQO_NUMERIC_DOMAIN;
        out[i] = v;
    }
    return KQO_OK;
}

int kqo_f32_multiply(const float *a, const float *b, uint64_t n, float *out) {
    uint64_t i;
    if (!finite_vec(a, n) || !finite_vec(b, n)) return KQO_NUMERIC_DOMAIN;
    for (i = 0U; i < n; ++i) {
        float v = a[i] * b[i];
        if (!isfinite(v)) return KQO_NUMERIC_DOMAIN;
        out[i] = v;
    }
    return KQO_OK;
}

int kqo_f32_scale(const float *a, uint64_t n, float s, float *out) {
    uint64_t i;
    if (!isfinite(s) || !finite_vec(a, n)) return KQO_NUMERIC_DOMAIN;
    for (i = 0U; i < n; ++i) {
        out[i] = a[i] * s;
        if (!isfinite(out[i])) return KQO_NUMERIC_DOMAIN;
    }
    return KQO_OK;
}

int kqo_f32_dot(const float *a, const float *b, uint64_t n, float *out) {
    float acc = 0.0f;
    uint64_t i;
    if (n == 0U) return KQO_INVALID_ARGUMENT;
    if (!finite_vec(a, n) || !finite_vec(b, n)) return KQO_NUMERIC_DOMAIN;
    for (i = 0U; i < n; ++i) {
        float product = a[i] * b[i];
        acc = acc + product;
    }
    if (!isfinite(acc)) return KQO_NUMERIC_DOMAIN;
    *out = acc;
    return KQO_OK;
}

/* src/kq_numeric.c:628-638 (sign-stable logistic). */
static float sigmoid_scalar(float x) {
    if (x >= 0.0f) {
        float e = kqo_expf(-x);
        return 1.0f / (1.0f + e);
    } else {
        float e = kqo_expf(x);
        return e / (1.0f + e);
    }
}

int kqo_f32_sigmoid(const float *a, uint64_t n, float *out) {
    uint64_t i;
    if (!finite_vec(a, n)) return KQO_NUMERIC_DOMAIN;
    for (i = 0U; i < n; ++i) {
        out[i] = sigmoid_scalar(a[i]);
        if (!isfinite(out[i])) return KQO_NUMERIC_DOMAIN;
    }
    return KQO_OK;
}

int kqo_f32_silu(const float *a, uint64_t n, float *out) {
    uint64_t i;
    if (!finite_vec(a, n)) return KQO_NUMERIC_DOMAIN;
    for (i = 0U; i < n; ++i) {
        float s = sigmoid_scalar(a[i]);
        out[i] = a[i] * s;
        if (!isfinite(out[i])) return KQO_NUMERIC_DOMAIN;
    }
    return KQO_OK;
}

/* src/kq_numeric.c:690-720: silu(g) = g * sigmoid(g), then * up. */
int kqo_f32_swiglu(const float *g, const float *u, uint64_t n, float *out) {
    uint64_t i;
    if (!finite_vec(g, n) || !finite_vec(u, n)) return KQO_NUMERIC_DOMAIN;
    for (i = 0U; i < n; ++i) {
        float s = sigmoid_scalar(g[i]);
        float silu = g[i] * s;
        out[i] = silu * u[i];
        if (!isfinite(out[i])) return KQO_NUMERIC_DOMAIN;
    }
    return KQO_OK;
}

/* src/kq_moe_qwen38.c:436-459 (kq_moe_expert_member) as called by
 * kq_moe_execute_routed_expert_f32 (:461-566): gate and up rows as
 * left-to-right dots (kq_moe_project, :198-209), SwiGLU, the down rows over
 * the activated vector; the output is written only on success. */
int kqo_moe_routed_expert_f32(uint32_t hidden, uint32_t inter, const float *gate,
                              const float *up, const float *down, const float *x, float *out) {
    float *g = (float *)malloc((size_t)inter * 3u * sizeof(float) + (size_t)hidden * sizeof(float));
    float *u, *a, *o;
    int st = KQO_OK;
    uint32_t r;
    if (g == NULL) return KQO_INVALID_ARGUMENT;
    u = g + inter;
    a = u + inter;
    o = a + inter;
    for (r = 0U; r < inter && st == KQO_OK; ++r)
        st = kqo_f32_dot(gate + (size_t)r * hidden, x, hidden, &g[r]);
    for (r = 0U; r < inter && st == KQO_OK; ++r)
        st = kqo_f32_dot(up + (size_t)r * hidden, x, hidden, &u[r]);
    if (st == KQO_OK) st = kqo_f32_swiglu(g, u, inter, a);
    for (r = 0U; r < hidden && st == KQO_OK; ++r)
        st = kqo_f32_dot(down + (size_t)r * inter, a, inter, &o[r]);
    if (st == KQO_OK) memcpy(out, o, (size_t)hidden * sizeof(float));
    free(g);
    return st;
}

int kqo_f32_rms_norm(const float *a, const float *w, uint64_t n, float eps,
                     float *out) {
    float sum = 0.0f, mean, inv;
    uint64_t i;
    if (!isfinite(eps) || eps <= 0.0f) return KQO_NUMERIC_DOMAIN;
    if (!finite_vec(a, n) || !finite_vec(w, n)) return KQO_NUMERIC_DOMAIN;
    for (i = 0U; i < n; ++i) {
        float sq = a[i] * a[i];
        sum = sum + sq;
    }
    mean = sum / (float)n;
    inv = 1.0f / sqrtf(mean + eps);
    if (!isfinite(inv)) return KQO_NUMERIC_DOMAIN;
    for (i = 0U; i < n; ++i) {
        float nv = a[i] * inv;
        float wt = 1.0f + w[i];
        out[i] = nv * wt;
        if (!isfinite(out[i])) return KQO_NUMERIC_DOMAIN;
    }
    return KQO_OK;
}

/* src/kq_numeric.c:776-813: max, expf(x - max), left-to-right sum, divide. */
int kqo_f32_softmax(const float *a, uint64_t n, float *out) {
    float m, sum = 0.0f;
    uint64_t i;
    if (n == 0U) return KQO_INVALID_ARGUMENT;
    if (!finite_vec(a, n)) return KQO_NUMERIC_DOMAIN;
    m = a[0];
    for (i = 1U; i < n; ++i)
        if (a[i] > m) m = a[i];
    for (i = 0U; i < n; ++i) {
        out[i] = kqo_expf(a[i] - m);
        sum = sum + out[i];
    }
    if (!isfinite(sum) || sum <= 0.0f) return KQO_NUMERIC_DOMAIN;
    for (i = 0U; i < n; ++i) out[i] = out[i] / sum;
    return KQO_OK;
}

int kqo_f32_renormalize(const float *a, uint64_t n, float *out) {
    float sum = 0.0f;
    uint64_t i;
    if (!finite_vec(a, n)) return KQO_NUMERIC_DOMAIN;
    for (i = 0U; i < n; ++i) {
        if (a[i] < 0.0f) return KQO_NUMERIC_DOMAIN;
        sum = sum + a[i];
    }
    if (!isfinite(sum) || sum <= 0.0f) return KQO_NUMERIC_DOMAIN;
    for (i = 0U; i < n; ++i) out[i] = a[i] / sum;
    return KQO_OK;
}

/* src/kq_numeric.c:815-876: repeated best-remaining selection, ties to the
 * lower index. */
int kqo_f32_stable_top_k(const float *s, uint64_t n, uint32_t k,
                         uint32_t *idx, float *val) {
    uint32_t sel;
    uint64_t c;
    if (k == 0U || (uint64_t)k > n) return KQO_INVALID_ARGUMENT;
    if (!finite_vec(s, n)) return KQO_NUMERIC_DOMAIN;
    for (sel = 0U; sel < k; ++sel) {
        uint32_t best = UINT32_MAX;
        float bv = 0.0f;
        for (c = 0U; c < n; ++c) {
            uint32_t p;
            int taken = 0;
            for (p = 0U; p < sel; ++p)
                if (idx[p] == (uint32_t)c) { taken = 1; break; }
            if (!taken && (best == UINT32_MAX || s[c] > bv ||
                           (s[c] == bv && c < (uint64_t)best))) {
                best = (uint32_t)c;
                bv = s[c];
            }
        }
        idx[sel] = best;
        val[sel] = bv;
    }
    return KQO_OK;
}

/* src/kq_moe_qwen38.c:211-245: partial selection. Seed ids 0..k-1; a later
 * candidate replaces the current worst (lowest value, lowest id among equal
 * lowest) only if strictly greater; then insertion sort by descending value,
 * ascending id. */
void kqo_moe_select_top_k(const float *p, uint32_t n, uint32_t k,
                          uint32_t *ids) {
    uint32_t i;
    for (i = 0U; i < k; ++i) ids[i] = i;
    for (i = k; i < n; ++i) {
        uint32_t pos, worst = 0U;
        for (pos = 1U; pos < k; ++pos) {
            uint32_t c = ids[pos], w = ids[worst];
            if (p[c] < p[w] || (p[c] == p[w] && c < w)) worst = pos;
        }
        if (p[i] > p[ids[worst]]) ids[worst] = i;
    }
    for (i = 1U; i < k; ++i) {
        uint32_t v = ids[i], pos = i;
        while (pos > 0U) {
            uint32_t prev = ids[pos - 1U];
            if (p[prev] > p[v] || (p[prev] == p[v] && prev < v)) break;
            ids[pos] = prev;
            pos -= 1U;
        }
        ids[pos] = v;
    }
}

/* src/kq_moe_qwen38.c:247-274 */
static int finish_route(const kqo_moe_dims *d, const float *logits,
                        float *probs, uint32_t *ids, float *weights) {
    float sum = 0.0f;
    uint32_t p;
    int st = kqo_f32_softmax(logits, d->experts, probs);
    if (st != KQO_OK) return st;
    kqo_moe_select_top_k(probs, d->experts, d->top_k, ids);
    for (p = 0U; p < d->top_k; ++p) {
        weights[p] = probs[ids[p]];
        sum += weights[p];
    }
    if (!(sum > 0.0f) || !isfinite(sum)) return KQO_NUMERIC_DOMAIN;
    for (p = 0U; p < d->top_k; ++p) {
        weights[p] /= sum;
        if (!isfinite(weights[p])) return KQO_NUMERIC_DOMAIN;
    }
    return KQO_OK;
}

static uint64_t role_row_bytes(uint32_t type, uint64_t cols) {
    uint32_t be = 1U, bb = 4U;
    kqo_geometry(type, &be, &bb);
    return cols / be * bb;
}

/* One semantic linear (src/kq_moe_qwen38.c:198-209 for F32 weights,
 * kq_weight_provider_linear_f32 for packed ones): rows x row-dot. */
static int linear(const kqo_tensor *t, uint64_t matrix_index, uint64_t rows,
                  uint64_t cols, const float *x, float *y, int threads) {
    uint64_t rb = role_row_bytes(t->type, cols);
    const unsigned char *base =
        (const unsigned char *)t->data + matrix_index * rows * rb;
    if (t->type == KQO_F32) {
        int64_t r;
        int failed = KQO_OK;
        const float *wf = (const float *)(const void *)base;
#ifdef _OPENMP
#pragma omp parallel for schedule(static) num_threads(threads > 0 ? threads : 1) if (threads > 1)
#endif
        for (r = 0; r < (int64_t)rows; ++r) {
            int s = kqo_f32_dot(wf + (uint64_t)r * cols, x, cols, &y[r]);
            if (s != KQO_OK) {
#ifdef _OPENMP
#pragma omp critical
#endif
                failed = s;
            }
        }
        return failed;
    }
    return kqo_matvec_f32(t->type, base, rows, cols, x, 1U, y, threads);
}

int kqo_moe_route_f32(const kqo_moe_dims *d, const kqo_tensor *router,
                      const float *x, float *logits, float *probs,
                      uint32_t *ids, float *weights, int threads) {
    int st = linear(router, 0U, d->experts, d->hidden, x, logits, threads);
    if (st != KQO_OK) return st;
    return finish_route(d, logits, probs, ids, weights);
}

static int find_selected(const uint32_t *ids, uint32_t k, uint32_t e,
                         uint32_t *pos) {
    uint32_t i;
    for (i = 0U; i < k; ++i)
        if (ids[i] == e) { *pos = i; return 1; }
    return 0;
}

/* src/kq_moe_qwen38.c:604-867 (kq_moe_execute_common). */
int kqo_moe_execute(const kqo_moe_dims *d, const kqo_moe_weights *w,
                    const float *hidden, uint64_t tokens, float *out,
                    kqo_moe_trace *tr, int threads) {
    uint64_t H = d->hidden, E = d->experts, K = d->top_k, I = d->inter,
             S = d->shared_inter;
    float *logits, *probs, *sw, *gate, *up, *act, *eo, *wo, *sum, *sg, *su,
        *sa, *so, *gs;
    uint32_t *ids;
    uint64_t t;
    int st = KQO_OK;
    if (d == NULL || w == NULL || hidden == NULL || out == NULL || tokens == 0U ||
        K == 0U || K > E)
        return KQO_INVALID_ARGUMENT;
    logits = (float *)malloc(E * sizeof(float));
    probs = (float *)malloc(E * sizeof(float));
    sw = (float *)malloc(K * sizeof(float));
    ids = (uint32_t *)malloc(K * sizeof(uint32_t));
    gate = (float *)malloc(I * sizeof(float));
    up = (float *)malloc(I * sizeof(float));
    act = (float *)malloc(I * sizeof(float));
    eo = (float *)malloc(H * sizeof(float));
    wo = (float *)malloc(H * sizeof(float));
    sum = (float *)malloc(H * sizeof(float));
    sg = (float *)malloc(S * sizeof(float));
    su = (float *)malloc(S * sizeof(float));
    sa = (float *)malloc(S * sizeof(float));
    so = (float *)malloc(H * sizeof(float));
    gs = (float *)malloc(H * sizeof(float));
    if (!logits || !probs || !sw || !ids || !gate || !up || !act || !eo ||
        !wo || !sum || !sg || !su || !sa || !so || !gs) {
        st = KQO_INVALID_ARGUMENT;
        goto done;
    }
    if (!finite_vec(hidden, tokens * H)) { st = KQO_NUMERIC_DOMAIN; goto done; }
    for (t = 0U; t < tokens && st == KQO_OK; ++t) {
        const float *x = hidden + t * H;
        float *y = out + t * H;
        float logit = 0.0f, scale = 0.0f;
        uint32_t e;
        uint64_t f;
        st = kqo_moe_route_f32(d, &w->router, x, logits, probs, ids, sw, threads);
        if (st != KQO_OK) break;
        if (tr) {
            if (tr->router_logits) memcpy(tr->router_logits + t * E, logits, E * 4U);
            if (tr->router_probs) memcpy(tr->router_probs + t * E, probs, E * 4U);
            if (tr->selected_ids) memcpy(tr->selected_ids + t * K, ids, K * 4U);
            if (tr->selected_weights) memcpy(tr->selected_weights + t * K, sw, K * 4U);
        }
        memset(sum, 0, H * sizeof(float));
        for (e = 0U; e < E; ++e) {
            uint32_t pos = 0U;
            if (!find_selected(ids, (uint32_t)K, e, &pos)) continue;
            st = linear(&w->gate, e, I, H, x, gate, threads);
            if (st == KQO_OK) st = linear(&w->up, e, I, H, x, up, threads);
            if (st == KQO_OK) st = kqo_f32_swiglu(gate, up, I, act);
            if (st == KQO_OK) st = linear(&w->down, e, H, I, act, eo, threads);
            if (st == KQO_OK) st = kqo_f32_scale(eo, H, sw[pos], wo);
            if (st != KQO_OK) break;
            for (f = 0U; f < H; ++f) {
                sum[f] = sum[f] + wo[f];
                if (!isfinite(sum[f])) { st = KQO_NUMERIC_DOMAIN; break; }
            }
            if (st != KQO_OK) break;
            if (tr) {
                uint64_t o = (t * K + pos);
                if (tr->expert_gate) memcpy(tr->expert_gate + o * I, gate, I * 4U);
                if (tr->expert_up) memcpy(tr->expert_up + o * I, up, I * 4U);
                if (tr->expert_activated) memcpy(tr->expert_activated + o * I, act, I * 4U);
                if (tr->expert_output) memcpy(tr->expert_output + o * H, eo, H * 4U);
                if (tr->expert_weighted) memcpy(tr->expert_weighted + o * H, wo, H * 4U);
            }
        }
        if (st != KQO_OK) break;
        st = linear(&w->shared_gate, 0U, S, H, x, sg, threads);
        if (st == KQO_OK) st = linear(&w->shared_up, 0U, S, H, x, su, threads);
        if (st == KQO_OK) st = kqo_f32_swiglu(sg, su, S, sa);
        if (st == KQO_OK) st = linear(&w->shared_down, 0U, H, S, sa, so, threads);
        if (st == KQO_OK) st = linear(&w->shared_gate_weight, 0U, 1U, H, x, &logit, 1);
        if (st == KQO_OK) st = kqo_f32_sigmoid(&logit, 1U, &scale);
        if (st == KQO_OK) st = kqo_f32_scale(so, H, scale, gs);
        if (st == KQO_OK) st = kqo_f32_add(sum, gs, H, y);
        if (st != KQO_OK) break;
        if (tr) {
            if (tr->routed_sum) memcpy(tr->routed_sum + t * H, sum, H * 4U);
            if (tr->shared_gate_proj) memcpy(tr->shared_gate_proj + t * S, sg, S * 4U);
            if (tr->shared_up_proj) memcpy(tr->shared_up_proj + t * S, su, S * 4U);
            if (tr->shared_activated) memcpy(tr->shared_activated + t * S, sa, S * 4U);
            if (tr->shared_output) memcpy(tr->shared_output + t * H, so, H * 4U);
            if (tr->shared_scale_logit) tr->shared_scale_logit[t] = logit;
            if (tr->shared_scale) tr->shared_scale[t] = scale;
            if (tr->gated_shared) memcpy(tr->gated_shared + t * H, gs, H * 4U);
        }
    }
done:
    free(logits); free(probs); free(sw); free(ids); free(gate); free(up);
    free(act); free(eo); free(wo); free(sum); free(sg); free(su); free(sa);
    free(so); free(gs);
    return st;
}

int kqo_moe_permutation(const uint32_t *ids, uint64_t tokens, uint32_t top_k,
                        uint32_t experts, uint32_t *expert_offsets,
                        uint32_t *pair_token, uint32_t *pair_slot) {
    uint32_t *cursor;
    uint64_t t;
    uint32_t e, s;
    if (ids == NULL || expert_offsets == NULL || pair_token == NULL ||
        pair_slot == NULL || experts == 0U)
        return KQO_INVALID_ARGUMENT;
    cursor = (uint32_t *)calloc(experts, sizeof(uint32_t));
    if (cursor == NULL) return KQO_INVALID_ARGUMENT;
    for (t = 0U; t < tokens * top_k; ++t) {
        if (ids[t] >= experts) { free(cursor); return KQO_INVALID_ARGUMENT; }
        cursor[ids[t]] += 1U;
    }
    expert_offsets[0] = 0U;
    for (e = 0U; e < experts; ++e) {
        expert_offsets[e + 1U] = expert_offsets[e] + cursor[e];
        cursor[e] = 0U;
    }
    for (t = 0U; t < tokens; ++t) {
        for (s = 0U; s < top_k; ++s) {
            uint32_t ex = ids[t * top_k + s];
            uint32_t at = expert_offsets[ex] + cursor[ex]++;
            pair_token[at] = (uint32_t)t;
            pair_slot[at] = s;
        }
    }
    free(cursor);
    return KQO_OK;
}


/* ------------------------------------------------------------------ */
/* Gated residual around a layer block (hyper-connection read / write).
 *
 * Restates kq_layer_gr_read_common (src/kq_layer_qwen38.c:40-172) and
 * kq_layer_gr_write_f32 (:196-208): per branch RMS norm; a rank-r down
 * projection divided by the branch count and passed through SiLU; an up
 * projection to per-element sigmoid read gates; the gate-weighted branch
 * mix divided by the branch count; the per-branch write gate
 * 2 * sigmoid(inject . normalized / branches). The down and up weights are
 * F32 (the reference's F32 path: left-to-right sums of rounded products)
 * or packed blocks (its provider path through kq_weight_provider_linear_f32,
 * i.e. row dots); both are row dots here. All sums are left to right in
 * binary32 (the reference's -ffp-contract=off order). */
int kqo_gr_read(uint32_t nbranch, uint32_t hidden, uint32_t rank, float eps,
                const float *branches, const float *norm, uint32_t down_type,
                const void *down, uint32_t up_type, const void *up, const float *inject,
                float *normalized, float *read_gate, float *mixed, float *rank_ws,
                float *write_gate) {
    const uint64_t width = (uint64_t)nbranch * hidden;
    uint64_t i;
    uint32_t b;
    int st;
    if (nbranch == 0U || hidden == 0U || rank == 0U || branches == NULL || norm == NULL ||
        down == NULL || up == NULL || inject == NULL || normalized == NULL ||
        read_gate == NULL || mixed == NULL || rank_ws == NULL || write_gate == NULL)
        return KQO_INVALID_ARGUMENT;
    for (b = 0U; b < nbranch; ++b) {
        st = kqo_f32_rms_norm(branches + (uint64_t)b * hidden, norm + (uint64_t)b * hidden,
                              hidden, eps, normalized + (uint64_t)b * hidden);
        if (st != KQO_OK) return st;
    }
    st = kqo_matvec_f32(down_type, down, rank, width, normalized, 1U, rank_ws, 1);
    if (st != KQO_OK) return st;
    for (i = 0U; i < rank; ++i) rank_ws[i] /= (float)nbranch;
    for (i = 0U; i < rank; ++i) {
        const float s = sigmoid_scalar(rank_ws[i]);
        rank_ws[i] *= s;
    }
    st = kqo_matvec_f32(up_type, up, width, rank, rank_ws, 1U, read_gate, 1);
    if (st != KQO_OK) return st;
    for (i = 0U; i < width; ++i) read_gate[i] = sigmoid_scalar(read_gate[i]);
    for (i = 0U; i < hidden; ++i) {
        float sum = 0.0f;
        for (b = 0U; b < nbranch; ++b) {
            const uint64_t o = (uint64_t)b * hidden + i;
            const float p = read_gate[o] * normalized[o];
            sum += p;
        }
        mixed[i] = sum / (float)nbranch;
    }
    for (b = 0U; b < nbranch; ++b) {
        float sum = 0.0f;
        for (i = 0U; i < width; ++i) {
            const float p = inject[(uint64_t)b * width + i] * normalized[i];
            sum += p;
        }
        write_gate[b] = sum;
    }
    for (b = 0U; b < nbranch; ++b) write_gate[b] /= (float)nbranch;
    for (b = 0U; b < nbranch; ++b) write_gate[b] = 2.0f * sigmoid_scalar(write_gate[b]);
    return KQO_OK;
}

void kqo_gr_write(uint32_t nbranch, uint32_t hidden, const float *branches,
                  const float *block_output, const float *write_gate, float *out) {
    uint32_t b, i;
    for (b = 0U; b < nbranch; ++b)
        for (i = 0U; i < hidden; ++i) {
            const uint64_t o = (uint64_t)b * hidden + i;
            const float p = block_output[i] * write_gate[b];
            out[o] = branches[o] + p;
        }
}
