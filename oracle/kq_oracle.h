/*
 * kq_oracle.h — CPU restatement of Kestrel-Q's quantized-weight path.
 *
 * TEST INFRASTRUCTURE ONLY. This library is the checker: tests/, the smoke
 * check in __graft_entry__.py and the cpu_baseline leg of bench.py load it.
 * The product (libkq_hip.so) never links, loads or calls it.
 *
 * Built with the reference's floating-point flags (CMakeLists.txt:104-117:
 * -O2 -fno-fast-math -ffp-contract=off, no SIMD intrinsics) so every product
 * and sum is a separately rounded IEEE binary32 operation in source order.
 *
 * Each function cites the reference function it restates. Parity status of
 * each piece (what pins it) is listed in the header comment of kq_oracle.c.
 */
#ifndef KQ_ORACLE_H
#define KQ_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF type ids (include/kq_gguf.h:15-23); Q6_K = 14 from the GGML enum. */
enum {
    KQO_F32 = 0,
    KQO_Q5_1 = 7,
    KQO_Q8_0 = 8,
    KQO_Q4_K = 12,
    KQO_Q5_K = 13,
    KQO_Q6_K = 14,
    KQO_IQ4_NL = 20,
    KQO_BF16 = 30
};

/* Status codes: same integers as include/kq_status.h. */
enum {
    KQO_OK = 0,
    KQO_INVALID_ARGUMENT = 1,
    KQO_UNSUPPORTED_TENSOR_TYPE = 12,
    KQO_ARITHMETIC_OVERFLOW = 13,
    KQO_INVALID_TOKEN_ID = 31,
    KQO_BUFFER_TOO_SMALL = 32,
    KQO_MALFORMED_QUANTIZED_DATA = 38,
    KQO_NUMERIC_DOMAIN = 39,
    KQO_DIMENSION_MISMATCH = 40
};

int kqo_geometry(uint32_t type_id, uint32_t *block_elements,
                 uint32_t *bytes_per_block);
float kqo_f16_to_f32(uint16_t value);
void kqo_f16_to_f32_array(const uint16_t *in, uint64_t n, float *out);
float kqo_expf(float x);
void kqo_expf_array(const float *in, uint64_t n, float *out, int threads);
uint64_t kqo_expf_libm_mismatches(uint64_t start, uint64_t count,
                                  int threads);

int kqo_dequantize_blocks_f32(uint32_t type_id, const void *packed,
                              uint64_t packed_bytes, float *output,
                              uint64_t output_capacity,
                              uint64_t *output_count);
int kqo_row_dot_f32(uint32_t type_id, const void *packed,
                    uint64_t packed_bytes, const float *x, uint64_t count,
                    float *output);
/* y[b*rows + r] = row_dot(W row r, x[b*cols ...]); rows in parallel over
 * `threads` OpenMP threads with per-row arithmetic unchanged. */
int kqo_matvec_f32(uint32_t type_id, const void *w, uint64_t rows,
                   uint64_t cols, const float *x, uint32_t batch, float *y,
                   int threads);
int kqo_argmax_f32(const float *logits, uint64_t count, uint32_t *id);

int kqo_f32_add(const float *a, const float *b, uint64_t n, float *out);
int kqo_f32_multiply(const float *a, const float *b, uint64_t n, float *out);
int kqo_f32_scale(const float *a, uint64_t n, float s, float *out);
int kqo_f32_dot(const float *a, const float *b, uint64_t n, float *out);
int kqo_f32_sigmoid(const float *a, uint64_t n, float *out);
int kqo_f32_silu(const float *a, uint64_t n, float *out);
int kqo_f32_swiglu(const float *g, const float *u, uint64_t n, float *out);
/* one routed expert on F32 member matrices (src/kq_moe_qwen38.c:436-566) */
int kqo_moe_routed_expert_f32(uint32_t hidden, uint32_t inter, const float *gate,
                              const float *up, const float *down, const float *x, float *out);
int kqo_f32_rms_norm(const float *a, const float *w, uint64_t n, float eps,
                     float *out);
int kqo_f32_softmax(const float *a, uint64_t n, float *out);
int kqo_f32_renormalize(const float *a, uint64_t n, float *out);
int kqo_f32_stable_top_k(const float *s, uint64_t n, uint32_t k,
                         uint32_t *idx, float *val);

void kqo_moe_select_top_k(const float *probs, uint32_t n, uint32_t k,
                          uint32_t *ids);

typedef struct kqo_moe_dims {
    uint32_t hidden;
    uint32_t experts;
    uint32_t top_k;
    uint32_t inter;
    uint32_t shared_inter;
} kqo_moe_dims;

/* One weight role: F32 row-major floats or packed GGUF blocks, rows of
 * `cols` elements; routed roles hold `experts` matrices back to back. */
typedef struct kqo_tensor {
    uint32_t type;
    const void *data;
} kqo_tensor;

typedef struct kqo_moe_weights {
    kqo_tensor router;             /* [experts][hidden] */
    kqo_tensor gate;               /* [experts][inter][hidden] */
    kqo_tensor up;                 /* [experts][inter][hidden] */
    kqo_tensor down;               /* [experts][hidden][inter] */
    kqo_tensor shared_gate;        /* [shared_inter][hidden] */
    kqo_tensor shared_up;          /* [shared_inter][hidden] */
    kqo_tensor shared_down;        /* [hidden][shared_inter] */
    kqo_tensor shared_gate_weight; /* [hidden] */
} kqo_moe_weights;

/* Optional per-token record of the checkpoints the reference emits
 * (include/kq_moe.h:23-70). Any pointer may be NULL. Sized per token. */
typedef struct kqo_moe_trace {
    float *router_logits;      /* [tokens][experts] */
    float *router_probs;       /* [tokens][experts] */
    uint32_t *selected_ids;    /* [tokens][top_k] */
    float *selected_weights;   /* [tokens][top_k] */
    float *routed_sum;         /* [tokens][hidden] */
    float *shared_gate_proj;   /* [tokens][shared_inter] */
    float *shared_up_proj;     /* [tokens][shared_inter] */
    float *shared_activated;   /* [tokens][shared_inter] */
    float *shared_output;      /* [tokens][hidden] */
    float *shared_scale_logit; /* [tokens] */
    float *shared_scale;       /* [tokens] */
    float *gated_shared;       /* [tokens][hidden] */
    /* routed per (token, top_k position): */
    float *expert_gate;        /* [tokens][top_k][inter] */
    float *expert_up;          /* [tokens][top_k][inter] */
    float *expert_activated;   /* [tokens][top_k][inter] */
    float *expert_output;      /* [tokens][top_k][hidden] */
    float *expert_weighted;    /* [tokens][top_k][hidden] */
} kqo_moe_trace;

int kqo_moe_route_f32(const kqo_moe_dims *d, const kqo_tensor *router,
                      const float *x, float *logits, float *probs,
                      uint32_t *ids, float *weights, int threads);
int kqo_moe_execute(const kqo_moe_dims *d, const kqo_moe_weights *w,
                    const float *hidden, uint64_t tokens, float *out,
                    kqo_moe_trace *trace, int threads);

/* Stable counting sort of (token, slot) pairs by expert id, tokens ascending
 * within an expert: the permutation the prefill grouped path must produce. */
int kqo_moe_permutation(const uint32_t *ids, uint64_t tokens, uint32_t top_k,
                        uint32_t experts, uint32_t *expert_offsets,
                        uint32_t *pair_token, uint32_t *pair_slot);

/* gated residual read / write around a layer block
 * (src/kq_layer_qwen38.c:40-208): branches [nbranch][hidden], norm
 * [nbranch*hidden], down [rank][width] and up [width][rank] as F32 or packed
 * rows, inject [nbranch][width] F32. */
int kqo_gr_read(uint32_t nbranch, uint32_t hidden, uint32_t rank, float eps,
                const float *branches, const float *norm, uint32_t down_type,
                const void *down, uint32_t up_type, const void *up, const float *inject,
                float *normalized, float *read_gate, float *mixed, float *rank_ws,
                float *write_gate);
void kqo_gr_write(uint32_t nbranch, uint32_t hidden, const float *branches,
                  const float *block_output, const float *write_gate, float *out);

/* GDN layouts: the provider's row and column maps and its linear for the
 * GDN roles (src/kq_weight_provider.c:205-248, :438-475). */
enum {
    KQO_GDN_NONE = 0,
    KQO_GDN_QKV = 1,
    KQO_GDN_GATE = 2,
    KQO_GDN_ALPHA = 3,
    KQO_GDN_BETA = 4,
    KQO_GDN_CONV = 5,
    KQO_GDN_OUT = 6
};
uint64_t kqo_gdn_physical_row(uint32_t transform, uint64_t canonical_row);
uint64_t kqo_gdn_physical_column(uint32_t transform, uint64_t canonical_column);
int kqo_gdn_linear_f32(uint32_t transform, uint32_t type_id, const void *w, uint64_t rows,
                       uint64_t cols, const float *x, float *y, int threads);

/* kq_sample.c: the reference's sampler (src/kq_sampling.c). The RNG
 * record has the layout of kq_sampling_rng_state (include/kq_sampling.h). */
typedef struct kqo_rng_state {
    uint32_t version;
    uint32_t reserved;
    uint64_t seed;
    uint64_t stream;
    uint64_t state;
    uint64_t increment;
    uint64_t draws;
    uint64_t integrity;
} kqo_rng_state;

typedef struct kqo_sample_result {
    uint32_t selected_token_id;
    uint32_t top_k_retained_count;
    uint32_t retained_count;
    uint32_t rng_word;
    float selected_probability;
    float maximum_probability;
    float normalized_sum_f32;
    uint32_t reserved;
    double uniform_value;
} kqo_sample_result;

void kqo_rng_seed(uint64_t seed, uint64_t stream, kqo_rng_state *out);
uint32_t kqo_rng_next(kqo_rng_state *state);
/* one selection with the RNG word already drawn; scores_out / probs_out
 * (optional, count each) receive the processed logits and the final
 * probabilities (zero outside the kept set) */
int kqo_sample_f32(float temperature, float top_p, uint32_t top_k, uint32_t canonical_count,
                   const float *logits, uint32_t count, uint32_t word, kqo_sample_result *result,
                   float *scores_out, float *probs_out);

/* kq_certify.c: the device's certified one-token routing restated on the
 * CPU (ids of the certified selection, or *certified = 0), and a campaign
 * of random and near-tie cases against kqo_moe_route_f32. */
int kqo_route_certify(uint32_t experts, uint32_t hidden, uint32_t top_k, const float *router,
                      const float *x, uint32_t *ids, int *certified);
int kqo_certify_campaign(uint64_t seed, uint64_t trials, uint32_t experts, uint32_t hidden,
                         uint32_t top_k, int mode, float sigma, double slack, int threads,
                         uint64_t *stats);

#ifdef __cplusplus
}
#endif

#endif
