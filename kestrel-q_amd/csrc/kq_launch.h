/*
 * kq_launch.h — internal launcher interface between the C host layer
 * (kq_hip_api.c, validation and orchestration) and the HIP kernel files.
 * Not installed; the public boundary is include/kq_hip.h.
 *
 * Launchers enqueue on the given stream and return the launch status only;
 * numeric failures found on the device are OR-ed into *status.
 */
#ifndef KQ_LAUNCH_H
#define KQ_LAUNCH_H

#include <hip/hip_runtime_api.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KQ_LAUNCH_F32 0u
#define KQ_LAUNCH_Q5_1 7u
#define KQ_LAUNCH_Q8_0 8u
#define KQ_LAUNCH_Q4_K 12u
#define KQ_LAUNCH_Q5_K 13u
#define KQ_LAUNCH_Q6_K 14u
#define KQ_LAUNCH_IQ4_NL 20u
#define KQ_LAUNCH_BF16 30u

/* dequant (kq_dequant.hip) */
hipError_t kq_launch_dequant(uint32_t type, const void *packed, uint64_t blocks,
                             float *out, uint32_t *status, hipStream_t stream);

/* matvec / argmax (kq_matvec.hip) */
int kq_launch_matvec_supported(uint32_t type, uint32_t cols, uint32_t batch);
uint32_t kq_launch_matvec_waves(uint32_t type, uint32_t rows, uint32_t cols, uint32_t batch);
/* part_v/part_i (optional): per batch column, part_stride argmax partials;
 * the launch's waves fill the first kq_launch_matvec_waves of them and the
 * rest get the neutral entry (-inf, UINT32_MAX). */
hipError_t kq_launch_matvec(uint32_t type, const void *W, uint32_t rows, uint32_t cols,
                            const float *x, uint32_t batch, float *y, uint32_t *status,
                            float *part_v, uint32_t *part_i, uint32_t part_stride,
                            hipStream_t stream);
/* y[t] = W x[t] for many tokens, Q8_0 W on MFMA (kq_grouped.hip): row
 * lengths 256, 320, 512, 640, 1024, 2048 or 10240 */
int kq_launch_gemm_q8_0_supported(uint32_t rows, uint32_t cols);
/* one Q8_0 matrix (w1: also the up matrix of a gate/up pair, SwiGLU'd)
 * against many split activation rows on MFMA (kq_dense.hip): out
 * [splits][tokens][rows], the splits summed by the caller;
 * kq_launch_dense_split forms xh, xl [tokens][k] and sig [tokens] (a
 * non-finite row flags the input (input != 0) or a numeric failure) */
int kq_launch_dense_q8_supported(uint32_t rows, uint32_t k, uint32_t tokens);
uint32_t kq_launch_dense_q8_splits(uint32_t k, uint32_t splits);
hipError_t kq_launch_dense_split(const float *x, uint32_t tokens, uint32_t k, void *xh, void *xl,
                                 int *sig, int input, uint32_t *status, hipStream_t s);
/* a gate/up pair launched with splits > 1 leaves gate and up partials
 * [splits][tokens][2 rows]; kq_launch_dense_swiglu sums them in order and
 * writes swiglu(gate, up) [tokens][rows] */
hipError_t kq_launch_dense_swiglu(const float *parts, uint32_t splits, uint32_t tokens,
                                  uint32_t rows, float *out, uint32_t *status, hipStream_t s);
hipError_t kq_launch_dense_q8(const void *w0, const void *w1, uint32_t rows, uint32_t k,
                              const void *xh, const void *xl, const int *sig, uint32_t tokens,
                              uint32_t splits, float *out, uint32_t *status, hipStream_t s);
hipError_t kq_launch_gemm_q8_0(const void *W, uint32_t rows, uint32_t cols, const float *x,
                               uint32_t tokens, float *y, uint32_t *status, hipStream_t stream);
/* batched Q6_K matvec on MFMA (kq_grouped.hip), used by kq_launch_matvec
 * where supported; same partials contract */
int kq_launch_matvec_mfma_supported(uint32_t type, uint32_t rows, uint32_t cols, uint32_t batch);
uint32_t kq_launch_matvec_mfma_waves(uint32_t rows, uint32_t cols);
hipError_t kq_launch_matvec_mfma(const void *W, uint32_t rows, uint32_t cols, const float *x,
                                 uint32_t batch, float *y, uint32_t *status, float *part_v,
                                 uint32_t *part_i, uint32_t part_stride, hipStream_t stream);
uint32_t kq_launch_argmax_parts(uint32_t count);
hipError_t kq_launch_argmax(const float *logits, uint32_t count, uint32_t batch,
                            float *part_v, uint32_t *part_i, uint32_t *ids,
                            uint32_t *status, hipStream_t stream);
hipError_t kq_launch_argmax_from_parts(const float *part_v, const uint32_t *part_i,
                                       uint32_t nparts, uint32_t batch, uint32_t *ids,
                                       hipStream_t stream);
/* The allocation-free LM head's partials: a file-scope device array of
 * kq_launch_noalloc_parts() (value, row) pairs per device. _init (with
 * `device` current) returns its device address, looked up once per device;
 * the values come first, then the row ids. */
uint32_t kq_launch_noalloc_parts(void);
hipError_t kq_launch_noalloc_scratch_init(int device, void **out);

/* gated residual around a layer block (kq_gr.hip) */
hipError_t kq_launch_gr_norm(const float *x, const float *norm, uint32_t tokens,
                             uint32_t branches, uint32_t hidden, float eps, float *normalized,
                             uint32_t *status, hipStream_t stream);
hipError_t kq_launch_gr_rank(float *rank, uint32_t n, uint32_t branches, const float *parts,
                             uint32_t nparts, uint32_t *status, hipStream_t s);
hipError_t kq_launch_gr_mix(const float *read_raw, const float *normalized, const float *inject,
                            uint32_t tokens, uint32_t branches, uint32_t hidden, float *mixed,
                            float *write_gate, uint32_t *status, hipStream_t stream);
hipError_t kq_launch_gr_write(const float *x, const float *block_output, const float *write_gate,
                              uint32_t tokens, uint32_t branches, uint32_t hidden, float *out,
                              uint32_t *status, hipStream_t stream);
/* y[b][r] = W[r] . x[b] for F32 weights [rows][cols], cols % 4 == 0 */
/* y = W x for Q8_0 rows of more than 2048 columns in one launch (batch
 * chunks of 4), the gated residual's rank projection */
hipError_t kq_launch_matvec_q8w(const void *W, uint32_t rows, uint32_t cols, const float *x,
                                uint32_t batch, float *y, uint32_t *status, hipStream_t s);
hipError_t kq_launch_matvec_f32w(const float *W, uint32_t rows, uint32_t cols, const float *x,
                                 uint32_t batch, float *y, uint32_t *status, hipStream_t stream);

/* elementwise expf (kq_dequant.hip), used to pin the device expf */
hipError_t kq_launch_expf(const float *in, uint64_t n, float *out, hipStream_t stream);

/* MoE (kq_moe.hip) */
typedef struct kq_launch_moe_dims {
    uint32_t hidden;
    uint32_t experts;
    uint32_t top_k;
    uint32_t inter;
    uint32_t shared_inter;
} kq_launch_moe_dims;

typedef struct kq_launch_moe_weights {
    const float *router;
    uint32_t gate_type;
    const void *gate;
    uint32_t up_type;
    const void *up;
    uint32_t down_type;
    const void *down;
    uint32_t shared_gate_type;
    const void *shared_gate;
    uint32_t shared_up_type;
    const void *shared_up;
    uint32_t shared_down_type;
    const void *shared_down;
    const float *shared_gate_weight;
} kq_launch_moe_weights;

/* Device workspace carved by the host from caller scratch
 * (kq_launch_moe_ws_bytes gives the size for a token count). */
typedef struct kq_launch_moe_ws {
    float *router_t;      /* router rows + shared gate row, transposed to
                             [hidden/4][experts_padded][4] (several tokens) */
    float *logits;        /* [tokens][experts] */
    float *probs;         /* [tokens][experts] */
    uint32_t *ids;        /* [tokens][top_k], descending probability */
    float *weights;       /* [tokens][top_k] */
    uint32_t *order;      /* [tokens][top_k]: slots sorted by ascending id */
    float *shared_logit;  /* [tokens] */
    float *shared_scale;  /* [tokens] */
    float *act;           /* [tokens][top_k + 1][max(inter, shared_inter)]; the grouped
                             path uses it as [tokens * top_k + tokens][inter]: routed
                             pairs in permuted order, then the shared expert's rows */
    uint32_t *offsets;    /* [experts + 1]: first permuted position of each expert */
    uint32_t *perm_tok;   /* [tokens * top_k]: token at each permuted position */
    uint32_t *pos;        /* [tokens][top_k]: permuted position of each (token, slot) */
    float *outp;          /* [tokens * top_k + tokens][hidden]: down outputs */
    double *bound;        /* [experts + 1][2]: exact product sums and the bound on the
                             CPU's sequential sum (certified one-token routing) */
    uint32_t *certified;  /* one-token route: 1 certified, 2 refined, 0 exact */
    void *dstage;         /* grouped Q6_K down pass: act split per position */
    void *gitems;         /* grouped passes' work list (kq_launch_gu_lds) */
} kq_launch_moe_ws;

uint32_t kq_launch_moe_experts_padded(uint32_t experts);
uint64_t kq_launch_moe_ws_bytes(const kq_launch_moe_dims *d, uint32_t tokens);
void kq_launch_moe_ws_carve(const kq_launch_moe_dims *d, uint32_t tokens, void *base,
                            kq_launch_moe_ws *ws);
int kq_launch_moe_supported(const kq_launch_moe_dims *d, const kq_launch_moe_weights *w);
/* logits (+ shared gate logit), softmax, partial-selection top-k, weights.
 * certify != 0 (one token, only the ids needed exactly): selects from exact
 * product sums with a proven error bound when the bound separates the
 * selection, from the exact chains of the contenders when that separates
 * it, and from every exact chain otherwise; the logits and probabilities
 * are then not always written and the weights are within fp32 tolerance of
 * the CPU's. ids_out (optional) also receives the ids. stage (optional,
 * several tokens): where the route finish also splits every token's row for
 * the grouped gate/up pass (kq_launch_moe_grouped_stage). */
hipError_t kq_launch_moe_route(const kq_launch_moe_dims *d, const float *router,
                               const float *shared_gate_weight, const float *hidden,
                               uint32_t tokens, const kq_launch_moe_ws *ws, uint32_t *status,
                               int certify, uint32_t *ids_out, void *stage,
                               hipStream_t stream);
/* grouped multi-token path (kq_grouped.hip): stable permutation, per-expert
 * MFMA gate/up + SwiGLU and down over all of an expert's tokens, ordered
 * combine; needs the route results in ws */
int kq_launch_moe_grouped_supported(const kq_launch_moe_dims *d, const kq_launch_moe_weights *w);
/* the permutation alone (pair_slot optional) */
hipError_t kq_launch_moe_permute(const uint32_t *ids, uint32_t tokens, uint32_t top_k,
                                 uint32_t experts, uint32_t *offsets, uint32_t *pair_token,
                                 uint32_t *pos, uint32_t *pair_slot, uint32_t *status,
                                 hipStream_t stream);
/* prefill gate/up of Q4_K or Q5_K experts (type) through LDS
 * (kq_grouped_gu.hip): the per-token activation split, then the pass over
 * the routed experts' 16-token chunks (and the shared expert's,
 * with_shared, in the same format) on a persistent grid; items is scratch
 * of kq_launch_gu_items_bytes */
int kq_launch_gu_lds_supported(uint32_t type, uint32_t hidden);
uint64_t kq_launch_gu_stage_bytes(uint32_t tokens, uint32_t hidden);
hipError_t kq_launch_gu_stage(const float *hidden_states, uint32_t tokens, uint32_t hidden,
                              void *staged, uint32_t *status, hipStream_t s);
uint64_t kq_launch_gu_items_bytes(uint32_t experts, uint32_t tokens, uint32_t top_k);
/* items_ready: the permutation already wrote the item list (moe_permute);
 * posmax (hidden 2048 only, zeroed beforehand, or NULL): each position's
 * largest |act| as float bits, for kq_launch_dn_lds */
hipError_t kq_launch_gu_lds(uint32_t type, uint32_t hidden, const void *gate, const void *up,
                            const void *shared_gate, const void *shared_up, const void *staged,
                            const uint32_t *offsets, const uint32_t *perm_tok, uint32_t experts,
                            uint32_t tokens, uint32_t top_k, uint32_t rows, int with_shared,
                            int items_ready, void *items, float *act, uint32_t *posmax,
                            uint32_t *status, hipStream_t s);
/* prefill Q5_1 or Q8_0 down (type) over the same item list
 * (kq_grouped_dn.hip); staged is scratch of kq_launch_dn_stage_bytes */
int kq_launch_dn_small_supported(uint32_t type, uint32_t inter);
hipError_t kq_launch_dn_small(uint32_t type, uint32_t inter, uint32_t hidden, const void *down,
                              const void *shared_down, const float *act, uint32_t tokens,
                              uint32_t top_k, const void *items, void *staged, float *out,
                              uint32_t *status, hipStream_t s);
/* prefill Q6_K down over the gate/up pass's item list (kq_grouped_dn.hip) */
int kq_launch_dn_lds_supported(uint32_t inter);
uint64_t kq_launch_dn_stage_bytes(uint32_t npos, uint32_t inter);
hipError_t kq_launch_dn_lds(uint32_t inter, uint32_t hidden, const void *down,
                            const void *shared_down, const float *act, uint32_t tokens,
                            uint32_t top_k, const void *items, void *staged,
                            const uint32_t *posmax, float *out, uint32_t *status,
                            hipStream_t s);
/* where the Q4_K / Q5_K gate/up pass reads its per-token activation split (ws's
 * outp), or NULL when these weights take another pass; the route can form
 * it (kq_launch_moe_route's stage), and staged tells the grouped path so */
void *kq_launch_moe_grouped_stage(const kq_launch_moe_dims *d, const kq_launch_moe_weights *w,
                                  const kq_launch_moe_ws *ws);
hipError_t kq_launch_moe_grouped(const kq_launch_moe_dims *d, const kq_launch_moe_weights *w,
                                 const float *hidden, uint32_t tokens,
                                 const kq_launch_moe_ws *ws, int staged, float *out,
                                 uint32_t *status, hipStream_t stream);
hipError_t kq_launch_moe_experts(const kq_launch_moe_dims *d, const kq_launch_moe_weights *w,
                                 const float *hidden, uint32_t tokens,
                                 const kq_launch_moe_ws *ws, float *out, uint32_t *status,
                                 hipStream_t stream);
/* the exact softmax, partial-selection top-k, weights, ascending-id order
 * and shared gate from logits [tokens][experts] and shared_logit [tokens]
 * (experts <= 960) */
hipError_t kq_launch_moe_route_finish(const float *logits, const float *shared_logit,
                                      uint32_t experts, uint32_t top_k, uint32_t tokens,
                                      float *probs, uint32_t *ids, float *weights,
                                      uint32_t *order, float *shared_scale, uint32_t *status,
                                      hipStream_t stream);

/* GDN canonical-order copies (kq_layout.hip): `units` units of unit_bytes
 * (even) gathered from physical into canonical order; rows (columns == 0):
 * unit j <- j below prefix, else prefix + grouped_to_tiled(j - prefix,
 * width); columns: 128-column unit u of each row of units_per_row (48)
 * <- unit (u % 3) * 16 + u / 3 */
hipError_t kq_launch_gdn_gather(const void *physical, void *canonical, uint64_t units,
                                uint32_t unit_bytes, int columns, uint64_t prefix, uint32_t width,
                                uint32_t units_per_row, hipStream_t s);

/* MoE on F32 expert weights in the reference's order (kq_moe_f32.hip) */
typedef struct kq_launch_moe_f32_weights {
    const float *router;             /* [experts][hidden] */
    const float *gate, *up, *down;   /* [E][I][H], [E][I][H], [E][H][I] */
    const float *shared_gate, *shared_up, *shared_down; /* [S][H], [S][H], [H][S] */
    const float *shared_gate_weight; /* [hidden] */
} kq_launch_moe_f32_weights;

/* every intermediate, per token (the checkpoint trace); Ip = max(I, S) */
typedef struct kq_launch_moe_f32_ws {
    float *logits, *probs;            /* [T][E] */
    uint32_t *ids, *order;            /* [T][K] */
    float *weights;                   /* [T][K] */
    float *shared_logit, *shared_scale; /* [T] */
    float *gate, *up, *act;           /* [T][K+1][Ip] (slot K: the shared expert) */
    float *out, *weighted;            /* [T][K+1][H] */
    float *routed_sum;                /* [T][H] */
} kq_launch_moe_f32_ws;

hipError_t kq_launch_f32_scan(const float *p, uint64_t n, uint32_t *status, hipStream_t s);
/* one routed expert on F32 member matrices (gate/up [I][H], down [H][I]):
 * gate, up, activated [I] and the output [H], every dot the reference's
 * left-to-right binary32 chain */
hipError_t kq_launch_routed_expert_f32(const float *gate_w, const float *up_w,
                                       const float *down_w, const float *x, uint32_t hidden,
                                       uint32_t inter, float *gate, float *up, float *act,
                                       float *out, uint32_t *status, hipStream_t s);
hipError_t kq_launch_moe_f32(const kq_launch_moe_dims *d, const kq_launch_moe_f32_weights *w,
                             const float *hidden, uint32_t tokens,
                             const kq_launch_moe_f32_ws *ws, float *out, uint32_t *status,
                             hipStream_t s);

/* The token sampler (kq_sample.hip). status: the first failure, in the
 * reference's order of checks: a numeric failure before the RNG draw, one
 * inside the categorical walk, or a selected id at or past the canonical
 * token count (the record is filled in that case too). */
enum {
    KQ_SAMPLE_OK = 0,
    KQ_SAMPLE_NUMERIC_BEFORE_DRAW = 1,
    KQ_SAMPLE_NUMERIC_IN_DRAW = 2,
    KQ_SAMPLE_INVALID_TOKEN = 3,
    KQ_SAMPLE_FULL_SORT = 4 /* the fast path's top did not fit: run _full */
};

typedef struct kq_launch_sample_out {
    uint32_t status;
    uint32_t selected;
    uint32_t top_k_retained;
    uint32_t retained;
    float selected_probability;
    float maximum_probability;
    float normalized_sum;
    uint32_t reserved;
    double uniform;
} kq_launch_sample_out;

typedef struct kq_launch_sample_args {
    const float *logits; /* [count] */
    uint32_t count;      /* vocabulary */
    uint32_t canonical;  /* ids at or past this are padding */
    uint32_t top_k;      /* 0: off */
    float temperature;
    float top_p;
    uint32_t word;       /* the RNG word of this draw */
    /* device work arrays of count entries each */
    float *scores;
    uint32_t *keys, *ids, *sorted_keys, *sorted_ids;
    float *probs;
    uint32_t *bad_per_block; /* ceil(count / 256) */
    uint32_t *max_per_block; /* ceil(count / 256) */
    void *sort_temp;
    size_t sort_bytes;   /* kq_launch_sample_sort_bytes(count) */
    kq_launch_sample_out *out;
    uint32_t sequential_draw; /* nonzero: over many kept ids, always the
                                 sequential binary64 walk (diagnostic) */
} kq_launch_sample_args;

hipError_t kq_launch_sample_sort_bytes(uint32_t count, size_t *bytes);
/* prep, then a tail without the full sort where kq_launch_sample_fast is
 * nonzero (1: top-k 1..64 over at most 1024 prep blocks; 2: nothing cut,
 * top-k 0 or the whole vocabulary with top-p 1, more than 4096 ids), else
 * the full sort and its tail */
hipError_t kq_launch_sample(const kq_launch_sample_args *args, hipStream_t s);
int kq_launch_sample_fast(uint32_t count, uint32_t top_k, float top_p);
/* the full sort and the tail on the prep already in the scratch */
hipError_t kq_launch_sample_full(const kq_launch_sample_args *args, hipStream_t s);

#ifdef __cplusplus
}
#endif

#endif
