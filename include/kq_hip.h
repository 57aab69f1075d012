/*
 * kq_hip.h — C ABI of the MI355X (gfx950) backend for Kestrel-Q's
 * quantized-weight path: GGUF block dequantization fused into
 * matrix-vector products, the MoE expert FFN and the LM head, fed from
 * GGUF files. Packed formats: Q4_K, Q5_K, Q6_K, Q5_1, Q8_0, IQ4_NL; F32 and
 * BF16 are decoded and ingested.
 *
 * Conventions (same as the reference library):
 *  - every entry point returns kq_status and fills the optional
 *    kq_diagnostic (include/kq_status.h);
 *  - arguments are validated before any device work is enqueued and bad
 *    arguments fail closed with the reference's status codes;
 *  - the caller owns every buffer, including device scratch.
 * Device pointers are plain `void *` / `float *` obtained from
 * kq_hip_malloc (or any allocation on the context's device); packed weights
 * are byte-identical GGUF blocks (kq_tensor_view_physical_data). Weight and
 * activation pointers must be 16-byte aligned.
 *
 * Execution: work is enqueued on the context's stream. In the default
 * synchronous mode each call waits for its work and reports device-detected
 * failures (non-finite block scales -> KQ_STATUS_MALFORMED_QUANTIZED_DATA,
 * non-finite inputs/results -> KQ_STATUS_NUMERIC_DOMAIN). In asynchronous
 * mode calls return after enqueueing and kq_hip_context_synchronize reports
 * them.
 *
 * Commit on success: the reference stages its outputs and copies them only
 * when a call succeeds (src/kq_weight_provider.c:420, :480,
 * src/kq_moe_qwen38.c:562-565). A synchronous call here does the same for
 * device outputs: it copies their prior contents aside before its first
 * launch (one device-to-device copy of the outputs) and copies them back if
 * the call fails, so a failed call leaves its outputs as they were
 * (kq_hip_context_set_commit_on_success turns this off). Asynchronous calls
 * and kq_hip_lm_head_greedy_f32_noalloc (which may not allocate the copy)
 * write in place: their outputs are unspecified when the status reports a
 * failure.
 */
#ifndef KQ_HIP_H
#define KQ_HIP_H

#include <stdint.h>

#include "kq_gguf.h"
#include "kq_status.h"

#ifdef __cplusplus
extern "C" {
#endif

/* GGUF tensor type ids (include/kq_gguf.h:15-23; Q6_K = 14, the GGML id). */
#define KQ_HIP_TYPE_F32 0U
#define KQ_HIP_TYPE_Q5_1 7U
#define KQ_HIP_TYPE_Q8_0 8U
#define KQ_HIP_TYPE_Q4_K 12U
#define KQ_HIP_TYPE_Q5_K 13U
#define KQ_HIP_TYPE_Q6_K 14U
#define KQ_HIP_TYPE_IQ4_NL 20U
#define KQ_HIP_TYPE_BF16 30U

typedef struct kq_hip_context kq_hip_context;

/* ------------------------------------------------------------------ */
/* Context, stream and memory. The reference has no device runtime; its
 * only device entry point is `int kq_cuda_smoke(void)` (include/kq_cuda.h:9). */

kq_status kq_hip_context_create(int device, kq_hip_context **out_context,
                                kq_diagnostic *diagnostic);
void kq_hip_context_destroy(kq_hip_context *context);
/* 0 = synchronous (default), 1 = asynchronous. */
kq_status kq_hip_context_set_async(kq_hip_context *context, int async,
                                   kq_diagnostic *diagnostic);
/* 1 = synchronous calls restore their device outputs when they fail
 * (default), 0 = outputs of a failed call are unspecified. */
kq_status kq_hip_context_set_commit_on_success(kq_hip_context *context, int commit,
                                               kq_diagnostic *diagnostic);
/* Waits for enqueued work; reports and clears device-detected failures. */
kq_status kq_hip_context_synchronize(kq_hip_context *context,
                                     kq_diagnostic *diagnostic);
/* The hipStream_t the context enqueues on (as an opaque pointer). */
void *kq_hip_context_stream(const kq_hip_context *context);

kq_status kq_hip_malloc(kq_hip_context *context, uint64_t bytes,
                        void **out_device_ptr, kq_diagnostic *diagnostic);
void kq_hip_free(kq_hip_context *context, void *device_ptr);
kq_status kq_hip_upload(kq_hip_context *context, void *device_dst,
                        const void *host_src, uint64_t bytes,
                        kq_diagnostic *diagnostic);
kq_status kq_hip_download(kq_hip_context *context, void *host_dst,
                          const void *device_src, uint64_t bytes,
                          kq_diagnostic *diagnostic);

/* ------------------------------------------------------------------ */
/* Quant geometry (host only).
 * Replaces kq_quant_geometry_for_type / kq_quant_packed_size
 * (include/kq_tensor_view.h:85-92, src/kq_tensor_view.c:44-108). */

typedef struct kq_hip_quant_geometry {
    uint32_t type_id;
    uint64_t block_elements;
    uint64_t bytes_per_block;
} kq_hip_quant_geometry;

kq_status kq_hip_quant_geometry_for_type(uint32_t type_id,
                                         kq_hip_quant_geometry *out_geometry,
                                         kq_diagnostic *diagnostic);
kq_status kq_hip_quant_packed_size(uint32_t type_id, uint64_t element_count,
                                   uint64_t *out_packed_bytes,
                                   kq_diagnostic *diagnostic);
/* Byte span of expert `expert_id` in a contiguous [experts][rows][cols]
 * packed stack. Replaces the member addressing of
 * kq_tensor_view_open_expert_member (src/kq_tensor_view.c:664-807). */
kq_status kq_hip_expert_member_span(uint32_t type_id, uint64_t rows,
                                    uint64_t cols, uint32_t expert_count,
                                    uint32_t expert_id,
                                    uint64_t *out_byte_offset,
                                    uint64_t *out_byte_count,
                                    kq_diagnostic *diagnostic);

/* ------------------------------------------------------------------ */
/* GGUF ingestion: packed tensor bytes from a parsed file (include/kq_gguf.h)
 * into device memory, byte for byte. The reference reads the same bytes
 * through kq_tensor_view_physical_data (src/kq_tensor_view.c) and its
 * tensor span (src/kq_gguf.c:1019-1078). */

/* Byte span of expert `expert_id` in a routed expert stack: the experts are
 * the slowest (last) GGUF dimension, so the member is the tensor's
 * element_count / dimensions[rank-1] elements at expert_id times that.
 * Mirrors kq_tensor_view_open_expert_member (src/kq_tensor_view.c:664-807)
 * without the semantic registry: rank below 2 fails with
 * INVALID_QUANTIZED_GEOMETRY, an expert past the stack with
 * SPAN_OUT_OF_RANGE, a member that is not whole blocks with
 * NONCONTIGUOUS_TENSOR_VIEW. */
kq_status kq_hip_gguf_expert_member(const kq_gguf_tensor *tensor,
                                    uint32_t expert_id,
                                    uint64_t *out_byte_offset,
                                    uint64_t *out_byte_count,
                                    kq_diagnostic *diagnostic);

/* Copies the tensor's packed_bytes to device_dst (device_capacity bytes,
 * else BUFFER_TOO_SMALL). The tensor must be one of gguf's descriptors
 * (TENSOR_OWNERSHIP_MISMATCH). Synchronous; file pages are mapped a window
 * at a time and staged through pinned host buffers. */
kq_status kq_hip_gguf_upload_tensor(kq_hip_context *context,
                                    const kq_gguf *gguf,
                                    const kq_gguf_tensor *tensor,
                                    void *device_dst,
                                    uint64_t device_capacity,
                                    kq_diagnostic *diagnostic);

/* Copies one expert member (kq_hip_gguf_expert_member) to device_dst. */
kq_status kq_hip_gguf_upload_expert_member(kq_hip_context *context,
                                           const kq_gguf *gguf,
                                           const kq_gguf_tensor *tensor,
                                           uint32_t expert_id,
                                           void *device_dst,
                                           uint64_t device_capacity,
                                           kq_diagnostic *diagnostic);

/* Logical element ranges to whole blocks (host only). Replaces
 * kq_quant_element_to_block / kq_quant_range_to_blocks
 * (include/kq_tensor_view.h:93-104, src/kq_tensor_view.c:110-215), same
 * checks and statuses. */
typedef struct kq_hip_quant_block_span {
    uint64_t requested_element_offset;
    uint64_t requested_element_count;
    uint64_t first_block;
    uint64_t block_count;
    uint64_t physical_byte_offset;
    uint64_t physical_byte_length;
    uint64_t leading_elements;
    uint64_t trailing_elements;
} kq_hip_quant_block_span;

kq_status kq_hip_quant_element_to_block(uint32_t type_id, uint64_t total_elements,
                                        uint64_t element_index, uint64_t *out_block_index,
                                        uint64_t *out_element_in_block,
                                        kq_diagnostic *diagnostic);
kq_status kq_hip_quant_range_to_blocks(uint32_t type_id, uint64_t total_elements,
                                       uint64_t element_offset, uint64_t element_count,
                                       kq_hip_quant_block_span *out_span,
                                       kq_diagnostic *diagnostic);

/* ------------------------------------------------------------------ */
/* Device tensor views: the packed blocks of one tensor (or expert member,
 * or span) in device memory, with the layout facts the reference's
 * kq_tensor_view_info carries for the numeric path (include/kq_tensor_view.h:
 * 26-31, 52-80). */
typedef enum kq_hip_tensor_layout {
    KQ_HIP_LAYOUT_CANONICAL_CONTIGUOUS = 0,
    KQ_HIP_LAYOUT_TRANSFORMED_PHYSICAL,
    KQ_HIP_LAYOUT_SPLIT_SEGMENT,
    KQ_HIP_LAYOUT_FUSED_MEMBER
} kq_hip_tensor_layout;

/* kq_numeric_view_order (include/kq_numeric.h:15-18) */
typedef enum kq_hip_view_order {
    KQ_HIP_PHYSICAL_ORDER = 0,
    KQ_HIP_REQUIRE_CANONICAL_ORDER
} kq_hip_view_order;

typedef struct kq_hip_tensor_view {
    uint32_t type_id;
    uint32_t layout;               /* kq_hip_tensor_layout */
    uint64_t block_elements;
    uint64_t bytes_per_block;
    uint64_t block_count;
    uint32_t canonical_contiguous; /* 1: blocks in canonical element order */
    uint32_t reserved;
    const void *device_data;       /* the view's first block */
    uint64_t mapped_bytes;         /* bytes of device_data the view covers */
} kq_hip_tensor_view;

/* A view of `bytes` packed bytes at device_data (whole blocks, else
 * MALFORMED_QUANTIZED_DATA). A canonical-contiguous layout sets
 * canonical_contiguous; TRANSFORMED_PHYSICAL (the GDN tensors as stored)
 * and SPLIT_SEGMENT do not. */
kq_status kq_hip_tensor_view_init(uint32_t type_id, const void *device_data, uint64_t bytes,
                                  uint32_t layout, kq_hip_tensor_view *out_view,
                                  kq_diagnostic *diagnostic);

/* Replaces kq_dequantize_view_blocks_f32 (include/kq_numeric.h:28-36,
 * src/kq_numeric.c:361-418): blocks [relative_first_block, + block_count)
 * of the view, bit-identical decode. KQ_HIP_REQUIRE_CANONICAL_ORDER on a
 * view that is not canonical-contiguous (or is transformed or a split
 * segment) fails with TENSOR_LAYOUT_MISMATCH; a range past the view with
 * SPAN_OUT_OF_RANGE; a view without data or geometry with
 * TENSOR_OWNERSHIP_MISMATCH. */
kq_status kq_hip_dequantize_view_blocks_f32(kq_hip_context *context,
                                            const kq_hip_tensor_view *view,
                                            uint64_t relative_first_block,
                                            uint64_t block_count, uint32_t order,
                                            float *device_output, uint64_t output_capacity,
                                            uint64_t *output_count,
                                            kq_diagnostic *diagnostic);

/* ------------------------------------------------------------------ */
/* GDN row and column layouts. The model stores the value-head rows of
 * attn_qkv, attn_gate, ssm_alpha, ssm_beta and ssm_conv1d, and the columns
 * of ssm_out, tiled by repeat; the reference reorders them at every linear
 * (physical_row_for, grouped_to_tiled, the GDN_OUT activation permutation:
 * src/kq_weight_provider.c:205-248, :438-451). */
typedef enum kq_hip_gdn_layout {
    KQ_HIP_GDN_NONE = 0,
    KQ_HIP_GDN_QKV,   /* rows: 4096 q/k rows, then 6144 value rows (width 128) */
    KQ_HIP_GDN_GATE,  /* rows: 6144 (width 128) */
    KQ_HIP_GDN_ALPHA, /* rows: 48 (width 1) */
    KQ_HIP_GDN_BETA,  /* rows: 48 (width 1) */
    KQ_HIP_GDN_CONV,  /* rows: as QKV */
    KQ_HIP_GDN_OUT    /* columns: 6144 (width 128) */
} kq_hip_gdn_layout;

/* The physical row (column) holding canonical row (column) `index` of a
 * matrix of `rows` x `columns` in a GDN layout (host only): the reference's
 * physical_row_for / grouped_to_tiled. A geometry the layout does not map
 * onto itself fails with TENSOR_LAYOUT_MISMATCH. */
kq_status kq_hip_gdn_physical_row(uint32_t gdn_layout, uint64_t rows, uint64_t canonical_row,
                                  uint64_t *out_physical_row, kq_diagnostic *diagnostic);
kq_status kq_hip_gdn_physical_column(uint32_t gdn_layout, uint64_t columns,
                                     uint64_t canonical_column, uint64_t *out_physical_column,
                                     kq_diagnostic *diagnostic);

/* Writes the canonical-order copy of a packed matrix stored in a GDN
 * layout: row r of the copy is physical row physical_row(r); for GDN_OUT
 * each row's 128-column units move whole (32-element block formats and
 * F32 / BF16; K-quants give UNSUPPORTED_TENSOR_TYPE). The ordinary matvec on
 * the copy then equals the reference's provider linear on the stored
 * tensor (src/kq_weight_provider.c:438-475). Synchronous unless the
 * context is asynchronous. */
kq_status kq_hip_gdn_canonicalize(kq_hip_context *context, uint32_t gdn_layout,
                                  uint32_t type_id, const void *device_physical, uint64_t rows,
                                  uint64_t columns, void *device_canonical,
                                  uint64_t canonical_capacity, kq_diagnostic *diagnostic);

/* ------------------------------------------------------------------ */
/* Numeric core. */

/* Replaces kq_dequantize_blocks_f32 (include/kq_numeric.h:20-26,
 * src/kq_numeric.c:297-359). Bit-identical decode. *output_count receives
 * the required element count (also on KQ_STATUS_BUFFER_TOO_SMALL). */
kq_status kq_hip_dequantize_blocks_f32(kq_hip_context *context,
                                       uint32_t type_id,
                                       const void *device_packed,
                                       uint64_t packed_bytes,
                                       float *device_output,
                                       uint64_t output_capacity,
                                       uint64_t *output_count,
                                       kq_diagnostic *diagnostic);

/* Replaces kq_quantized_row_dot_f32 (include/kq_numeric.h:38-44,
 * src/kq_numeric.c:420-503): one packed row dotted with x. */
kq_status kq_hip_quantized_row_dot_f32(kq_hip_context *context,
                                       uint32_t type_id,
                                       const void *device_packed,
                                       uint64_t packed_bytes,
                                       const float *device_activation,
                                       uint64_t activation_count,
                                       float *device_output,
                                       kq_diagnostic *diagnostic);

/* Replaces kq_weight_provider_linear_f32 (include/kq_weight_provider.h:56-61,
 * src/kq_weight_provider.c:378-509), extended to `batch` activation vectors:
 * y[b*rows + r] = row r of W (packed, rows contiguous) . x[b*columns ...].
 * batch 1..8; columns any whole number of blocks up to 65536; the packed
 * matrix below 4 GiB. */
kq_status kq_hip_quantized_matvec_f32(kq_hip_context *context,
                                      uint32_t type_id,
                                      const void *device_weights,
                                      uint64_t rows, uint64_t columns,
                                      const float *device_input,
                                      uint32_t batch, float *device_output,
                                      uint64_t output_capacity,
                                      kq_diagnostic *diagnostic);

/* Replaces kq_model_exec_greedy_argmax_f32 (include/kq_model_exec.h:200-202,
 * src/kq_model_exec.c:566-584) for `batch` logit rows of logit_count each:
 * first maximum, ties to the lowest id, non-finite logits rejected. */
kq_status kq_hip_greedy_argmax_f32(kq_hip_context *context,
                                   const float *device_logits,
                                   uint64_t logit_count, uint32_t batch,
                                   uint32_t *device_token_ids,
                                   kq_diagnostic *diagnostic);

/* The LM-head call plus greedy selection (src/kq_model_exec.c:830-846 and
 * :1095-1113): logits = W_lm h for `batch` hidden states, then argmax per
 * batch row, fused (the argmax partials come out of the matvec kernel). */
kq_status kq_hip_lm_head_greedy_f32(kq_hip_context *context,
                                    uint32_t type_id,
                                    const void *device_weights,
                                    uint64_t vocab, uint64_t columns,
                                    const float *device_hidden,
                                    uint32_t batch, float *device_logits,
                                    uint32_t *device_token_ids,
                                    kq_diagnostic *diagnostic);

/* kq_hip_lm_head_greedy_f32 without any allocation: no counterpart in the
 * reference. For callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops): the argmax partials, which the
 * entry point above allocates in the context on first use and grows on
 * demand, live here in a static array of 131,072 (value, row) pairs
 * (1 MiB) that each device holds for the life of the process. Same
 * arguments, validation, kernels and results; a call needing more
 * partials than the array holds (wave count of its launches x batch)
 * fails with KQ_STATUS_LIMIT_EXCEEDED before any launch. All calls on one
 * device share the array: calls that overlap in time on the same device
 * (other streams or contexts) race. */
kq_status kq_hip_lm_head_greedy_f32_noalloc(kq_hip_context *context,
                                            uint32_t type_id,
                                            const void *device_weights,
                                            uint64_t vocab, uint64_t columns,
                                            const float *device_hidden,
                                            uint32_t batch, float *device_logits,
                                            uint32_t *device_token_ids,
                                            kq_diagnostic *diagnostic);

/* ------------------------------------------------------------------ */
/* MoE operator. */

/* Mirrors kq_moe_dimensions (src/kq_moe_internal.h:10-17) for F32
 * activations; configs come from kq_hip_moe_config_create, which mirrors
 * the test-config constructor kq_moe_test_config_create
 * (src/kq_moe.c:283-297) and its validation (src/kq_moe.c:83-140). */
typedef struct kq_hip_moe_dimensions {
    uint32_t hidden_size;
    uint32_t expert_count;
    uint32_t top_k;
    uint32_t routed_intermediate_size;
    uint32_t shared_intermediate_size;
} kq_hip_moe_dimensions;

typedef struct kq_hip_moe_config kq_hip_moe_config;

kq_status kq_hip_moe_config_create(const kq_hip_moe_dimensions *dimensions,
                                   kq_hip_moe_config **out_config,
                                   kq_diagnostic *diagnostic);
void kq_hip_moe_config_close(kq_hip_moe_config *config);
/* Device scratch needed by route/execute for `token_count` tokens. */
uint64_t kq_hip_moe_config_scratch_bytes(const kq_hip_moe_config *config,
                                         uint64_t token_count);

/* Mirrors kq_moe_weights_f32 (include/kq_moe.h:72-89) with a GGUF type per
 * packed role. Routed roles are contiguous expert stacks:
 * gate/up [experts][routed_inter][hidden], down [experts][hidden][routed_inter]
 * (the GGUF dims [cols, rows, experts], src/kq_tensor_view.c:664-807).
 * router [experts][hidden] and shared_gate_weight [hidden] are F32. */
typedef struct kq_hip_moe_weights {
    const float *router;
    uint32_t routed_gate_type;
    const void *routed_gate;
    uint32_t routed_up_type;
    const void *routed_up;
    uint32_t routed_down_type;
    const void *routed_down;
    uint32_t shared_gate_type;
    const void *shared_gate;
    uint32_t shared_up_type;
    const void *shared_up;
    uint32_t shared_down_type;
    const void *shared_down;
    const float *shared_gate_weight;
} kq_hip_moe_weights;

/* Replaces kq_moe_route_f32 (include/kq_moe.h:128-141,
 * src/kq_moe_qwen38.c:276-376) for token_count tokens: logits, softmax
 * probabilities, top-k ids (bit-identical to the CPU partial selection)
 * and renormalised weights, each [tokens][...] in device memory.
 * router_weight_count must be experts x hidden (DIMENSION_MISMATCH); each
 * capacity counts values and must hold tokens x experts (logits,
 * probabilities) or tokens x top_k (ids, weights), else BUFFER_TOO_SMALL
 * with the required counts in the message; outputs that overlap each other
 * or an input fail with ALIASING_VIOLATION. The results are formed in
 * scratch and written to the outputs only once the call has succeeded (in
 * a synchronous call). device_shared_gate_weight [hidden] is read for the
 * layer's shared gate logit, which the route leaves in scratch. */
kq_status kq_hip_moe_route_f32(kq_hip_context *context,
                               const kq_hip_moe_config *config,
                               const float *device_router_weight,
                               uint64_t router_weight_count,
                               const float *device_shared_gate_weight,
                               const float *device_hidden,
                               uint64_t token_count,
                               float *device_router_logits,
                               uint64_t router_logits_capacity,
                               float *device_router_probabilities,
                               uint64_t router_probabilities_capacity,
                               uint32_t *device_selected_ids,
                               uint64_t selected_ids_capacity,
                               float *device_selected_weights,
                               uint64_t selected_weights_capacity,
                               void *device_scratch, uint64_t scratch_bytes,
                               kq_diagnostic *diagnostic);

/* Mirrors kq_moe_routed_expert_weights_f32 (include/kq_moe.h:91-98): one
 * routed expert's member matrices, gate/up [routed_inter][hidden] and down
 * [hidden][routed_inter], with element counts. */
typedef struct kq_hip_moe_routed_expert_weights_f32 {
    const float *gate;
    uint64_t gate_count;
    const float *up;
    uint64_t up_count;
    const float *down;
    uint64_t down_count;
} kq_hip_moe_routed_expert_weights_f32;

/* Device scratch of kq_hip_moe_execute_routed_expert_f32: gate, up,
 * activated [routed_inter] and the expert's output [hidden] (the
 * reference's one-expert workspace, src/kq_moe.c). */
uint64_t kq_hip_moe_config_one_expert_scratch_bytes(const kq_hip_moe_config *config);

/* Replaces kq_moe_execute_routed_expert_f32 (include/kq_moe.h:143-152,
 * src/kq_moe_qwen38.c:461-566): output_token [hidden] = down .
 * swiglu(gate . x, up . x) for one expert's member matrices, every dot the
 * reference's left-to-right binary32 chain (bit-identical). expert_id only
 * names the member (INVALID_ARGUMENT past the config's experts). Checks in
 * the reference's order: arguments, expert id, output and scratch sizes
 * (BUFFER_TOO_SMALL), member counts (DIMENSION_MISMATCH), overlaps
 * (ALIASING_VIOLATION); non-finite weights, input or results give
 * NUMERIC_DOMAIN. The output is written only when the call succeeds. */
kq_status kq_hip_moe_execute_routed_expert_f32(kq_hip_context *context,
                                               const kq_hip_moe_config *config,
                                               const kq_hip_moe_routed_expert_weights_f32 *weights,
                                               uint32_t expert_id,
                                               const float *device_hidden_token,
                                               float *device_output_token,
                                               uint64_t output_capacity,
                                               void *device_scratch, uint64_t scratch_bytes,
                                               kq_diagnostic *diagnostic);

/* Replaces kq_moe_execute_quantized (src/kq_moe_internal.h:56-64,
 * src/kq_moe_qwen38.c:882-901) / kq_moe_execute_f32 (include/kq_moe.h:154-166):
 * hidden [tokens][hidden] -> output [tokens][hidden]. Optional
 * device_selected_ids [tokens][top_k] receives the routing; it must be
 * 4-byte aligned and overlap neither the input, the output nor the scratch
 * (ALIASING_VIOLATION). */
kq_status kq_hip_moe_execute_quantized(kq_hip_context *context,
                                       const kq_hip_moe_config *config,
                                       const kq_hip_moe_weights *weights,
                                       const float *device_hidden,
                                       uint64_t token_count,
                                       float *device_output,
                                       uint64_t output_capacity,
                                       uint32_t *device_selected_ids,
                                       void *device_scratch,
                                       uint64_t scratch_bytes,
                                       kq_diagnostic *diagnostic);

/* ------------------------------------------------------------------ */
/* MoE on F32 expert weights, with the reference's observers. */

/* Mirrors kq_moe_weights_f32 (include/kq_moe.h:72-89): device pointers
 * with element counts. Routed stacks gate/up [experts][routed_inter][hidden],
 * down [experts][hidden][routed_inter]; shared gate/up [shared_inter][hidden],
 * down [hidden][shared_inter]; router [experts][hidden]; shared gate
 * weight [hidden]. */
typedef struct kq_hip_moe_weights_f32 {
    const float *router;
    uint64_t router_count;
    const float *routed_gate;
    uint64_t routed_gate_count;
    const float *routed_up;
    uint64_t routed_up_count;
    const float *routed_down;
    uint64_t routed_down_count;
    const float *shared_gate;
    uint64_t shared_gate_count;
    const float *shared_up;
    uint64_t shared_up_count;
    const float *shared_down;
    uint64_t shared_down_count;
    const float *shared_gate_weight;
    uint64_t shared_gate_weight_count;
} kq_hip_moe_weights_f32;

/* The reference's checkpoint kinds, records and observers
 * (include/kq_moe.h:13-70), same values and layouts; `values` point to
 * host copies valid during the callback. */
#define KQ_HIP_MOE_NO_EXPERT UINT32_MAX
typedef enum kq_hip_moe_checkpoint_kind {
    KQ_HIP_MOE_CHECKPOINT_ROUTER_LOGITS = 0,
    KQ_HIP_MOE_CHECKPOINT_ROUTER_PROBABILITIES,
    KQ_HIP_MOE_CHECKPOINT_SELECTED_WEIGHTS,
    KQ_HIP_MOE_CHECKPOINT_ROUTED_GATE,
    KQ_HIP_MOE_CHECKPOINT_ROUTED_UP,
    KQ_HIP_MOE_CHECKPOINT_ROUTED_ACTIVATED,
    KQ_HIP_MOE_CHECKPOINT_ROUTED_EXPERT_OUTPUT,
    KQ_HIP_MOE_CHECKPOINT_ROUTED_WEIGHTED_OUTPUT,
    KQ_HIP_MOE_CHECKPOINT_ROUTED_WEIGHTED_SUM,
    KQ_HIP_MOE_CHECKPOINT_SHARED_GATE_PROJECTION,
    KQ_HIP_MOE_CHECKPOINT_SHARED_UP_PROJECTION,
    KQ_HIP_MOE_CHECKPOINT_SHARED_ACTIVATED,
    KQ_HIP_MOE_CHECKPOINT_SHARED_OUTPUT,
    KQ_HIP_MOE_CHECKPOINT_SHARED_SCALE_LOGIT,
    KQ_HIP_MOE_CHECKPOINT_SHARED_SCALE,
    KQ_HIP_MOE_CHECKPOINT_GATED_SHARED_OUTPUT,
    KQ_HIP_MOE_CHECKPOINT_OPERATOR_OUTPUT
} kq_hip_moe_checkpoint_kind;

typedef struct kq_hip_moe_checkpoint {
    kq_hip_moe_checkpoint_kind kind;
    uint64_t token_index;
    uint32_t expert_id;
    uint32_t top_k_position;
    uint32_t rank;
    uint64_t dimensions[2];
    const float *values;
    uint64_t value_count;
} kq_hip_moe_checkpoint;

typedef void (*kq_hip_moe_checkpoint_observer)(const kq_hip_moe_checkpoint *checkpoint,
                                               void *user_data);

typedef struct kq_hip_moe_route {
    uint64_t token_index;
    const float *router_logits;
    const float *router_probabilities;
    uint64_t expert_count;
    const uint32_t *selected_expert_ids;
    const float *selected_weights;
    uint32_t selected_count;
} kq_hip_moe_route;

typedef void (*kq_hip_moe_route_observer)(const kq_hip_moe_route *route, void *user_data);

/* Device scratch of kq_hip_moe_execute_f32 for `token_count` tokens: every
 * intermediate of every token (the checkpoints). */
uint64_t kq_hip_moe_config_f32_scratch_bytes(const kq_hip_moe_config *config,
                                             uint64_t token_count);

/* Replaces kq_moe_execute_f32 (include/kq_moe.h:154-166,
 * src/kq_moe_qwen38.c:604-880): every checkpoint bit-identical to the
 * reference's (one device thread per output runs the reference's
 * left-to-right binary32 sums). Any hidden size; at most 65,535 tokens and
 * 960 experts. Weight counts must match the config (DIMENSION_MISMATCH);
 * non-finite weights, inputs or results give NUMERIC_DOMAIN. The observers
 * (optional) are called after the device work succeeds, synchronously, in
 * the reference's order (per token: route, router logits, probabilities,
 * selected weights, each selected expert in ascending id, routed sum, the
 * shared expert's checkpoints, output); a failed call calls none. Always
 * synchronous. */
kq_status kq_hip_moe_execute_f32(kq_hip_context *context, const kq_hip_moe_config *config,
                                 const kq_hip_moe_weights_f32 *weights,
                                 const float *device_hidden, uint64_t token_count,
                                 float *device_output, uint64_t output_capacity,
                                 void *device_scratch, uint64_t scratch_bytes,
                                 kq_hip_moe_route_observer route_observer,
                                 kq_hip_moe_checkpoint_observer checkpoint_observer,
                                 void *observer_user_data, kq_diagnostic *diagnostic);

/* The token->expert permutation that the multi-token execution runs its
 * grouped expert GEMMs over: the (token, slot) pairs of selected_ids
 * [tokens][top_k] (from kq_hip_moe_route_f32) stably sorted by expert id,
 * tokens ascending within an expert. expert_offsets [experts + 1] holds
 * each expert's first position; pair_token / pair_slot [tokens * top_k] the
 * pair at each position. device_scratch needs tokens * top_k * 4 bytes.
 * No entry point of the reference corresponds: it runs the tokens one by
 * one (kq_moe_execute_common, src/kq_moe_qwen38.c:666-865); this exposes
 * the permutation so callers can check it. An id >= expert_count fails
 * with KQ_STATUS_INVALID_ARGUMENT. */
kq_status kq_hip_moe_token_permutation(kq_hip_context *context,
                                       const kq_hip_moe_config *config,
                                       const uint32_t *device_selected_ids,
                                       uint64_t token_count,
                                       uint32_t *device_expert_offsets,
                                       uint32_t *device_pair_token,
                                       uint32_t *device_pair_slot,
                                       void *device_scratch,
                                       uint64_t scratch_bytes,
                                       kq_diagnostic *diagnostic);

/* ------------------------------------------------------------------ */
/* The gated residual around a layer block: the hyper-connection read and
 * write of src/kq_layer_qwen38.c:40-208, which src/kq_layer.c:779-813 calls
 * around the MoE. A token's state is branch_count residual branches of
 * hidden_size values (width = branch_count * hidden_size). */
typedef struct kq_hip_gr_dimensions {
    uint32_t branch_count;
    uint32_t hidden_size;
    uint32_t rank;
    float rms_epsilon;
} kq_hip_gr_dimensions;

/* Mirrors kq_layer_gr_weights_f32 (src/kq_layer_internal.h) with a type for
 * each projection: the reference's provider path reads them as packed rows
 * (the model's blk.N.hc_ffn_down / hc_ffn_up are Q8_0). norm [width] and
 * inject [branch_count][width] are F32; down [rank][width] and up
 * [width][rank] are F32 (KQ_HIP_TYPE_F32, width and rank multiples of 4) or
 * packed rows of a matvec type. */
typedef struct kq_hip_gr_weights {
    const float *norm;
    uint32_t down_type;
    const void *down;
    uint32_t up_type;
    const void *up;
    const float *inject;
} kq_hip_gr_weights;

/* Device scratch of kq_hip_gr_read_f32 for `token_count` tokens. */
uint64_t kq_hip_gr_scratch_bytes(const kq_hip_gr_dimensions *dimensions, uint64_t token_count);

/* Replaces kq_layer_gr_read_f32 / kq_layer_gr_read_quantized_f32
 * (src/kq_layer_internal.h:81-92, src/kq_layer_qwen38.c:175-194):
 * branches [tokens][width] -> mixed [tokens][hidden] (the block input) and
 * write_gate [tokens][branch_count]. Fails with NUMERIC_DOMAIN on a
 * non-finite input, norm weight or result. */
kq_status kq_hip_gr_read_f32(kq_hip_context *context, const kq_hip_gr_dimensions *dimensions,
                             const kq_hip_gr_weights *weights, const float *device_branches,
                             uint64_t token_count, float *device_mixed,
                             float *device_write_gate, void *device_scratch,
                             uint64_t scratch_bytes, kq_diagnostic *diagnostic);

/* Replaces kq_layer_gr_write_f32 (src/kq_layer_internal.h:93-95,
 * src/kq_layer_qwen38.c:196-208): output[t][b][i] = branches[t][b][i] +
 * block_output[t][i] * write_gate[t][b], exact. output may be branches. */
kq_status kq_hip_gr_write_f32(kq_hip_context *context, const kq_hip_gr_dimensions *dimensions,
                              const float *device_branches, const float *device_block_output,
                              const float *device_write_gate, uint64_t token_count,
                              float *device_output, kq_diagnostic *diagnostic);

/* Device scratch of kq_hip_moe_block_f32 for `token_count` tokens. */
uint64_t kq_hip_moe_block_scratch_bytes(const kq_hip_gr_dimensions *dimensions,
                                        const kq_hip_moe_config *config,
                                        uint64_t token_count);

/* The MoE step of a layer with its gated residual (src/kq_layer.c:779-813):
 * mixed, write_gate = gr_read(branches); moe = MoE(mixed);
 * output = gr_write(branches, moe, write_gate). branches and output are
 * [tokens][width] and must not overlap; optional device_selected_ids
 * [tokens][top_k] receives the routing (4-byte aligned, overlapping neither
 * the branches, the output nor the scratch). */
kq_status kq_hip_moe_block_f32(kq_hip_context *context, const kq_hip_gr_dimensions *dimensions,
                               const kq_hip_gr_weights *gr_weights,
                               const kq_hip_moe_config *config,
                               const kq_hip_moe_weights *moe_weights,
                               const float *device_branches, uint64_t token_count,
                               float *device_output, uint32_t *device_selected_ids,
                               void *device_scratch, uint64_t scratch_bytes,
                               kq_diagnostic *diagnostic);

/* ------------------------------------------------------------------ */
/* Elementwise binary32 expf with the bits of the libm expf the reference
 * calls (src/kq_numeric.c:628-638, :776-813). No reference entry point of
 * its own; it exposes the device expf that the softmax uses so callers can
 * check it. */
kq_status kq_hip_f32_expf(kq_hip_context *context, const float *device_input,
                          uint64_t count, float *device_output,
                          kq_diagnostic *diagnostic);

/* ------------------------------------------------------------------ */
/* Token sampling on the device. Replaces include/kq_sampling.h (all of
 * it) and src/kq_sampling.c: the same policy, RNG state record and
 * result record, field for field; the same PCG-XSH-RR 64/32 stream and
 * integrity word; the same statuses in the same order; the same selected
 * id, RNG word and float bits. The logits and the scratch are device
 * memory; the RNG state and the result stay in host memory, and the state
 * advances only when a call succeeds. */

#define KQ_HIP_SAMPLING_QWEN38_VOCAB_SIZE UINT32_C(248320)
#define KQ_HIP_SAMPLING_QWEN38_CANONICAL_TOKEN_COUNT UINT32_C(248077)
#define KQ_HIP_SAMPLING_QWEN38_EOS_ID UINT32_C(248046)
#define KQ_HIP_SAMPLING_QWEN38_PAD_ID UINT32_C(248044)
#define KQ_HIP_SAMPLING_POLICY_VERSION UINT32_C(1)
#define KQ_HIP_SAMPLING_RNG_STATE_VERSION UINT32_C(1)
#define KQ_HIP_SAMPLING_DEFAULT_STREAM UINT64_C(0x4b515f53414d504c)
#define KQ_HIP_SAMPLING_MAX_STREAM UINT64_C(0x7fffffffffffffff)

typedef struct kq_hip_sampling_config kq_hip_sampling_config;

/* kq_sampling_policy (include/kq_sampling.h:23-30): top_k 0 keeps every
 * id; top_p 1 switches the nucleus cut off. */
typedef struct kq_hip_sampling_policy {
    uint32_t version;
    uint32_t flags;
    float temperature;
    float top_p;
    uint32_t top_k;
    uint32_t reserved[3];
} kq_hip_sampling_policy;

/* kq_sampling_rng_state (include/kq_sampling.h:32-41) */
typedef struct kq_hip_sampling_rng_state {
    uint32_t version;
    uint32_t reserved;
    uint64_t seed;
    uint64_t stream;
    uint64_t state;
    uint64_t increment;
    uint64_t draws;
    uint64_t integrity;
} kq_hip_sampling_rng_state;

/* kq_sampling_result (include/kq_sampling.h:43-55) */
typedef struct kq_hip_sampling_result {
    uint32_t selected_token_id;
    uint32_t top_k_retained_count;
    uint32_t retained_count;
    uint32_t rng_word;
    float selected_probability;
    float maximum_probability;
    float normalized_sum_f32;
    uint32_t reserved;
    double uniform_value;
    uint64_t rng_draws_before;
    uint64_t rng_draws_after;
} kq_hip_sampling_result;

/* kq_sampling_policy_qwen38_default (src/kq_sampling.c:161-170):
 * temperature 1, top-p 0.95, top-k 20. */
void kq_hip_sampling_policy_qwen38_default(kq_hip_sampling_policy *policy);

/* kq_sampling_config_open_qwen38 (src/kq_sampling.c:172-225): the policy
 * checks and statuses of the reference, for the model's 248,320-entry
 * vocabulary of which 248,077 ids are canonical. Looks up the device
 * sort's work size on the current HIP device (DEVICE_FAILURE without
 * one). */
kq_status kq_hip_sampling_config_open_qwen38(const kq_hip_sampling_policy *policy,
                                             kq_hip_sampling_config **output,
                                             kq_diagnostic *diagnostic);
/* The same for another vocabulary: 1 <= canonical_token_count <=
 * vocabulary_size <= 2^24, top_k <= vocabulary_size. No counterpart in
 * the reference, which fixes the model's vocabulary. */
kq_status kq_hip_sampling_config_open(const kq_hip_sampling_policy *policy,
                                      uint32_t vocabulary_size,
                                      uint32_t canonical_token_count,
                                      kq_hip_sampling_config **output,
                                      kq_diagnostic *diagnostic);
void kq_hip_sampling_config_close(kq_hip_sampling_config *config);
uint64_t kq_hip_sampling_config_owned_bytes(const kq_hip_sampling_config *config);
uint32_t kq_hip_sampling_config_vocabulary_size(const kq_hip_sampling_config *config);
/* Device scratch bytes a select call needs (kq_sampling_required_scratch_
 * bytes, src/kq_sampling.c:242-244, there host bytes): six arrays of
 * one entry per vocabulary id, two per 256 ids (finiteness flags and
 * maxima), the sort's work area and the device result record. 0 for an
 * invalid config. */
uint64_t kq_hip_sampling_required_scratch_bytes(const kq_hip_sampling_config *config);

/* The RNG record (src/kq_sampling.c:246-322): host functions, the same
 * statuses. */
kq_status kq_hip_sampling_rng_seed(uint64_t seed, uint64_t stream,
                                   kq_hip_sampling_rng_state *output,
                                   kq_diagnostic *diagnostic);
kq_status kq_hip_sampling_rng_reset(kq_hip_sampling_rng_state *state,
                                    kq_diagnostic *diagnostic);
kq_status kq_hip_sampling_rng_snapshot(const kq_hip_sampling_rng_state *state,
                                       kq_hip_sampling_rng_state *output,
                                       kq_diagnostic *diagnostic);
kq_status kq_hip_sampling_rng_import(const kq_hip_sampling_rng_state *snapshot,
                                     kq_hip_sampling_rng_state *output,
                                     kq_diagnostic *diagnostic);
kq_status kq_hip_sampling_rng_next_u32(kq_hip_sampling_rng_state *state, uint32_t *word,
                                       kq_diagnostic *diagnostic);

/* kq_sampling_select_f32 (src/kq_sampling.c:576-772) with device logits
 * [logit_count == the config's vocabulary] and device scratch of at least
 * kq_hip_sampling_required_scratch_bytes (any alignment; it must not
 * overlap the logits). Synchronous: returns once the result is on the
 * host. On success *state has advanced by one draw; on any failure
 * neither *state nor *result is written. */
kq_status kq_hip_sampling_select_f32(kq_hip_context *context,
                                     const kq_hip_sampling_config *config,
                                     kq_hip_sampling_rng_state *state,
                                     const float *device_logits, uint64_t logit_count,
                                     void *device_scratch, uint64_t scratch_bytes,
                                     kq_hip_sampling_result *result,
                                     kq_diagnostic *diagnostic);

/* The LM head and the sampler in one call, the logits never leaving the
 * device (the sampled counterpart of kq_hip_lm_head_greedy_f32, for one
 * hidden state): device_logits [vocab] receives W_lm h, then the sampler
 * runs on it as kq_hip_sampling_select_f32. vocab must equal the
 * config's vocabulary. */
kq_status kq_hip_lm_head_sample_f32(kq_hip_context *context,
                                    const kq_hip_sampling_config *config,
                                    kq_hip_sampling_rng_state *state,
                                    uint32_t type_id, const void *device_weights,
                                    uint64_t vocab, uint64_t columns,
                                    const float *device_hidden, float *device_logits,
                                    void *device_scratch, uint64_t scratch_bytes,
                                    kq_hip_sampling_result *result,
                                    kq_diagnostic *diagnostic);

/* kq_sampling_copy_work_for_test (src/kq_sampling.c:474-505): the last
 * select's processed logits (scores) and final probabilities by id, copied
 * from the device scratch to host arrays of output_capacity >= the
 * vocabulary entries each. */
kq_status kq_hip_sampling_copy_work(kq_hip_context *context,
                                    const kq_hip_sampling_config *config,
                                    const void *device_scratch, uint64_t scratch_bytes,
                                    float *scores, float *probabilities,
                                    uint64_t output_capacity, kq_diagnostic *diagnostic);

#ifdef __cplusplus
}
#endif

#endif
