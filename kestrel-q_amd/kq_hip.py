"""Python binding (ctypes) of the kq_hip C ABI, include/kq_hip.h.

Mirrors the reference's operator interface for the quantized-weight path:
dequantize / row dot / linear (matvec) / greedy argmax / LM head / MoE route
and execute, with the reference's status codes raised as KqError. Device
memory comes from the library's own allocator (kq_hip_malloc); numpy arrays
are uploaded and downloaded explicitly.

The shared library is built in-tree (kestrel-q_amd/_build/libkq_hip.so). If it
is missing, loading raises: there is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get("KQ_HIP_LIB", HERE / "_build" / "libkq_hip.so"))

TYPE_F32, TYPE_Q8_0, TYPE_Q4_K, TYPE_Q6_K = 0, 8, 12, 14
TYPE_Q5_1, TYPE_Q5_K, TYPE_IQ4_NL, TYPE_BF16 = 7, 13, 20, 30
TYPE_IDS = {"F32": TYPE_F32, "Q8_0": TYPE_Q8_0, "Q4_K": TYPE_Q4_K, "Q6_K": TYPE_Q6_K,
            "Q5_1": TYPE_Q5_1, "Q5_K": TYPE_Q5_K, "IQ4_NL": TYPE_IQ4_NL, "BF16": TYPE_BF16}
GEOMETRY = {TYPE_Q8_0: (32, 34), TYPE_Q4_K: (256, 144), TYPE_Q6_K: (256, 210),
            TYPE_Q5_1: (32, 24), TYPE_Q5_K: (256, 176), TYPE_IQ4_NL: (32, 18),
            TYPE_F32: (1, 4), TYPE_BF16: (1, 2)}

STATUS = {0: "OK", 1: "INVALID_ARGUMENT", 2: "OUT_OF_MEMORY", 3: "FILE_OPEN_FAILED",
          4: "FILE_SIZE_FAILED", 5: "FILE_MAP_FAILED", 6: "TRUNCATED", 7: "BAD_MAGIC",
          8: "UNSUPPORTED_VERSION", 9: "MALFORMED_METADATA", 10: "UNSUPPORTED_METADATA",
          11: "MALFORMED_TENSOR", 17: "DUPLICATE_METADATA", 18: "DUPLICATE_TENSOR",
          19: "INCONSISTENT_DATA_SECTION", 12: "UNSUPPORTED_TENSOR_TYPE",
          13: "ARITHMETIC_OVERFLOW", 14: "LIMIT_EXCEEDED", 15: "INVALID_ALIGNMENT",
          16: "SPAN_OUT_OF_RANGE", 25: "INVALID_QUANTIZED_GEOMETRY",
          26: "NONCONTIGUOUS_TENSOR_VIEW", 27: "TENSOR_LAYOUT_MISMATCH",
          28: "TENSOR_OWNERSHIP_MISMATCH", 31: "INVALID_TOKEN_ID", 32: "BUFFER_TOO_SMALL",
          38: "MALFORMED_QUANTIZED_DATA", 39: "NUMERIC_DOMAIN", 40: "DIMENSION_MISMATCH",
          41: "ALIASING_VIOLATION", 46: "INCOMPATIBLE_MOE", 54: "INCOMPATIBLE_SAMPLING",
          55: "INVALID_RNG_STATE", 1000: "DEVICE_FAILURE"}
CODES = {v: k for k, v in STATUS.items()}


class Diagnostic(C.Structure):
    _fields_ = [("status", C.c_int), ("message", C.c_char * 256)]


class Geometry(C.Structure):
    _fields_ = [("type_id", C.c_uint32), ("block_elements", C.c_uint64),
                ("bytes_per_block", C.c_uint64)]


class MoeDims(C.Structure):
    _fields_ = [("hidden_size", C.c_uint32), ("expert_count", C.c_uint32),
                ("top_k", C.c_uint32), ("routed_intermediate_size", C.c_uint32),
                ("shared_intermediate_size", C.c_uint32)]


class GrDims(C.Structure):
    _fields_ = [("branch_count", C.c_uint32), ("hidden_size", C.c_uint32),
                ("rank", C.c_uint32), ("rms_epsilon", C.c_float)]


class GrWeights(C.Structure):
    _fields_ = [("norm", C.c_void_p), ("down_type", C.c_uint32), ("down", C.c_void_p),
                ("up_type", C.c_uint32), ("up", C.c_void_p), ("inject", C.c_void_p)]


class MoeWeights(C.Structure):
    _fields_ = [("router", C.c_void_p),
                ("routed_gate_type", C.c_uint32), ("routed_gate", C.c_void_p),
                ("routed_up_type", C.c_uint32), ("routed_up", C.c_void_p),
                ("routed_down_type", C.c_uint32), ("routed_down", C.c_void_p),
                ("shared_gate_type", C.c_uint32), ("shared_gate", C.c_void_p),
                ("shared_up_type", C.c_uint32), ("shared_up", C.c_void_p),
                ("shared_down_type", C.c_uint32), ("shared_down", C.c_void_p),
                ("shared_gate_weight", C.c_void_p)]


class MoeWeightsF32(C.Structure):
    _fields_ = [(n, t) for role in ("router", "routed_gate", "routed_up", "routed_down",
                                    "shared_gate", "shared_up", "shared_down",
                                    "shared_gate_weight")
                for n, t in ((role, C.c_void_p), (role + "_count", C.c_uint64))]


class RoutedExpertWeightsF32(C.Structure):
    _fields_ = [(n, t) for role in ("gate", "up", "down")
                for n, t in ((role, C.c_void_p), (role + "_count", C.c_uint64))]


class MoeCheckpoint(C.Structure):
    _fields_ = [("kind", C.c_int), ("token_index", C.c_uint64), ("expert_id", C.c_uint32),
                ("top_k_position", C.c_uint32), ("rank", C.c_uint32),
                ("dimensions", C.c_uint64 * 2), ("values", C.POINTER(C.c_float)),
                ("value_count", C.c_uint64)]


class MoeRoute(C.Structure):
    _fields_ = [("token_index", C.c_uint64), ("router_logits", C.POINTER(C.c_float)),
                ("router_probabilities", C.POINTER(C.c_float)), ("expert_count", C.c_uint64),
                ("selected_expert_ids", C.POINTER(C.c_uint32)),
                ("selected_weights", C.POINTER(C.c_float)), ("selected_count", C.c_uint32)]


CHECKPOINT_OBSERVER = C.CFUNCTYPE(None, C.POINTER(MoeCheckpoint), C.c_void_p)
ROUTE_OBSERVER = C.CFUNCTYPE(None, C.POINTER(MoeRoute), C.c_void_p)
# kq_hip_moe_checkpoint_kind, in enum order
CHECKPOINT_KINDS = ("router_logits", "router_probabilities", "selected_weights", "routed_gate",
                    "routed_up", "routed_activated", "routed_expert_output",
                    "routed_weighted_output", "routed_weighted_sum", "shared_gate_projection",
                    "shared_up_projection", "shared_activated", "shared_output",
                    "shared_scale_logit", "shared_scale", "gated_shared_output",
                    "operator_output")


class QuantBlockSpan(C.Structure):
    _fields_ = [(n, C.c_uint64) for n in (
        "requested_element_offset", "requested_element_count", "first_block", "block_count",
        "physical_byte_offset", "physical_byte_length", "leading_elements",
        "trailing_elements")]


class TensorView(C.Structure):
    _fields_ = [("type_id", C.c_uint32), ("layout", C.c_uint32), ("block_elements", C.c_uint64),
                ("bytes_per_block", C.c_uint64), ("block_count", C.c_uint64),
                ("canonical_contiguous", C.c_uint32), ("reserved", C.c_uint32),
                ("device_data", C.c_void_p), ("mapped_bytes", C.c_uint64)]


LAYOUT_CANONICAL, LAYOUT_TRANSFORMED, LAYOUT_SPLIT, LAYOUT_FUSED = 0, 1, 2, 3
PHYSICAL_ORDER, CANONICAL_ORDER = 0, 1
GDN = {"none": 0, "qkv": 1, "gate": 2, "alpha": 3, "beta": 4, "conv": 5, "out": 6}


class SamplingPolicy(C.Structure):
    _fields_ = [("version", C.c_uint32), ("flags", C.c_uint32), ("temperature", C.c_float),
                ("top_p", C.c_float), ("top_k", C.c_uint32), ("reserved", C.c_uint32 * 3)]


class RngState(C.Structure):
    _fields_ = [("version", C.c_uint32), ("reserved", C.c_uint32)] + \
        [(n, C.c_uint64) for n in ("seed", "stream", "state", "increment", "draws", "integrity")]


class SamplingResult(C.Structure):
    _fields_ = [("selected_token_id", C.c_uint32), ("top_k_retained_count", C.c_uint32),
                ("retained_count", C.c_uint32), ("rng_word", C.c_uint32),
                ("selected_probability", C.c_float), ("maximum_probability", C.c_float),
                ("normalized_sum_f32", C.c_float), ("reserved", C.c_uint32),
                ("uniform_value", C.c_double), ("rng_draws_before", C.c_uint64),
                ("rng_draws_after", C.c_uint64)]


QWEN38_VOCAB, QWEN38_CANONICAL = 248320, 248077
SAMPLING_DEFAULT_STREAM = 0x4B515F53414D504C


class StringView(C.Structure):
    _fields_ = [("data", C.c_void_p), ("length", C.c_uint64)]

    def bytes(self) -> bytes:
        return C.string_at(self.data, self.length) if self.length else b""


class GgufTensor(C.Structure):
    _fields_ = [("name", StringView), ("rank", C.c_uint32), ("dimensions", C.c_uint64 * 8),
                ("type_id", C.c_uint32), ("block_elements", C.c_uint64),
                ("bytes_per_block", C.c_uint64), ("element_count", C.c_uint64),
                ("relative_offset", C.c_uint64), ("data_offset", C.c_uint64),
                ("packed_bytes", C.c_uint64)]


class GgufMetadata(C.Structure):
    _fields_ = [("key", StringView), ("value_type", C.c_uint32),
                ("array_element_type", C.c_uint32), ("array_length", C.c_uint64),
                ("scalar_value", C.c_uint64), ("string_value", StringView),
                ("array_data", StringView)]


class GgufTypeInfo(C.Structure):
    _fields_ = [("type_id", C.c_uint32), ("name", C.c_char_p), ("block_elements", C.c_uint64),
                ("bytes_per_block", C.c_uint64)]


class KqError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"{STATUS.get(status, status)}: {message}")
        self.status = status
        self.name = STATUS.get(status, str(status))


_P = C.c_void_p
_TP = C.POINTER(GgufTensor)
_MP = C.POINTER(GgufMetadata)

# Every function declared in include/kq_hip.h, kq_gguf.h, kq_file.h and
# kq_status.h.
SIGNATURES = {
    "kq_file_open_readonly": (C.c_int, [C.c_wchar_p, _P, _P]),
    "kq_file_open_readonly_utf8": (C.c_int, [C.c_char_p, _P, _P]),
    "kq_file_size": (C.c_uint64, [_P]),
    "kq_file_close": (None, [_P]),
    "kq_file_view_open": (C.c_int, [_P, C.c_uint64, C.c_uint64, _P, _P]),
    "kq_file_view_data": (_P, [_P]),
    "kq_file_view_offset": (C.c_uint64, [_P]),
    "kq_file_view_length": (C.c_uint64, [_P]),
    "kq_file_view_close": (None, [_P]),
    "kq_gguf_open": (C.c_int, [_P, _P, _P]),
    "kq_gguf_close": (None, [_P]),
    "kq_gguf_version": (C.c_uint32, [_P]),
    "kq_gguf_metadata_count": (C.c_uint64, [_P]),
    "kq_gguf_tensor_count": (C.c_uint64, [_P]),
    "kq_gguf_alignment": (C.c_uint64, [_P]),
    "kq_gguf_directory_end_offset": (C.c_uint64, [_P]),
    "kq_gguf_data_section_offset": (C.c_uint64, [_P]),
    "kq_gguf_packed_tensor_bytes": (C.c_uint64, [_P]),
    "kq_gguf_format_overhead_bytes": (C.c_uint64, [_P]),
    "kq_gguf_directory_bytes_parsed": (C.c_uint64, [_P]),
    "kq_gguf_payload_bytes_accessed": (C.c_uint64, [_P]),
    "kq_gguf_architecture": (StringView, [_P]),
    "kq_gguf_metadata_at": (_MP, [_P, C.c_uint64]),
    "kq_gguf_find_metadata": (_MP, [_P, C.c_char_p]),
    "kq_gguf_tensor_at": (_TP, [_P, C.c_uint64]),
    "kq_gguf_find_tensor": (_TP, [_P, C.c_char_p]),
    "kq_gguf_type_info_for": (C.POINTER(GgufTypeInfo), [C.c_uint32]),
    "kq_string_view_equal": (C.c_int, [_P, _P]),
    "kq_string_view_equal_cstr": (C.c_int, [_P, C.c_char_p]),
    "kq_gguf_metadata_u16": (C.c_int, [_MP, _P]),
    "kq_gguf_metadata_u32": (C.c_int, [_MP, _P]),
    "kq_gguf_metadata_i32": (C.c_int, [_MP, _P]),
    "kq_gguf_metadata_array_i32_at": (C.c_int, [_MP, C.c_uint64, _P]),
    "kq_gguf_metadata_array_u64_at": (C.c_int, [_MP, C.c_uint64, _P]),
    "kq_gguf_metadata_array_string_at": (C.c_int, [_MP, C.c_uint64, _P]),
    "kq_hip_gguf_expert_member": (C.c_int, [_TP, C.c_uint32, _P, _P, _P]),
    "kq_hip_gguf_upload_tensor": (C.c_int, [_P, _P, _TP, _P, C.c_uint64, _P]),
    "kq_hip_gguf_upload_expert_member": (C.c_int, [_P, _P, _TP, C.c_uint32, _P, C.c_uint64,
                                                    _P]),
    "kq_status_string": (C.c_char_p, [C.c_int]),
    "kq_diagnostic_clear": (None, [C.c_void_p]),
    "kq_hip_context_create": (C.c_int, [C.c_int, C.c_void_p, C.c_void_p]),
    "kq_hip_context_destroy": (None, [C.c_void_p]),
    "kq_hip_context_set_async": (C.c_int, [C.c_void_p, C.c_int, C.c_void_p]),
    "kq_hip_context_set_commit_on_success": (C.c_int, [C.c_void_p, C.c_int, C.c_void_p]),
    "kq_hip_context_synchronize": (C.c_int, [C.c_void_p, C.c_void_p]),
    "kq_hip_context_stream": (C.c_void_p, [C.c_void_p]),
    "kq_hip_malloc": (C.c_int, [C.c_void_p, C.c_uint64, C.c_void_p, C.c_void_p]),
    "kq_hip_free": (None, [C.c_void_p, C.c_void_p]),
    "kq_hip_upload": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint64, C.c_void_p]),
    "kq_hip_download": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint64, C.c_void_p]),
    "kq_hip_quant_geometry_for_type": (C.c_int, [C.c_uint32, C.c_void_p, C.c_void_p]),
    "kq_hip_quant_packed_size": (C.c_int, [C.c_uint32, C.c_uint64, C.c_void_p, C.c_void_p]),
    "kq_hip_expert_member_span": (C.c_int, [C.c_uint32, C.c_uint64, C.c_uint64, C.c_uint32,
                                            C.c_uint32, C.c_void_p, C.c_void_p, C.c_void_p]),
    "kq_hip_quant_element_to_block": (C.c_int, [C.c_uint32, C.c_uint64, C.c_uint64, C.c_void_p,
                                                C.c_void_p, C.c_void_p]),
    "kq_hip_quant_range_to_blocks": (C.c_int, [C.c_uint32, C.c_uint64, C.c_uint64, C.c_uint64,
                                               C.c_void_p, C.c_void_p]),
    "kq_hip_tensor_view_init": (C.c_int, [C.c_uint32, C.c_void_p, C.c_uint64, C.c_uint32,
                                          C.c_void_p, C.c_void_p]),
    "kq_hip_dequantize_view_blocks_f32": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint64,
                                                    C.c_uint64, C.c_uint32, C.c_void_p,
                                                    C.c_uint64, C.c_void_p, C.c_void_p]),
    "kq_hip_gdn_physical_row": (C.c_int, [C.c_uint32, C.c_uint64, C.c_uint64, C.c_void_p,
                                          C.c_void_p]),
    "kq_hip_gdn_physical_column": (C.c_int, [C.c_uint32, C.c_uint64, C.c_uint64, C.c_void_p,
                                             C.c_void_p]),
    "kq_hip_gdn_canonicalize": (C.c_int, [C.c_void_p, C.c_uint32, C.c_uint32, C.c_void_p,
                                          C.c_uint64, C.c_uint64, C.c_void_p, C.c_uint64,
                                          C.c_void_p]),
    "kq_hip_dequantize_blocks_f32": (C.c_int, [C.c_void_p, C.c_uint32, C.c_void_p, C.c_uint64,
                                               C.c_void_p, C.c_uint64, C.c_void_p, C.c_void_p]),
    "kq_hip_quantized_row_dot_f32": (C.c_int, [C.c_void_p, C.c_uint32, C.c_void_p, C.c_uint64,
                                               C.c_void_p, C.c_uint64, C.c_void_p, C.c_void_p]),
    "kq_hip_quantized_matvec_f32": (C.c_int, [C.c_void_p, C.c_uint32, C.c_void_p, C.c_uint64,
                                              C.c_uint64, C.c_void_p, C.c_uint32, C.c_void_p,
                                              C.c_uint64, C.c_void_p]),
    "kq_hip_greedy_argmax_f32": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint64, C.c_uint32,
                                           C.c_void_p, C.c_void_p]),
    "kq_hip_lm_head_greedy_f32": (C.c_int, [C.c_void_p, C.c_uint32, C.c_void_p, C.c_uint64,
                                            C.c_uint64, C.c_void_p, C.c_uint32, C.c_void_p,
                                            C.c_void_p, C.c_void_p]),
    "kq_hip_lm_head_greedy_f32_noalloc": (C.c_int, [C.c_void_p, C.c_uint32, C.c_void_p,
                                                    C.c_uint64, C.c_uint64, C.c_void_p,
                                                    C.c_uint32, C.c_void_p, C.c_void_p,
                                                    C.c_void_p]),
    "kq_hip_moe_config_create": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p]),
    "kq_hip_moe_config_close": (None, [C.c_void_p]),
    "kq_hip_moe_config_scratch_bytes": (C.c_uint64, [C.c_void_p, C.c_uint64]),
    "kq_hip_moe_route_f32": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint64,
                                       C.c_void_p, C.c_void_p, C.c_uint64,
                                       C.c_void_p, C.c_uint64, C.c_void_p, C.c_uint64,
                                       C.c_void_p, C.c_uint64, C.c_void_p, C.c_uint64,
                                       C.c_void_p, C.c_uint64, C.c_void_p]),
    "kq_hip_moe_config_one_expert_scratch_bytes": (C.c_uint64, [C.c_void_p]),
    "kq_hip_moe_execute_routed_expert_f32": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p,
                                                       C.c_uint32, C.c_void_p, C.c_void_p,
                                                       C.c_uint64, C.c_void_p, C.c_uint64,
                                                       C.c_void_p]),
    "kq_hip_moe_execute_quantized": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                               C.c_uint64, C.c_void_p, C.c_uint64, C.c_void_p,
                                               C.c_void_p, C.c_uint64, C.c_void_p]),
    "kq_hip_moe_config_f32_scratch_bytes": (C.c_uint64, [C.c_void_p, C.c_uint64]),
    "kq_hip_moe_execute_f32": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                         C.c_uint64, C.c_void_p, C.c_uint64, C.c_void_p,
                                         C.c_uint64, ROUTE_OBSERVER, CHECKPOINT_OBSERVER,
                                         C.c_void_p, C.c_void_p]),
    "kq_hip_moe_token_permutation": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint64,
                                               C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                               C.c_uint64, C.c_void_p]),
    "kq_hip_f32_expf": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint64, C.c_void_p, C.c_void_p]),
    "kq_hip_sampling_policy_qwen38_default": (None, [_P]),
    "kq_hip_sampling_config_open_qwen38": (C.c_int, [_P, _P, _P]),
    "kq_hip_sampling_config_open": (C.c_int, [_P, C.c_uint32, C.c_uint32, _P, _P]),
    "kq_hip_sampling_config_close": (None, [_P]),
    "kq_hip_sampling_config_owned_bytes": (C.c_uint64, [_P]),
    "kq_hip_sampling_config_vocabulary_size": (C.c_uint32, [_P]),
    "kq_hip_sampling_required_scratch_bytes": (C.c_uint64, [_P]),
    "kq_hip_sampling_rng_seed": (C.c_int, [C.c_uint64, C.c_uint64, _P, _P]),
    "kq_hip_sampling_rng_reset": (C.c_int, [_P, _P]),
    "kq_hip_sampling_rng_snapshot": (C.c_int, [_P, _P, _P]),
    "kq_hip_sampling_rng_import": (C.c_int, [_P, _P, _P]),
    "kq_hip_sampling_rng_next_u32": (C.c_int, [_P, _P, _P]),
    "kq_hip_sampling_select_f32": (C.c_int, [_P, _P, _P, _P, C.c_uint64, _P, C.c_uint64, _P,
                                             _P]),
    "kq_hip_lm_head_sample_f32": (C.c_int, [_P, _P, _P, C.c_uint32, _P, C.c_uint64, C.c_uint64,
                                            _P, _P, _P, C.c_uint64, _P, _P]),
    "kq_hip_sampling_copy_work": (C.c_int, [_P, _P, _P, C.c_uint64, _P, _P, C.c_uint64, _P]),
    "kq_hip_gr_scratch_bytes": (C.c_uint64, [C.c_void_p, C.c_uint64]),
    "kq_hip_gr_read_f32": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                     C.c_uint64, C.c_void_p, C.c_void_p, C.c_void_p,
                                     C.c_uint64, C.c_void_p]),
    "kq_hip_gr_write_f32": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                      C.c_void_p, C.c_uint64, C.c_void_p, C.c_void_p]),
    "kq_hip_moe_block_scratch_bytes": (C.c_uint64, [C.c_void_p, C.c_void_p, C.c_uint64]),
    "kq_hip_moe_block_f32": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                       C.c_void_p, C.c_void_p, C.c_uint64, C.c_void_p,
                                       C.c_void_p, C.c_void_p, C.c_uint64, C.c_void_p]),
}

_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"kq_hip library is not built: {LIB_PATH} "
                               "(run `make -C kestrel-q_amd` or __graft_entry__.build())")
        _lib = C.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(_lib, name)
            fn.restype = res
            fn.argtypes = args
    return _lib


def check(status: int, diag: Diagnostic) -> None:
    if status != 0:
        raise KqError(status, diag.message.decode(errors="replace"))


def geometry(type_id: int) -> tuple[int, int]:
    g, d = Geometry(), Diagnostic()
    check(lib().kq_hip_quant_geometry_for_type(type_id, C.byref(g), C.byref(d)), d)
    return g.block_elements, g.bytes_per_block


def packed_size(type_id: int, elements: int) -> int:
    out, d = C.c_uint64(), Diagnostic()
    check(lib().kq_hip_quant_packed_size(type_id, elements, C.byref(out), C.byref(d)), d)
    return out.value


def element_to_block(type_id: int, total: int, index: int) -> tuple[int, int]:
    b, w, d = C.c_uint64(), C.c_uint64(), Diagnostic()
    check(lib().kq_hip_quant_element_to_block(type_id, total, index, C.byref(b), C.byref(w),
                                              C.byref(d)), d)
    return b.value, w.value


def range_to_blocks(type_id: int, total: int, offset: int, count: int) -> QuantBlockSpan:
    sp, d = QuantBlockSpan(), Diagnostic()
    check(lib().kq_hip_quant_range_to_blocks(type_id, total, offset, count, C.byref(sp),
                                             C.byref(d)), d)
    return sp


def tensor_view(type_id: int, data, nbytes: int, layout: int = LAYOUT_CANONICAL) -> TensorView:
    v, d = TensorView(), Diagnostic()
    ptr = data.ptr if hasattr(data, "ptr") else data
    check(lib().kq_hip_tensor_view_init(type_id, C.c_void_p(ptr), nbytes, layout, C.byref(v),
                                        C.byref(d)), d)
    return v


def gdn_physical_index(layout: str, n: int, index: int, columns: bool = False) -> int:
    o, d = C.c_uint64(), Diagnostic()
    fn = lib().kq_hip_gdn_physical_column if columns else lib().kq_hip_gdn_physical_row
    check(fn(GDN[layout], n, index, C.byref(o), C.byref(d)), d)
    return o.value


def expert_member_span(type_id, rows, cols, experts, expert_id) -> tuple[int, int]:
    off, cnt, d = C.c_uint64(), C.c_uint64(), Diagnostic()
    check(lib().kq_hip_expert_member_span(type_id, rows, cols, experts, expert_id,
                                          C.byref(off), C.byref(cnt), C.byref(d)), d)
    return off.value, cnt.value


class DeviceBuffer:
    """Device allocation owned by a Context (freed with it or on close())."""

    def __init__(self, ctx: "Context", nbytes: int):
        self.ctx = ctx
        self.nbytes = int(nbytes)
        p, d = C.c_void_p(), Diagnostic()
        check(lib().kq_hip_malloc(ctx.handle, self.nbytes, C.byref(p), C.byref(d)), d)
        self.ptr = p.value

    def close(self) -> None:
        if self.ptr and self.ctx.handle:
            lib().kq_hip_free(self.ctx.handle, C.c_void_p(self.ptr))
        self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class MoeConfig:
    def __init__(self, hidden: int, experts: int, top_k: int, inter: int, shared_inter: int):
        self.dims = MoeDims(hidden, experts, top_k, inter, shared_inter)
        h, d = C.c_void_p(), Diagnostic()
        check(lib().kq_hip_moe_config_create(C.byref(self.dims), C.byref(h), C.byref(d)), d)
        self.handle = h.value
        self.hidden, self.experts, self.top_k = hidden, experts, top_k
        self.inter, self.shared_inter = inter, shared_inter

    def scratch_bytes(self, tokens: int) -> int:
        return lib().kq_hip_moe_config_scratch_bytes(C.c_void_p(self.handle), tokens)

    def one_expert_scratch_bytes(self) -> int:
        return lib().kq_hip_moe_config_one_expert_scratch_bytes(C.c_void_p(self.handle))

    def f32_scratch_bytes(self, tokens: int) -> int:
        return lib().kq_hip_moe_config_f32_scratch_bytes(C.c_void_p(self.handle), tokens)

    def close(self) -> None:
        if self.handle:
            lib().kq_hip_moe_config_close(C.c_void_p(self.handle))
        self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def sampling_policy(temperature: float = 1.0, top_p: float = 0.95, top_k: int = 20,
                    version: int = 1, flags: int = 0, reserved=(0, 0, 0)) -> SamplingPolicy:
    p = SamplingPolicy()
    p.version, p.flags, p.temperature, p.top_p, p.top_k = version, flags, temperature, top_p, top_k
    for i, r in enumerate(reserved):
        p.reserved[i] = r
    return p


def default_policy() -> SamplingPolicy:
    p = SamplingPolicy()
    lib().kq_hip_sampling_policy_qwen38_default(C.byref(p))
    return p


def rng_seed(seed: int, stream: int = SAMPLING_DEFAULT_STREAM) -> RngState:
    st, d = RngState(), Diagnostic()
    check(lib().kq_hip_sampling_rng_seed(seed, stream, C.byref(st), C.byref(d)), d)
    return st


def rng_next(state: RngState) -> int:
    w, d = C.c_uint32(), Diagnostic()
    check(lib().kq_hip_sampling_rng_next_u32(C.byref(state), C.byref(w), C.byref(d)), d)
    return w.value


class SamplingConfig:
    """kq_hip_sampling_config: the model's vocabulary by default, or another
    (vocabulary, canonical) pair."""

    def __init__(self, policy: SamplingPolicy, vocabulary: int | None = None,
                 canonical: int | None = None):
        h, d = C.c_void_p(), Diagnostic()
        if vocabulary is None:
            check(lib().kq_hip_sampling_config_open_qwen38(C.byref(policy), C.byref(h),
                                                           C.byref(d)), d)
        else:
            check(lib().kq_hip_sampling_config_open(C.byref(policy), vocabulary, canonical,
                                                    C.byref(h), C.byref(d)), d)
        self.handle = h.value
        self.vocabulary = lib().kq_hip_sampling_config_vocabulary_size(C.c_void_p(self.handle))
        self.scratch_bytes = lib().kq_hip_sampling_required_scratch_bytes(
            C.c_void_p(self.handle))

    def close(self) -> None:
        if self.handle:
            lib().kq_hip_sampling_config_close(C.c_void_p(self.handle))
        self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Context:
    def __init__(self, device: int = 0):
        h, d = C.c_void_p(), Diagnostic()
        check(lib().kq_hip_context_create(device, C.byref(h), C.byref(d)), d)
        self.handle = h.value
        self._buffers: list[DeviceBuffer] = []

    # ---- lifetime / memory ----
    def close(self) -> None:
        for b in self._buffers:
            b.close()
        self._buffers.clear()
        if self.handle:
            lib().kq_hip_context_destroy(C.c_void_p(self.handle))
        self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @property
    def stream(self) -> int:
        return lib().kq_hip_context_stream(C.c_void_p(self.handle))

    def set_async(self, on: bool) -> None:
        d = Diagnostic()
        check(lib().kq_hip_context_set_async(C.c_void_p(self.handle), int(on), C.byref(d)), d)

    def set_commit_on_success(self, on: bool) -> None:
        d = Diagnostic()
        check(lib().kq_hip_context_set_commit_on_success(C.c_void_p(self.handle), int(on),
                                                         C.byref(d)), d)

    def synchronize(self) -> None:
        d = Diagnostic()
        check(lib().kq_hip_context_synchronize(C.c_void_p(self.handle), C.byref(d)), d)

    def alloc(self, nbytes: int) -> DeviceBuffer:
        b = DeviceBuffer(self, max(int(nbytes), 1))
        self._buffers.append(b)
        return b

    def upload(self, arr: np.ndarray, pad: int = 0) -> DeviceBuffer:
        arr = np.ascontiguousarray(arr)
        b = self.alloc(arr.nbytes + pad)
        d = Diagnostic()
        check(lib().kq_hip_upload(C.c_void_p(self.handle), C.c_void_p(b.ptr),
                                  arr.ctypes.data, arr.nbytes, C.byref(d)), d)
        return b

    def download(self, ptr, dtype, count: int) -> np.ndarray:
        out = np.empty(int(count), dtype=dtype)
        d = Diagnostic()
        src = ptr.ptr if isinstance(ptr, DeviceBuffer) else ptr
        check(lib().kq_hip_download(C.c_void_p(self.handle), out.ctypes.data, C.c_void_p(src),
                                    out.nbytes, C.byref(d)), d)
        return out

    # ---- numeric ----
    @property
    def _h(self) -> C.c_void_p:
        return C.c_void_p(self.handle)

    @staticmethod
    def _p(x) -> C.c_void_p:
        return C.c_void_p(x.ptr if isinstance(x, DeviceBuffer) else x)

    def dequantize(self, type_id: int, packed, packed_bytes: int, out, capacity: int) -> int:
        cnt, d = C.c_uint64(), Diagnostic()
        check(lib().kq_hip_dequantize_blocks_f32(self._h, type_id, self._p(packed),
                                                 packed_bytes, self._p(out), capacity,
                                                 C.byref(cnt), C.byref(d)), d)
        return cnt.value

    def dequantize_view(self, view: TensorView, first: int, count: int, order: int, out,
                        capacity: int) -> int:
        cnt, d = C.c_uint64(), Diagnostic()
        check(lib().kq_hip_dequantize_view_blocks_f32(self._h, C.byref(view), first, count, order,
                                                      self._p(out), capacity, C.byref(cnt),
                                                      C.byref(d)), d)
        return cnt.value

    def gdn_canonicalize(self, layout: str, type_id: int, phys, rows: int, cols: int, canon,
                         capacity: int) -> None:
        d = Diagnostic()
        check(lib().kq_hip_gdn_canonicalize(self._h, GDN[layout], type_id, self._p(phys), rows,
                                            cols, self._p(canon), capacity, C.byref(d)), d)

    def row_dot(self, type_id: int, packed, packed_bytes: int, x, count: int, out) -> None:
        d = Diagnostic()
        check(lib().kq_hip_quantized_row_dot_f32(self._h, type_id, self._p(packed),
                                                 packed_bytes, self._p(x), count, self._p(out),
                                                 C.byref(d)), d)

    def matvec(self, type_id: int, w, rows: int, cols: int, x, batch: int, y,
               capacity: int | None = None) -> None:
        d = Diagnostic()
        cap = rows * batch if capacity is None else capacity
        check(lib().kq_hip_quantized_matvec_f32(self._h, type_id, self._p(w), rows, cols,
                                                self._p(x), batch, self._p(y), cap,
                                                C.byref(d)), d)

    def argmax(self, logits, count: int, batch: int, ids) -> None:
        d = Diagnostic()
        check(lib().kq_hip_greedy_argmax_f32(self._h, self._p(logits), count, batch,
                                             self._p(ids), C.byref(d)), d)

    def lm_head(self, type_id: int, w, vocab: int, cols: int, h, batch: int, logits, ids,
                noalloc: bool = False) -> None:
        d = Diagnostic()
        fn = lib().kq_hip_lm_head_greedy_f32_noalloc if noalloc else \
            lib().kq_hip_lm_head_greedy_f32
        check(fn(self._h, type_id, self._p(w), vocab, cols, self._p(h), batch, self._p(logits),
                 self._p(ids), C.byref(d)), d)

    def sample(self, cfg: SamplingConfig, state: RngState, logits, scratch,
               scratch_bytes: int | None = None) -> SamplingResult:
        r, d = SamplingResult(), Diagnostic()
        nb = cfg.scratch_bytes if scratch_bytes is None else scratch_bytes
        check(lib().kq_hip_sampling_select_f32(self._h, C.c_void_p(cfg.handle), C.byref(state),
                                               self._p(logits), cfg.vocabulary,
                                               self._p(scratch), nb, C.byref(r), C.byref(d)), d)
        return r

    def lm_head_sample(self, cfg: SamplingConfig, state: RngState, type_id: int, w, vocab: int,
                       cols: int, h, logits, scratch) -> SamplingResult:
        r, d = SamplingResult(), Diagnostic()
        check(lib().kq_hip_lm_head_sample_f32(self._h, C.c_void_p(cfg.handle), C.byref(state),
                                              type_id, self._p(w), vocab, cols, self._p(h),
                                              self._p(logits), self._p(scratch),
                                              cfg.scratch_bytes, C.byref(r), C.byref(d)), d)
        return r

    def sampling_work(self, cfg: SamplingConfig, scratch) -> tuple[np.ndarray, np.ndarray]:
        sc = np.empty(cfg.vocabulary, np.float32)
        pr = np.empty(cfg.vocabulary, np.float32)
        d = Diagnostic()
        check(lib().kq_hip_sampling_copy_work(self._h, C.c_void_p(cfg.handle), self._p(scratch),
                                              cfg.scratch_bytes, sc.ctypes.data, pr.ctypes.data,
                                              cfg.vocabulary, C.byref(d)), d)
        return sc, pr

    def expf(self, x, count: int, out) -> None:
        d = Diagnostic()
        check(lib().kq_hip_f32_expf(self._h, self._p(x), count, self._p(out), C.byref(d)), d)

    # ---- MoE ----
    def moe_route(self, cfg: MoeConfig, router, shared_gate_weight, hidden, tokens: int,
                  logits, probs, ids, weights, scratch, scratch_bytes: int,
                  router_count: int | None = None, caps: tuple | None = None) -> None:
        """caps: (logits, probabilities, ids, weights) capacities in values;
        by default exactly what the tokens need."""
        d = Diagnostic()
        ne, nk = tokens * cfg.experts, tokens * cfg.top_k
        cl, cp, ci, cw = caps if caps is not None else (ne, ne, nk, nk)
        rc = cfg.experts * cfg.hidden if router_count is None else router_count
        check(lib().kq_hip_moe_route_f32(self._h, C.c_void_p(cfg.handle), self._p(router), rc,
                                         self._p(shared_gate_weight), self._p(hidden), tokens,
                                         self._p(logits), cl, self._p(probs), cp,
                                         self._p(ids), ci, self._p(weights), cw,
                                         self._p(scratch), scratch_bytes, C.byref(d)), d)

    def moe_routed_expert_f32(self, cfg: MoeConfig, gate, up, down, expert_id: int, hidden,
                              out, scratch, scratch_bytes: int, capacity: int | None = None,
                              counts: tuple | None = None) -> None:
        """One routed expert on F32 member matrices (device pointers);
        counts: (gate, up, down) element counts, by default the config's."""
        d = Diagnostic()
        m = cfg.inter * cfg.hidden
        gc, uc, dc = counts if counts is not None else (m, m, m)
        w = RoutedExpertWeightsF32(self._p(gate), gc, self._p(up), uc, self._p(down), dc)
        cap = cfg.hidden if capacity is None else capacity
        check(lib().kq_hip_moe_execute_routed_expert_f32(
            self._h, C.c_void_p(cfg.handle), C.byref(w), expert_id, self._p(hidden),
            self._p(out), cap, self._p(scratch), scratch_bytes, C.byref(d)), d)

    def moe_execute(self, cfg: MoeConfig, weights: MoeWeights, hidden, tokens: int, out,
                    ids, scratch, scratch_bytes: int, capacity: int | None = None) -> None:
        d = Diagnostic()
        cap = tokens * cfg.hidden if capacity is None else capacity
        check(lib().kq_hip_moe_execute_quantized(self._h, C.c_void_p(cfg.handle),
                                                 C.byref(weights), self._p(hidden), tokens,
                                                 self._p(out), cap,
                                                 self._p(ids) if ids is not None else None,
                                                 self._p(scratch), scratch_bytes, C.byref(d)), d)

    def moe_execute_f32(self, cfg: MoeConfig, weights: MoeWeightsF32, hidden, tokens: int, out,
                        scratch, scratch_bytes: int, capacity: int | None = None,
                        observe: bool = False):
        """F32 weights in the reference's order. observe: collect the route
        observer's and checkpoint observer's calls, in call order, as
        ("route", dict) / ("checkpoint", dict) with copied values."""
        d = Diagnostic()
        cap = tokens * cfg.hidden if capacity is None else capacity
        seen = []

        def on_route(r, _u):
            r = r.contents
            n, k = r.expert_count, r.selected_count
            seen.append(("route", {
                "token": r.token_index,
                "logits": np.ctypeslib.as_array(r.router_logits, (n,)).copy(),
                "probs": np.ctypeslib.as_array(r.router_probabilities, (n,)).copy(),
                "ids": np.ctypeslib.as_array(r.selected_expert_ids, (k,)).copy(),
                "weights": np.ctypeslib.as_array(r.selected_weights, (k,)).copy()}))

        def on_ckpt(c, _u):
            c = c.contents
            seen.append(("checkpoint", {
                "kind": CHECKPOINT_KINDS[c.kind], "token": c.token_index,
                "expert": c.expert_id, "position": c.top_k_position, "rank": c.rank,
                "dims": (c.dimensions[0], c.dimensions[1]),
                "values": np.ctypeslib.as_array(c.values, (c.value_count,)).copy()}))
        ro = ROUTE_OBSERVER(on_route) if observe else ROUTE_OBSERVER()
        co = CHECKPOINT_OBSERVER(on_ckpt) if observe else CHECKPOINT_OBSERVER()
        check(lib().kq_hip_moe_execute_f32(self._h, C.c_void_p(cfg.handle), C.byref(weights),
                                           self._p(hidden), tokens, self._p(out), cap,
                                           self._p(scratch), scratch_bytes, ro, co, None,
                                           C.byref(d)), d)
        return seen

    def gr_read(self, dims: GrDims, weights: GrWeights, x, tokens: int, mixed, write_gate,
                scratch, scratch_bytes: int) -> None:
        d = Diagnostic()
        check(lib().kq_hip_gr_read_f32(self._h, C.byref(dims), C.byref(weights), self._p(x),
                                       tokens, self._p(mixed), self._p(write_gate),
                                       self._p(scratch), scratch_bytes, C.byref(d)), d)

    def gr_write(self, dims: GrDims, x, block_output, write_gate, tokens: int, out) -> None:
        d = Diagnostic()
        check(lib().kq_hip_gr_write_f32(self._h, C.byref(dims), self._p(x),
                                        self._p(block_output), self._p(write_gate), tokens,
                                        self._p(out), C.byref(d)), d)

    def moe_block(self, dims: GrDims, gr: GrWeights, cfg: MoeConfig, moe: MoeWeights, x,
                  tokens: int, out, ids, scratch, scratch_bytes: int) -> None:
        d = Diagnostic()
        check(lib().kq_hip_moe_block_f32(self._h, C.byref(dims), C.byref(gr),
                                         C.c_void_p(cfg.handle), C.byref(moe), self._p(x),
                                         tokens, self._p(out),
                                         self._p(ids) if ids is not None else None,
                                         self._p(scratch), scratch_bytes, C.byref(d)), d)

    def moe_permutation(self, cfg: MoeConfig, ids, tokens: int, offsets, pair_token, pair_slot,
                        scratch, scratch_bytes: int) -> None:
        d = Diagnostic()
        check(lib().kq_hip_moe_token_permutation(self._h, C.c_void_p(cfg.handle), self._p(ids),
                                                 tokens, self._p(offsets), self._p(pair_token),
                                                 self._p(pair_slot), self._p(scratch),
                                                 scratch_bytes, C.byref(d)), d)


def moe_weights(bufs: dict, gate_type=TYPE_Q4_K, down_type=TYPE_Q6_K,
                shared_gate_type=None, shared_down_type=None) -> MoeWeights:
    """bufs: role -> DeviceBuffer (router, gate, up, down, shared_gate,
    shared_up, shared_down, shared_gate_weight). The shared expert takes the
    routed types unless given."""
    P = lambda k: C.c_void_p(bufs[k].ptr)
    sg = gate_type if shared_gate_type is None else shared_gate_type
    sd = down_type if shared_down_type is None else shared_down_type
    return MoeWeights(P("router"), gate_type, P("gate"), gate_type, P("up"), down_type,
                      P("down"), sg, P("shared_gate"), sg, P("shared_up"),
                      sd, P("shared_down"), P("shared_gate_weight"))


def moe_weights_f32(bufs: dict, counts: dict) -> MoeWeightsF32:
    """bufs: role -> DeviceBuffer, counts: role -> element count, roles as
    kq_hip_moe_weights_f32 (router, routed_gate, routed_up, routed_down,
    shared_gate, shared_up, shared_down, shared_gate_weight)."""
    w = MoeWeightsF32()
    for role in ("router", "routed_gate", "routed_up", "routed_down", "shared_gate",
                 "shared_up", "shared_down", "shared_gate_weight"):
        setattr(w, role, bufs[role].ptr if bufs.get(role) is not None else None)
        setattr(w, role + "_count", counts[role])
    return w


# ---------------------------------------------------------------- GGUF files


class File:
    """A read-only file (include/kq_file.h); views copy their bytes out."""

    def __init__(self, path, wide: bool = False):
        h, d = C.c_void_p(), Diagnostic()
        if wide:
            st = lib().kq_file_open_readonly(str(path), C.byref(h), C.byref(d))
        else:
            st = lib().kq_file_open_readonly_utf8(os.fsencode(path), C.byref(h), C.byref(d))
        check(st, d)
        self.handle = h.value

    @property
    def size(self) -> int:
        return lib().kq_file_size(C.c_void_p(self.handle))

    def view(self, offset: int, length: int) -> tuple[int, int, bytes]:
        """(offset, length, bytes) of a mapped view, closed before returning."""
        v, d = C.c_void_p(), Diagnostic()
        check(lib().kq_file_view_open(C.c_void_p(self.handle), offset, length, C.byref(v),
                                      C.byref(d)), d)
        try:
            L = lib()
            return (L.kq_file_view_offset(v), L.kq_file_view_length(v),
                    C.string_at(L.kq_file_view_data(v), L.kq_file_view_length(v)))
        finally:
            lib().kq_file_view_close(v)

    def close(self) -> None:
        if self.handle:
            lib().kq_file_close(C.c_void_p(self.handle))
        self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


class Gguf:
    """A parsed GGUF v3 file (include/kq_gguf.h). Tensor descriptors are
    ctypes pointers into the parser's own array (they stay valid until
    close()); upload_* copy their packed bytes to device memory."""

    def __init__(self, path, wide: bool = False):
        self.file = File(path, wide)
        h, d = C.c_void_p(), Diagnostic()
        st = lib().kq_gguf_open(C.c_void_p(self.file.handle), C.byref(h), C.byref(d))
        if st != 0:
            self.file.close()
            check(st, d)
        self.handle = h.value

    def _g(self):
        return C.c_void_p(self.handle)

    def close(self) -> None:
        if getattr(self, "handle", None):
            lib().kq_gguf_close(self._g())
        self.handle = None
        self.file.close()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def info(self) -> dict:
        L, g = lib(), self._g()
        return {"version": L.kq_gguf_version(g), "metadata_count": L.kq_gguf_metadata_count(g),
                "tensor_count": L.kq_gguf_tensor_count(g), "alignment": L.kq_gguf_alignment(g),
                "directory_end": L.kq_gguf_directory_end_offset(g),
                "data_section": L.kq_gguf_data_section_offset(g),
                "packed_bytes": L.kq_gguf_packed_tensor_bytes(g),
                "overhead_bytes": L.kq_gguf_format_overhead_bytes(g),
                "bytes_parsed": L.kq_gguf_directory_bytes_parsed(g),
                "payload_bytes_accessed": L.kq_gguf_payload_bytes_accessed(g),
                "architecture": L.kq_gguf_architecture(g).bytes().decode()}

    def tensor_at(self, index: int):
        p = lib().kq_gguf_tensor_at(self._g(), index)
        return p if p else None

    def tensor(self, name: str):
        p = lib().kq_gguf_find_tensor(self._g(), name.encode())
        return p if p else None

    def metadata_at(self, index: int):
        p = lib().kq_gguf_metadata_at(self._g(), index)
        return p if p else None

    def metadata(self, key: str):
        p = lib().kq_gguf_find_metadata(self._g(), key.encode())
        return p if p else None

    @staticmethod
    def scalar(meta, kind: str):
        """kind: u16 / u32 / i32; None when absent or of another type."""
        ct = {"u16": C.c_uint16, "u32": C.c_uint32, "i32": C.c_int32}[kind]
        out = ct()
        fn = getattr(lib(), f"kq_gguf_metadata_{kind}")
        return out.value if meta is not None and fn(meta, C.byref(out)) else None

    @staticmethod
    def array_item(meta, kind: str, index: int):
        """kind: i32 / u64 / string; None when out of range or of another type."""
        if kind == "string":
            out = StringView()
        else:
            out = {"i32": C.c_int32, "u64": C.c_uint64}[kind]()
        fn = getattr(lib(), f"kq_gguf_metadata_array_{kind}_at")
        if meta is None or not fn(meta, index, C.byref(out)):
            return None
        return out.bytes() if kind == "string" else out.value

    def upload_tensor(self, ctx: Context, tensor, dst, capacity: int) -> None:
        d = Diagnostic()
        check(lib().kq_hip_gguf_upload_tensor(ctx._h, self._g(), tensor, Context._p(dst),
                                              capacity, C.byref(d)), d)

    def upload_expert(self, ctx: Context, tensor, expert_id: int, dst, capacity: int) -> None:
        d = Diagnostic()
        check(lib().kq_hip_gguf_upload_expert_member(ctx._h, self._g(), tensor, expert_id,
                                                     Context._p(dst), capacity, C.byref(d)), d)


def gguf_expert_member(tensor, expert_id: int) -> tuple[int, int]:
    off, cnt, d = C.c_uint64(), C.c_uint64(), Diagnostic()
    check(lib().kq_hip_gguf_expert_member(tensor, expert_id, C.byref(off), C.byref(cnt),
                                          C.byref(d)), d)
    return off.value, cnt.value


def gguf_type_info(type_id: int):
    p = lib().kq_gguf_type_info_for(type_id)
    if not p:
        return None
    t = p.contents
    return t.name.decode(), t.block_elements, t.bytes_per_block


def gr_dims(branches: int, hidden: int, rank: int, eps: float = 1.0e-6) -> GrDims:
    return GrDims(branches, hidden, rank, eps)


def gr_scratch_bytes(dims: GrDims, tokens: int) -> int:
    return lib().kq_hip_gr_scratch_bytes(C.byref(dims), tokens)


def moe_block_scratch_bytes(dims: GrDims, cfg: MoeConfig, tokens: int) -> int:
    return lib().kq_hip_moe_block_scratch_bytes(C.byref(dims), C.c_void_p(cfg.handle), tokens)


def gr_weights(bufs: dict, down_type: int, up_type: int) -> GrWeights:
    """bufs: norm, down, up, inject -> DeviceBuffer."""
    return GrWeights(bufs["norm"].ptr, down_type, bufs["down"].ptr, up_type, bufs["up"].ptr,
                     bufs["inject"].ptr)
