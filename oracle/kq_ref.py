"""ctypes binding to the reference library built from its own sources.

TEST INFRASTRUCTURE ONLY: `make -C oracle ref` compiles the reference's
src/kq_status.c, kq_numeric.c, kq_tensor_view.c, kq_gguf.c, kq_model.c,
kq_moe.c and kq_moe_qwen38.c (C17, -fno-fast-math -ffp-contract=off, as in
the reference's CMakeLists.txt:104-117) into oracle/_ref/libkq_ref.so. The
Win32 file layer and weight provider are not part of it, so the library is
opened with lazy binding; none of the functions bound here reach them.

Used only by tests/test_oracle_vs_reference.py to check the oracle
(kq_oracle.c) against the reference's own code on the same inputs.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "_ref" / "libkq_ref.so"

_lib = None


class Diagnostic(C.Structure):
    # include/kq_status.h:69-74
    _fields_ = [("status", C.c_int), ("message", C.c_char * 256)]


class MoeDims(C.Structure):
    # src/kq_moe_internal.h:10-17
    _fields_ = [("hidden_size", C.c_uint32), ("expert_count", C.c_uint32),
                ("top_k", C.c_uint32), ("routed_intermediate_size", C.c_uint32),
                ("shared_intermediate_size", C.c_uint32), ("activation_dtype", C.c_int)]


class MoeWeightsF32(C.Structure):
    # include/kq_moe.h:72-89
    _fields_ = [(n, t) for role in ("router", "routed_gate", "routed_up", "routed_down",
                                    "shared_gate", "shared_up", "shared_down",
                                    "shared_gate_weight")
                for n, t in ((role, C.c_void_p), (role + "_count", C.c_uint64))]


class RoutedExpertWeightsF32(C.Structure):
    # include/kq_moe.h:91-98
    _fields_ = [(n, t) for role in ("gate", "up", "down")
                for n, t in ((role, C.c_void_p), (role + "_count", C.c_uint64))]


class QuantBlockSpan(C.Structure):
    # include/kq_tensor_view.h:39-48
    _fields_ = [(n, C.c_uint64) for n in (
        "requested_element_offset", "requested_element_count", "first_block", "block_count",
        "physical_byte_offset", "physical_byte_length", "leading_elements",
        "trailing_elements")]


class RefError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"reference status {status}: {message}")
        self.status = status


def available() -> bool:
    return LIB_PATH.exists()


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise FileNotFoundError(f"{LIB_PATH} not built (make -C oracle ref)")
        l = C.CDLL(str(LIB_PATH), mode=os.RTLD_LAZY | os.RTLD_LOCAL)
        vp, u64, u32, f32 = C.c_void_p, C.c_uint64, C.c_uint32, C.c_float
        dp = C.POINTER(Diagnostic)
        sig = {
            "kq_dequantize_blocks_f32": [u32, vp, u64, vp, u64, C.POINTER(u64), dp],
            "kq_quantized_row_dot_f32": [u32, vp, u64, vp, u64, vp, dp],
            "kq_f32_add": [vp, vp, u64, vp, dp],
            "kq_f32_multiply": [vp, vp, u64, vp, dp],
            "kq_f32_scale": [vp, u64, f32, vp, dp],
            "kq_f32_dot": [vp, vp, u64, vp, dp],
            "kq_f32_sigmoid": [vp, u64, vp, dp],
            "kq_f32_silu": [vp, u64, vp, dp],
            "kq_f32_swiglu": [vp, vp, u64, vp, dp],
            "kq_f32_rms_norm": [vp, vp, u64, f32, vp, dp],
            "kq_f32_softmax": [vp, u64, vp, dp],
            "kq_f32_stable_top_k": [vp, u64, u32, vp, vp, u64, dp],
            "kq_moe_test_config_create": [C.POINTER(MoeDims), C.POINTER(vp), dp],
            "kq_moe_config_scratch_bytes": [vp],
            "kq_moe_route_f32": [vp, vp, u64, vp, vp, u64, vp, u64, vp, u64, vp, u64, dp],
            "kq_moe_execute_f32": [vp, C.POINTER(MoeWeightsF32), vp, u64, vp, u64, vp, u64,
                                   vp, vp, vp, dp],
            "kq_moe_execute_routed_expert_f32": [vp, C.POINTER(RoutedExpertWeightsF32), u32, vp,
                                                 vp, u64, vp, u64, dp],
            "kq_quant_element_to_block": [u32, u64, u64, C.POINTER(u64), C.POINTER(u64), dp],
            "kq_quant_range_to_blocks": [u32, u64, u64, u64, C.POINTER(QuantBlockSpan), dp],
        }
        for name, args in sig.items():
            fn = getattr(l, name)
            fn.argtypes = args
            fn.restype = C.c_int
        l.kq_moe_config_scratch_bytes.restype = C.c_uint64
        l.kq_moe_config_one_expert_workspace_bytes.argtypes = [vp]
        l.kq_moe_config_one_expert_workspace_bytes.restype = C.c_uint64
        l.kq_moe_config_close.argtypes = [vp]
        l.kq_moe_config_close.restype = None
        _lib = l
    return _lib


def _p(a: np.ndarray) -> int:
    return a.ctypes.data


def _check(st: int, d: Diagnostic) -> None:
    if st != 0:
        raise RefError(st, d.message.decode(errors="replace"))


def element_to_block(type_id: int, total: int, index: int):
    """(status, block, within) from the reference's kq_quant_element_to_block."""
    b, w, d = C.c_uint64(), C.c_uint64(), Diagnostic()
    st = lib().kq_quant_element_to_block(type_id, total, index, C.byref(b), C.byref(w),
                                         C.byref(d))
    return st, b.value, w.value


def range_to_blocks(type_id: int, total: int, offset: int, count: int):
    """(status, span fields) from the reference's kq_quant_range_to_blocks."""
    sp, d = QuantBlockSpan(), Diagnostic()
    st = lib().kq_quant_range_to_blocks(type_id, total, offset, count, C.byref(sp), C.byref(d))
    return st, tuple(getattr(sp, n) for n, _ in QuantBlockSpan._fields_)


def dequantize(type_id: int, packed: np.ndarray, elements: int) -> np.ndarray:
    packed = np.ascontiguousarray(packed).view(np.uint8)
    out = np.empty(elements, np.float32)
    n = C.c_uint64()
    d = Diagnostic()
    _check(lib().kq_dequantize_blocks_f32(type_id, _p(packed), packed.nbytes, _p(out),
                                          elements, C.byref(n), C.byref(d)), d)
    return out[: n.value]


def row_dot(type_id: int, packed: np.ndarray, x: np.ndarray) -> float:
    packed = np.ascontiguousarray(packed).view(np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.zeros(1, np.float32)
    d = Diagnostic()
    _check(lib().kq_quantized_row_dot_f32(type_id, _p(packed), packed.nbytes, _p(x), x.size,
                                          _p(out), C.byref(d)), d)
    return out


def unary(name: str, a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty_like(a)
    d = Diagnostic()
    _check(getattr(lib(), "kq_f32_" + name)(_p(a), a.size, _p(out), C.byref(d)), d)
    return out


def binary(name: str, a: np.ndarray, b: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    out = np.empty_like(a)
    d = Diagnostic()
    _check(getattr(lib(), "kq_f32_" + name)(_p(a), _p(b), a.size, _p(out), C.byref(d)), d)
    return out


def scale(a: np.ndarray, s: float) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty_like(a)
    d = Diagnostic()
    _check(lib().kq_f32_scale(_p(a), a.size, s, _p(out), C.byref(d)), d)
    return out


def dot(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    out = np.zeros(1, np.float32)
    d = Diagnostic()
    _check(lib().kq_f32_dot(_p(a), _p(b), a.size, _p(out), C.byref(d)), d)
    return out


def rms_norm(a: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    out = np.empty_like(a)
    d = Diagnostic()
    _check(lib().kq_f32_rms_norm(_p(a), _p(w), a.size, eps, _p(out), C.byref(d)), d)
    return out


def stable_top_k(s: np.ndarray, k: int):
    s = np.ascontiguousarray(s, dtype=np.float32)
    idx = np.empty(k, np.uint32)
    val = np.empty(k, np.float32)
    d = Diagnostic()
    _check(lib().kq_f32_stable_top_k(_p(s), s.size, k, _p(idx), _p(val), k, C.byref(d)), d)
    return idx, val


class MoeConfig:
    """A reference MoE config from dimensions (kq_moe_test_config_create)."""

    def __init__(self, hidden, experts, top_k, inter, shared_inter):
        self.dims = (hidden, experts, top_k, inter, shared_inter)
        d = MoeDims(hidden, experts, top_k, inter, shared_inter, 0)
        h = C.c_void_p()
        diag = Diagnostic()
        _check(lib().kq_moe_test_config_create(C.byref(d), C.byref(h), C.byref(diag)), diag)
        self.h = h

    def close(self):
        if self.h:
            lib().kq_moe_config_close(self.h)
            self.h = C.c_void_p()

    def __del__(self):
        self.close()

    def route(self, router: np.ndarray, x: np.ndarray):
        H, E, K, _, _ = self.dims
        router = np.ascontiguousarray(router, dtype=np.float32)
        x = np.ascontiguousarray(x, dtype=np.float32)
        logits = np.empty(E, np.float32)
        probs = np.empty(E, np.float32)
        ids = np.empty(K, np.uint32)
        w = np.empty(K, np.float32)
        d = Diagnostic()
        _check(lib().kq_moe_route_f32(self.h, _p(router), router.size, _p(x), _p(logits), E,
                                      _p(probs), E, _p(ids), K, _p(w), K, C.byref(d)), d)
        return logits, probs, ids, w

    def execute(self, weights: dict, hidden: np.ndarray) -> np.ndarray:
        """weights: role -> fp32 ndarray (router, routed_gate, routed_up,
        routed_down, shared_gate, shared_up, shared_down, shared_gate_weight)."""
        H = self.dims[0]
        hidden = np.ascontiguousarray(np.atleast_2d(hidden), dtype=np.float32)
        T = hidden.shape[0]
        keep = {k: np.ascontiguousarray(v, dtype=np.float32) for k, v in weights.items()}
        mw = MoeWeightsF32(**{f: v for k, a in keep.items()
                              for f, v in ((k, a.ctypes.data), (k + "_count", a.size))})
        out = np.empty((T, H), np.float32)
        nbytes = lib().kq_moe_config_scratch_bytes(self.h)
        scratch = np.empty(max(1, nbytes), np.uint8)
        d = Diagnostic()
        _check(lib().kq_moe_execute_f32(self.h, C.byref(mw), _p(hidden), T, _p(out), out.size,
                                        _p(scratch), nbytes, None, None, None, C.byref(d)), d)
        return out


    def routed_expert(self, gate: np.ndarray, up: np.ndarray, down: np.ndarray, expert_id: int,
                      x: np.ndarray) -> np.ndarray:
        """kq_moe_execute_routed_expert_f32 on one expert's member matrices."""
        H = self.dims[0]
        keep = [np.ascontiguousarray(a, dtype=np.float32) for a in (gate, up, down)]
        x = np.ascontiguousarray(x, dtype=np.float32)
        w = RoutedExpertWeightsF32(keep[0].ctypes.data, keep[0].size, keep[1].ctypes.data,
                                   keep[1].size, keep[2].ctypes.data, keep[2].size)
        out = np.empty(H, np.float32)
        nbytes = lib().kq_moe_config_one_expert_workspace_bytes(self.h)
        scratch = np.empty(max(1, nbytes), np.float32)
        d = Diagnostic()
        _check(lib().kq_moe_execute_routed_expert_f32(self.h, C.byref(w), expert_id, _p(x),
                                                      _p(out), H, _p(scratch), nbytes,
                                                      C.byref(d)), d)
        return out


class RngState(C.Structure):
    # include/kq_sampling.h:40-49
    _fields_ = [("version", C.c_uint32), ("reserved", C.c_uint32), ("seed", C.c_uint64),
                ("stream", C.c_uint64), ("state", C.c_uint64), ("increment", C.c_uint64),
                ("draws", C.c_uint64), ("integrity", C.c_uint64)]


class SamplingPolicy(C.Structure):
    # include/kq_sampling.h:24-31
    _fields_ = [("version", C.c_uint32), ("flags", C.c_uint32), ("temperature", C.c_float),
                ("top_p", C.c_float), ("top_k", C.c_uint32), ("reserved", C.c_uint32 * 3)]


class SamplingResult(C.Structure):
    # include/kq_sampling.h:51-63
    _fields_ = [("selected_token_id", C.c_uint32), ("top_k_retained_count", C.c_uint32),
                ("retained_count", C.c_uint32), ("rng_word", C.c_uint32),
                ("selected_probability", C.c_float), ("maximum_probability", C.c_float),
                ("normalized_sum_f32", C.c_float), ("reserved", C.c_uint32),
                ("uniform_value", C.c_double), ("rng_draws_before", C.c_uint64),
                ("rng_draws_after", C.c_uint64)]


def sample(policy: dict, seed: int, stream: int, logits: np.ndarray):
    """The reference's kq_sampling_select_f32 on a fresh RNG (seed, stream):
    (status, SamplingResult, state after)."""
    l = lib()
    vp = C.c_void_p
    l.kq_sampling_rng_seed.argtypes = [C.c_uint64, C.c_uint64, C.POINTER(RngState),
                                       C.POINTER(Diagnostic)]
    l.kq_sampling_config_open_qwen38.argtypes = [C.POINTER(SamplingPolicy), C.POINTER(vp),
                                                 C.POINTER(Diagnostic)]
    l.kq_sampling_required_scratch_bytes.argtypes = [vp]
    l.kq_sampling_required_scratch_bytes.restype = C.c_uint64
    l.kq_sampling_config_close.argtypes = [vp]
    l.kq_sampling_config_close.restype = None
    l.kq_sampling_select_f32.argtypes = [vp, C.POINTER(RngState), vp, C.c_uint64, vp, C.c_uint64,
                                         C.POINTER(SamplingResult), C.POINTER(Diagnostic)]
    d = Diagnostic()
    st = RngState()
    _check(l.kq_sampling_rng_seed(seed, stream, C.byref(st), C.byref(d)), d)
    pol = SamplingPolicy(1, 0, policy["temperature"], policy["top_p"], policy["top_k"])
    cfg = vp()
    _check(l.kq_sampling_config_open_qwen38(C.byref(pol), C.byref(cfg), C.byref(d)), d)
    n = l.kq_sampling_required_scratch_bytes(cfg)
    scratch = np.zeros(n, np.uint8)
    lg = np.ascontiguousarray(logits, np.float32)
    res = SamplingResult()
    status = l.kq_sampling_select_f32(cfg, C.byref(st), _p(lg), lg.size, _p(scratch), n,
                                      C.byref(res), C.byref(d))
    l.kq_sampling_config_close(cfg)
    return status, res, st


class LayerDims(C.Structure):
    # src/kq_layer_internal.h:10-17
    _fields_ = [("layer_id", C.c_uint32), ("hidden_size", C.c_uint32),
                ("branch_count", C.c_uint32), ("gr_rank", C.c_uint32),
                ("rms_epsilon", C.c_float), ("family", C.c_int)]


class LayerConfig(C.Structure):
    # src/kq_layer_internal.h:19-31 (the fields the gated residual reads
    # are the magic and the dimensions; the rest stay zero)
    _fields_ = [("magic", C.c_uint32), ("model", C.c_void_p), ("dimensions", LayerDims),
                ("owns_subconfigs", C.c_int), ("subconfigs", C.c_void_p * 5),
                ("gr_bindings", C.c_void_p * 8), ("gr_workspace_bytes", C.c_uint64)]


class GrWeightsF32(C.Structure):
    # include/kq_layer.h:59-68
    _fields_ = [("norm", C.c_void_p), ("norm_count", C.c_uint64), ("down", C.c_void_p),
                ("down_count", C.c_uint64), ("up", C.c_void_p), ("up_count", C.c_uint64),
                ("inject", C.c_void_p), ("inject_count", C.c_uint64)]


def gr_read_f32(branches, hidden, rank, eps, norm, down, up, inject):
    """The reference's kq_layer_gr_read_f32 on F32 weights (one token):
    dict of normalized, read_gate, mixed, rank and write_gate."""
    l = lib()
    l.kq_layer_gr_read_f32.argtypes = [C.POINTER(LayerConfig), C.POINTER(GrWeightsF32)] + \
        [C.c_void_p] * 6 + [C.POINTER(Diagnostic)]
    b = np.ascontiguousarray(branches, np.float32).reshape(-1)
    nb = b.size // hidden
    width = nb * hidden
    arrs = [np.ascontiguousarray(a, np.float32).reshape(-1) for a in (norm, down, up, inject)]
    cfg = LayerConfig()
    cfg.magic = 0x4b514c43
    cfg.dimensions = LayerDims(0, hidden, nb, rank, eps, 0)
    w = GrWeightsF32(_p(arrs[0]), arrs[0].size, _p(arrs[1]), arrs[1].size, _p(arrs[2]),
                     arrs[2].size, _p(arrs[3]), arrs[3].size)
    out = {"normalized": np.zeros(width, np.float32), "read_gate": np.zeros(width, np.float32),
           "mixed": np.zeros(hidden, np.float32), "rank": np.zeros(rank, np.float32),
           "write_gate": np.zeros(nb, np.float32)}
    d = Diagnostic()
    _check(l.kq_layer_gr_read_f32(C.byref(cfg), C.byref(w), _p(b), _p(out["normalized"]),
                                  _p(out["read_gate"]), _p(out["mixed"]), _p(out["rank"]),
                                  _p(out["write_gate"]), C.byref(d)), d)
    return out
