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

STATUS = {0: "OK", 1: "INVALID_ARGUMENT", 2: "OUT_OF_MEMORY", 12: "UNSUPPORTED_TENSOR_TYPE",
          13: "ARITHMETIC_OVERFLOW", 14: "LIMIT_EXCEEDED", 15: "INVALID_ALIGNMENT",
          16: "SPAN_OUT_OF_RANGE", 25: "INVALID_QUANTIZED_GEOMETRY", 32: "BUFFER_TOO_SMALL",
          38: "MALFORMED_QUANTIZED_DATA", 39: "NUMERIC_DOMAIN", 40: "DIMENSION_MISMATCH",
          41: "ALIASING_VIOLATION", 46: "INCOMPATIBLE_MOE", 1000: "DEVICE_FAILURE"}
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


class MoeWeights(C.Structure):
    _fields_ = [("router", C.c_void_p),
                ("routed_gate_type", C.c_uint32), ("routed_gate", C.c_void_p),
                ("routed_up_type", C.c_uint32), ("routed_up", C.c_void_p),
                ("routed_down_type", C.c_uint32), ("routed_down", C.c_void_p),
                ("shared_gate_type", C.c_uint32), ("shared_gate", C.c_void_p),
                ("shared_up_type", C.c_uint32), ("shared_up", C.c_void_p),
                ("shared_down_type", C.c_uint32), ("shared_down", C.c_void_p),
                ("shared_gate_weight", C.c_void_p)]


class KqError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"{STATUS.get(status, status)}: {message}")
        self.status = status
        self.name = STATUS.get(status, str(status))


# Every function declared in include/kq_hip.h and include/kq_status.h.
SIGNATURES = {
    "kq_status_string": (C.c_char_p, [C.c_int]),
    "kq_diagnostic_clear": (None, [C.c_void_p]),
    "kq_hip_context_create": (C.c_int, [C.c_int, C.c_void_p, C.c_void_p]),
    "kq_hip_context_destroy": (None, [C.c_void_p]),
    "kq_hip_context_set_async": (C.c_int, [C.c_void_p, C.c_int, C.c_void_p]),
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
    "kq_hip_moe_config_create": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p]),
    "kq_hip_moe_config_close": (None, [C.c_void_p]),
    "kq_hip_moe_config_scratch_bytes": (C.c_uint64, [C.c_void_p, C.c_uint64]),
    "kq_hip_moe_route_f32": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                       C.c_void_p, C.c_uint64, C.c_void_p, C.c_void_p,
                                       C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint64,
                                       C.c_void_p]),
    "kq_hip_moe_execute_quantized": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                               C.c_uint64, C.c_void_p, C.c_uint64, C.c_void_p,
                                               C.c_void_p, C.c_uint64, C.c_void_p]),
    "kq_hip_moe_token_permutation": (C.c_int, [C.c_void_p, C.c_void_p, C.c_void_p, C.c_uint64,
                                               C.c_void_p, C.c_void_p, C.c_void_p, C.c_void_p,
                                               C.c_uint64, C.c_void_p]),
    "kq_hip_f32_expf": (C.c_int, [C.c_void_p, C.c_void_p, C.c_uint64, C.c_void_p, C.c_void_p]),
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

    def close(self) -> None:
        if self.handle:
            lib().kq_hip_moe_config_close(C.c_void_p(self.handle))
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

    def lm_head(self, type_id: int, w, vocab: int, cols: int, h, batch: int, logits, ids) -> None:
        d = Diagnostic()
        check(lib().kq_hip_lm_head_greedy_f32(self._h, type_id, self._p(w), vocab, cols,
                                              self._p(h), batch, self._p(logits), self._p(ids),
                                              C.byref(d)), d)

    def expf(self, x, count: int, out) -> None:
        d = Diagnostic()
        check(lib().kq_hip_f32_expf(self._h, self._p(x), count, self._p(out), C.byref(d)), d)

    # ---- MoE ----
    def moe_route(self, cfg: MoeConfig, router, shared_gate_weight, hidden, tokens: int,
                  logits, probs, ids, weights, scratch, scratch_bytes: int) -> None:
        d = Diagnostic()
        check(lib().kq_hip_moe_route_f32(self._h, C.c_void_p(cfg.handle), self._p(router),
                                         self._p(shared_gate_weight), self._p(hidden), tokens,
                                         self._p(logits), self._p(probs), self._p(ids),
                                         self._p(weights), self._p(scratch), scratch_bytes,
                                         C.byref(d)), d)

    def moe_execute(self, cfg: MoeConfig, weights: MoeWeights, hidden, tokens: int, out,
                    ids, scratch, scratch_bytes: int, capacity: int | None = None) -> None:
        d = Diagnostic()
        cap = tokens * cfg.hidden if capacity is None else capacity
        check(lib().kq_hip_moe_execute_quantized(self._h, C.c_void_p(cfg.handle),
                                                 C.byref(weights), self._p(hidden), tokens,
                                                 self._p(out), cap,
                                                 self._p(ids) if ids is not None else None,
                                                 self._p(scratch), scratch_bytes, C.byref(d)), d)

    def moe_permutation(self, cfg: MoeConfig, ids, tokens: int, offsets, pair_token, pair_slot,
                        scratch, scratch_bytes: int) -> None:
        d = Diagnostic()
        check(lib().kq_hip_moe_token_permutation(self._h, C.c_void_p(cfg.handle), self._p(ids),
                                                 tokens, self._p(offsets), self._p(pair_token),
                                                 self._p(pair_slot), self._p(scratch),
                                                 scratch_bytes, C.byref(d)), d)


def moe_weights(bufs: dict, gate_type=TYPE_Q4_K, down_type=TYPE_Q6_K) -> MoeWeights:
    """bufs: role -> DeviceBuffer (router, gate, up, down, shared_gate,
    shared_up, shared_down, shared_gate_weight)."""
    P = lambda k: C.c_void_p(bufs[k].ptr)
    return MoeWeights(P("router"), gate_type, P("gate"), gate_type, P("up"), down_type,
                      P("down"), gate_type, P("shared_gate"), gate_type, P("shared_up"),
                      down_type, P("shared_down"), P("shared_gate_weight"))
