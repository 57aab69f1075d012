"""ctypes wrapper over oracle/_build/libkq_oracle.so.

TEST INFRASTRUCTURE ONLY: the CPU restatement of the reference path used as
the checker by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline
leg. Nothing in the product package imports this module.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "libkq_oracle.so"

F32, Q5_1, Q8_0, Q4_K, Q5_K, Q6_K, IQ4_NL, BF16 = 0, 7, 8, 12, 13, 14, 20, 30
TYPE_IDS = {"F32": F32, "Q5_1": Q5_1, "Q8_0": Q8_0, "Q4_K": Q4_K,
            "Q5_K": Q5_K, "Q6_K": Q6_K, "IQ4_NL": IQ4_NL, "BF16": BF16}
OK = 0

_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(f"oracle library missing: {LIB_PATH} (run make -C oracle)")
        _lib = C.CDLL(str(LIB_PATH))
        _declare(_lib)
    return _lib


class MoeDims(C.Structure):
    _fields_ = [("hidden", C.c_uint32), ("experts", C.c_uint32),
                ("top_k", C.c_uint32), ("inter", C.c_uint32),
                ("shared_inter", C.c_uint32)]


class Tensor(C.Structure):
    _fields_ = [("type", C.c_uint32), ("data", C.c_void_p)]


class MoeWeights(C.Structure):
    _fields_ = [(n, Tensor) for n in ("router", "gate", "up", "down", "shared_gate",
                                      "shared_up", "shared_down", "shared_gate_weight")]


TRACE_FIELDS = ("router_logits", "router_probs", "selected_ids", "selected_weights",
                "routed_sum", "shared_gate_proj", "shared_up_proj", "shared_activated",
                "shared_output", "shared_scale_logit", "shared_scale", "gated_shared",
                "expert_gate", "expert_up", "expert_activated", "expert_output",
                "expert_weighted")


class MoeTrace(C.Structure):
    _fields_ = [(n, C.c_void_p) for n in TRACE_FIELDS]


class RngState(C.Structure):
    # include/kq_sampling.h:40-49
    _fields_ = [("version", C.c_uint32), ("reserved", C.c_uint32), ("seed", C.c_uint64),
                ("stream", C.c_uint64), ("state", C.c_uint64), ("increment", C.c_uint64),
                ("draws", C.c_uint64), ("integrity", C.c_uint64)]


class SampleResult(C.Structure):
    _fields_ = [("selected_token_id", C.c_uint32), ("top_k_retained_count", C.c_uint32),
                ("retained_count", C.c_uint32), ("rng_word", C.c_uint32),
                ("selected_probability", C.c_float), ("maximum_probability", C.c_float),
                ("normalized_sum_f32", C.c_float), ("reserved", C.c_uint32),
                ("uniform_value", C.c_double)]


def _declare(l: C.CDLL) -> None:
    P, U32, U64, F, I = C.c_void_p, C.c_uint32, C.c_uint64, C.c_float, C.c_int
    l.kqo_geometry.argtypes = [U32, C.POINTER(U32), C.POINTER(U32)]
    l.kqo_f16_to_f32.argtypes = [C.c_uint16]
    l.kqo_f16_to_f32.restype = F
    l.kqo_expf.argtypes = [F]
    l.kqo_expf.restype = F
    l.kqo_f16_to_f32_array.argtypes = [P, U64, P]
    l.kqo_f16_to_f32_array.restype = None
    l.kqo_expf_array.argtypes = [P, U64, P, I]
    l.kqo_expf_array.restype = None
    l.kqo_expf_libm_mismatches.argtypes = [U64, U64, I]
    l.kqo_expf_libm_mismatches.restype = U64
    l.kqo_dequantize_blocks_f32.argtypes = [U32, P, U64, P, U64, C.POINTER(U64)]
    l.kqo_row_dot_f32.argtypes = [U32, P, U64, P, U64, C.POINTER(F)]
    l.kqo_matvec_f32.argtypes = [U32, P, U64, U64, P, U32, P, I]
    l.kqo_argmax_f32.argtypes = [P, U64, C.POINTER(U32)]
    for n in ("kqo_f32_add", "kqo_f32_multiply", "kqo_f32_swiglu"):
        getattr(l, n).argtypes = [P, P, U64, P]
    for n in ("kqo_f32_sigmoid", "kqo_f32_silu", "kqo_f32_softmax", "kqo_f32_renormalize"):
        getattr(l, n).argtypes = [P, U64, P]
    l.kqo_f32_scale.argtypes = [P, U64, F, P]
    l.kqo_f32_dot.argtypes = [P, P, U64, C.POINTER(F)]
    l.kqo_f32_rms_norm.argtypes = [P, P, U64, F, P]
    l.kqo_gr_read.argtypes = [U32, U32, U32, F, P, P, U32, P, U32, P, P, P, P, P, P, P]
    l.kqo_gr_write.argtypes = [U32, U32, P, P, P, P]
    l.kqo_gr_write.restype = None
    l.kqo_f32_stable_top_k.argtypes = [P, U64, U32, P, P]
    l.kqo_moe_select_top_k.argtypes = [P, U32, U32, P]
    l.kqo_moe_select_top_k.restype = None
    l.kqo_moe_route_f32.argtypes = [C.POINTER(MoeDims), C.POINTER(Tensor), P, P, P, P, P, I]
    l.kqo_moe_execute.argtypes = [C.POINTER(MoeDims), C.POINTER(MoeWeights), P, U64, P,
                                  C.POINTER(MoeTrace), I]
    l.kqo_moe_permutation.argtypes = [P, U64, U32, U32, P, P, P]
    l.kqo_moe_routed_expert_f32.argtypes = [U32, U32, P, P, P, P, P]
    l.kqo_gdn_physical_row.argtypes = [U32, U64]
    l.kqo_gdn_physical_row.restype = U64
    l.kqo_gdn_physical_column.argtypes = [U32, U64]
    l.kqo_gdn_physical_column.restype = U64
    l.kqo_gdn_linear_f32.argtypes = [U32, U32, P, U64, U64, P, P, I]
    l.kqo_rng_seed.argtypes = [U64, U64, C.POINTER(RngState)]
    l.kqo_rng_seed.restype = None
    l.kqo_rng_next.argtypes = [C.POINTER(RngState)]
    l.kqo_rng_next.restype = U32
    l.kqo_sample_f32.argtypes = [F, F, U32, U32, P, U32, U32, C.POINTER(SampleResult), P, P]
    l.kqo_route_certify.argtypes = [U32, U32, U32, P, P, P, C.POINTER(I)]
    l.kqo_certify_campaign.argtypes = [U64, U64, U32, U32, U32, I, F, C.c_double, I, P]


def _p(a: np.ndarray) -> int:
    assert a.flags["C_CONTIGUOUS"]
    return a.ctypes.data


def geometry(type_id: int) -> tuple[int, int]:
    e, b = C.c_uint32(), C.c_uint32()
    st = lib().kqo_geometry(type_id, C.byref(e), C.byref(b))
    if st != OK:
        raise ValueError(f"unsupported type {type_id}")
    return e.value, b.value


def f16_to_f32(bits: int) -> float:
    return lib().kqo_f16_to_f32(bits)


def expf(x: float) -> float:
    return lib().kqo_expf(x)


def f16_to_f32_array(bits: np.ndarray) -> np.ndarray:
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(bits.size, np.float32)
    lib().kqo_f16_to_f32_array(_p(bits), bits.size, _p(out))
    return out


def expf_array(x: np.ndarray, threads: int = 1) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    lib().kqo_expf_array(_p(x), x.size, _p(out), threads)
    return out


def dequantize(type_id: int, packed: np.ndarray) -> np.ndarray:
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    e, b = geometry(type_id)
    n = packed.size // b * e
    out = np.empty(max(n, 1), dtype=np.float32)
    cnt = C.c_uint64()
    st = lib().kqo_dequantize_blocks_f32(type_id, _p(packed), packed.size, _p(out), n,
                                          C.byref(cnt))
    if st != OK:
        raise OracleError(st)
    return out[:n]


def row_dot(type_id: int, packed: np.ndarray, x: np.ndarray) -> float:
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = C.c_float()
    st = lib().kqo_row_dot_f32(type_id, _p(packed), packed.size, _p(x), x.size, C.byref(out))
    if st != OK:
        raise OracleError(st)
    return out.value


def matvec(type_id: int, w: np.ndarray, rows: int, cols: int, x: np.ndarray,
           threads: int = 1) -> np.ndarray:
    """x: [batch, cols] float32 -> y: [batch, rows]."""
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.float32)
    batch = x.shape[0]
    assert x.shape[1] == cols
    w = np.ascontiguousarray(w)
    y = np.empty((batch, rows), dtype=np.float32)
    st = lib().kqo_matvec_f32(type_id, _p(w), rows, cols, _p(x), batch, _p(y), threads)
    if st != OK:
        raise OracleError(st)
    return y


def argmax(logits: np.ndarray) -> int:
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    out = C.c_uint32()
    st = lib().kqo_argmax_f32(_p(logits), logits.size, C.byref(out))
    if st != OK:
        raise OracleError(st)
    return out.value


def unary(name: str, a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty_like(a)
    st = getattr(lib(), "kqo_f32_" + name)(_p(a), a.size, _p(out))
    if st != OK:
        raise OracleError(st)
    return out


def binary(name: str, a: np.ndarray, b: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    out = np.empty_like(a)
    st = getattr(lib(), "kqo_f32_" + name)(_p(a), _p(b), a.size, _p(out))
    if st != OK:
        raise OracleError(st)
    return out


def scale(a: np.ndarray, s: float) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty_like(a)
    st = lib().kqo_f32_scale(_p(a), a.size, C.c_float(s), _p(out))
    if st != OK:
        raise OracleError(st)
    return out


def dot(a: np.ndarray, b: np.ndarray) -> float:
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    out = C.c_float()
    st = lib().kqo_f32_dot(_p(a), _p(b), a.size, C.byref(out))
    if st != OK:
        raise OracleError(st)
    return out.value


def rms_norm(a: np.ndarray, w: np.ndarray, eps: float) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    out = np.empty_like(a)
    st = lib().kqo_f32_rms_norm(_p(a), _p(w), a.size, C.c_float(eps), _p(out))
    if st != OK:
        raise OracleError(st)
    return out


def stable_top_k(s: np.ndarray, k: int) -> tuple[np.ndarray, np.ndarray]:
    s = np.ascontiguousarray(s, dtype=np.float32)
    idx = np.empty(k, dtype=np.uint32)
    val = np.empty(k, dtype=np.float32)
    st = lib().kqo_f32_stable_top_k(_p(s), s.size, k, _p(idx), _p(val))
    if st != OK:
        raise OracleError(st)
    return idx, val


def moe_select_top_k(probs: np.ndarray, k: int) -> np.ndarray:
    probs = np.ascontiguousarray(probs, dtype=np.float32)
    ids = np.empty(k, dtype=np.uint32)
    lib().kqo_moe_select_top_k(_p(probs), probs.size, k, _p(ids))
    return ids


def _tensor(t) -> Tensor:
    type_id, data = t
    return Tensor(type_id, data.ctypes.data)


def moe_route(dims: dict, router: tuple, x: np.ndarray, threads: int = 1):
    d = MoeDims(**dims)
    E, K = dims["experts"], dims["top_k"]
    x = np.ascontiguousarray(x, dtype=np.float32)
    logits = np.empty(E, np.float32)
    probs = np.empty(E, np.float32)
    ids = np.empty(K, np.uint32)
    w = np.empty(K, np.float32)
    t = _tensor(router)
    st = lib().kqo_moe_route_f32(C.byref(d), C.byref(t), _p(x), _p(logits), _p(probs),
                                 _p(ids), _p(w), threads)
    if st != OK:
        raise OracleError(st)
    return logits, probs, ids, w


def moe_execute(dims: dict, weights: dict, hidden: np.ndarray, trace: bool = False,
                threads: int = 1):
    """weights: role -> (type_id, ndarray). hidden: [tokens, hidden]."""
    d = MoeDims(**dims)
    hidden = np.ascontiguousarray(np.atleast_2d(hidden), dtype=np.float32)
    T = hidden.shape[0]
    H, E, K, I, S = (dims["hidden"], dims["experts"], dims["top_k"], dims["inter"],
                     dims["shared_inter"])
    w = MoeWeights(**{k: _tensor(v) for k, v in weights.items()})
    out = np.empty((T, H), np.float32)
    tr_arrays = None
    tr_ptr = None
    if trace:
        shapes = {"router_logits": (T, E), "router_probs": (T, E),
                  "selected_ids": (T, K), "selected_weights": (T, K),
                  "routed_sum": (T, H), "shared_gate_proj": (T, S),
                  "shared_up_proj": (T, S), "shared_activated": (T, S),
                  "shared_output": (T, H), "shared_scale_logit": (T,),
                  "shared_scale": (T,), "gated_shared": (T, H),
                  "expert_gate": (T, K, I), "expert_up": (T, K, I),
                  "expert_activated": (T, K, I), "expert_output": (T, K, H),
                  "expert_weighted": (T, K, H)}
        tr_arrays = {k: np.zeros(s, np.uint32 if k == "selected_ids" else np.float32)
                     for k, s in shapes.items()}
        tr = MoeTrace(**{k: v.ctypes.data for k, v in tr_arrays.items()})
        tr_ptr = C.byref(tr)
    st = lib().kqo_moe_execute(C.byref(d), C.byref(w), _p(hidden), T, _p(out), tr_ptr, threads)
    if st != OK:
        raise OracleError(st)
    return (out, tr_arrays) if trace else out


def rng_seed(seed: int, stream: int) -> RngState:
    st = RngState()
    lib().kqo_rng_seed(seed, stream, C.byref(st))
    return st


def rng_next(state: RngState) -> int:
    return int(lib().kqo_rng_next(C.byref(state)))


def sample(policy: dict, logits: np.ndarray, word: int, canonical_count: int):
    """(status, SampleResult, scores, probabilities) of one selection with
    the RNG word drawn."""
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    r = SampleResult()
    sc = np.zeros(lg.size, np.float32)
    pr = np.zeros(lg.size, np.float32)
    st = lib().kqo_sample_f32(policy["temperature"], policy["top_p"], policy["top_k"],
                              canonical_count, _p(lg), lg.size, word, C.byref(r), _p(sc), _p(pr))
    return st, r, sc, pr


GDN = {"none": 0, "qkv": 1, "gate": 2, "alpha": 3, "beta": 4, "conv": 5, "out": 6}


def gdn_physical_row(transform: str, row: int) -> int:
    return int(lib().kqo_gdn_physical_row(GDN[transform], row))


def gdn_physical_column(transform: str, col: int) -> int:
    return int(lib().kqo_gdn_physical_column(GDN[transform], col))


def gdn_linear(transform: str, type_id: int, w: np.ndarray, rows: int, cols: int,
               x: np.ndarray, threads: int = 1) -> np.ndarray:
    """The provider's linear for a GDN role: physical rows, GDN_OUT's
    activation permutation (src/kq_weight_provider.c:438-475)."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    w = np.ascontiguousarray(w)
    y = np.empty(rows, np.float32)
    st = lib().kqo_gdn_linear_f32(GDN[transform], type_id, _p(w), rows, cols, _p(x), _p(y),
                                  threads)
    if st != OK:
        raise OracleError(st)
    return y


def route_certify(router: np.ndarray, x: np.ndarray, top_k: int):
    """The device's certified one-token routing restated (kq_certify.c):
    (certified, ids)."""
    router = np.ascontiguousarray(router, dtype=np.float32)
    x = np.ascontiguousarray(x, dtype=np.float32)
    E, H = router.shape
    ids = np.zeros(top_k, np.uint32)
    cert = C.c_int()
    st = lib().kqo_route_certify(E, H, top_k, _p(router), _p(x), _p(ids), C.byref(cert))
    if st != OK:
        raise OracleError(st)
    return bool(cert.value), ids


CAMPAIGN_MODES = {"random": 0, "tie-at-boundary": 1, "tie-inside": 2, "tie-below-bound": 3,
                  "large-activations": 4}


def certify_campaign(seed: int, trials: int, experts: int, hidden: int, top_k: int,
                     mode: str, sigma: float = 0.02, threads: int = 1,
                     slack: float = 1.0) -> dict:
    """Certified selections against the exact route on generated cases
    (kq_certify.c kqo_certify_campaign). slack < 1 scales the bounds and the
    margin down: a planted unsound certification, which the campaign must
    catch; a negative slack also drops the normal-probability rule."""
    st_arr = np.zeros(6, np.uint64)
    st = lib().kqo_certify_campaign(seed, trials, experts, hidden, top_k,
                                    CAMPAIGN_MODES[mode], sigma, slack, threads,
                                    _p(st_arr))
    if st != OK:
        raise OracleError(st)
    keys = ("trials", "certified", "certified_mismatch", "rounding_decided",
            "first_mismatch_plus_1", "route_failures")
    return {k: int(v) for k, v in zip(keys, st_arr)}


def moe_routed_expert(gate: np.ndarray, up: np.ndarray, down: np.ndarray,
                      x: np.ndarray) -> np.ndarray:
    """One routed expert on F32 member matrices gate/up [I][H], down [H][I]
    (kq_moe_execute_routed_expert_f32)."""
    x = np.ascontiguousarray(x, np.float32)
    H = x.size
    g, u, d = (np.ascontiguousarray(a, np.float32) for a in (gate, up, down))
    inter = g.size // H
    out = np.empty(H, np.float32)
    st = lib().kqo_moe_routed_expert_f32(H, inter, _p(g), _p(u), _p(d), _p(x), _p(out))
    if st != 0:
        raise OracleError(st)
    return out


def moe_permutation(ids: np.ndarray, experts: int):
    ids = np.ascontiguousarray(ids, dtype=np.uint32)
    T, K = ids.shape
    off = np.zeros(experts + 1, np.uint32)
    tok = np.zeros(T * K, np.uint32)
    slot = np.zeros(T * K, np.uint32)
    st = lib().kqo_moe_permutation(_p(ids), T, K, experts, _p(off), _p(tok), _p(slot))
    if st != OK:
        raise OracleError(st)
    return off, tok, slot


def gr_read(branches: np.ndarray, hidden: int, rank: int, eps: float, norm: np.ndarray,
            down: tuple, up: tuple, inject: np.ndarray) -> dict:
    """Gated-residual read of one token (src/kq_layer_qwen38.c:40-172).

    branches [nbranch * hidden]; down = (type, [rank][width] rows),
    up = (type, [width][rank] rows), inject [nbranch][width] F32. Returns
    normalized, read_gate, mixed (the block input), rank and write_gate."""
    b = np.ascontiguousarray(branches, dtype=np.float32).reshape(-1)
    nb = b.size // hidden
    width = nb * hidden
    norm = np.ascontiguousarray(norm, dtype=np.float32)
    dt, dw = down
    ut, uw = up
    dw, uw = np.ascontiguousarray(dw), np.ascontiguousarray(uw)
    inj = np.ascontiguousarray(inject, dtype=np.float32)
    out = {"normalized": np.zeros(width, np.float32), "read_gate": np.zeros(width, np.float32),
           "mixed": np.zeros(hidden, np.float32), "rank": np.zeros(rank, np.float32),
           "write_gate": np.zeros(nb, np.float32)}
    st = lib().kqo_gr_read(nb, hidden, rank, eps, _p(b), _p(norm), dt, _p(dw), ut, _p(uw),
                           _p(inj), _p(out["normalized"]), _p(out["read_gate"]),
                           _p(out["mixed"]), _p(out["rank"]), _p(out["write_gate"]))
    if st != OK:
        raise OracleError(st)
    return out


def gr_write(branches: np.ndarray, hidden: int, block_output: np.ndarray,
             write_gate: np.ndarray) -> np.ndarray:
    """out[b][i] = branches[b][i] + block_output[i] * write_gate[b]
    (src/kq_layer_qwen38.c:196-208)."""
    b = np.ascontiguousarray(branches, dtype=np.float32).reshape(-1)
    bo = np.ascontiguousarray(block_output, dtype=np.float32)
    wg = np.ascontiguousarray(write_gate, dtype=np.float32)
    out = np.zeros_like(b)
    lib().kqo_gr_write(b.size // hidden, hidden, _p(b), _p(bo), _p(wg), _p(out))
    return out


class OracleError(RuntimeError):
    def __init__(self, status: int):
        super().__init__(f"oracle status {status}")
        self.status = status


def cpu_threads() -> int:
    return int(os.environ.get("KQ_ORACLE_THREADS", os.cpu_count() or 1))
