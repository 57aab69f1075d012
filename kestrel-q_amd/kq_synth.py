"""Seeded synthetic inputs for the quantized-weight path.

Every tensor comes from a SplitMix64 stream keyed by (workload, role, expert)
under the master seed 0x4B514D4933353558 ("KQMI355X"), so the GPU path and the
CPU oracle always see identical bytes. Distributions:

  Q4_K block (144 B): d  f16 ~U[1e-3, 2e-2], dmin f16 ~U[0, 1e-2],
                      8 six-bit scales and 8 six-bit mins ~U{0..63} packed as
                      src/kq_numeric.c:161-174 unpacks them, 128 random quant B
  Q8_0 block (34 B):  d f16 ~U[1e-3, 2e-2], 32 int8 ~U{-127..127}
  Q6_K block (210 B): 128 B ql + 64 B qh random, 16 int8 sub-scales
                      ~U{-32..31}, d f16 ~U[1e-4, 2e-3]
  Q5_K block (176 B): as Q4_K, plus 32 random qh bytes (the fifth code bits)
  Q5_1 block (24 B):  d f16 ~U[1e-3, 2e-2], m f16 ~U[-1e-2, 1e-2], 4 random
                      qh bytes, 16 random quant bytes
  IQ4_NL block (18 B): d f16 ~U[1e-4, 2e-3], 16 random quant bytes
  activations:        N(mu, sigma) by Box-Muller in binary64, rounded to f32

Uniform floats are drawn in binary32 and rounded to binary16 to nearest even.
"""
from __future__ import annotations

import numpy as np

MASTER_SEED = 0x4B514D4933353558
_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)

# Workload ids used in stream keys.
W_MATVEC_Q4K, W_MATVEC_Q8_0, W_MATVEC_Q6K, W_DEQUANT, W_MOE, W_LM_HEAD, W_PREFILL = range(1, 8)
# Roles.
R_WEIGHT, R_X, R_ROUTER, R_GATE, R_UP, R_DOWN, R_SHARED_GATE, R_SHARED_UP, \
    R_SHARED_DOWN, R_SHARED_GATE_W, R_HIDDEN = range(1, 12)

Q4_K_BYTES, Q8_0_BYTES, Q6_K_BYTES = 144, 34, 210
Q5_K_BYTES, Q5_1_BYTES, IQ4_NL_BYTES = 176, 24, 18


def _mix(z: np.ndarray) -> np.ndarray:
    z = (z ^ (z >> np.uint64(30))) * _M1
    z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


def stream_key(workload: int, role: int, index: int = 0, sub: int = 0) -> int:
    return ((workload & 0xFF) << 56) | ((role & 0xFF) << 48) | ((sub & 0xFF) << 40) | \
        (index & 0xFFFFFFFFFF)


def u64(key: int, n: int) -> np.ndarray:
    """n outputs of the SplitMix64 stream selected by key."""
    with np.errstate(over="ignore"):
        base = _mix(np.array([MASTER_SEED ^ key], dtype=np.uint64))[0]
        i = np.arange(1, n + 1, dtype=np.uint64)
        return _mix(base + i * _GOLDEN)


def random_bytes(key: int, n: int) -> np.ndarray:
    words = u64(key, (n + 7) // 8)
    return words.view(np.uint8)[:n]


def uniform_f32(key: int, n: int, lo: float, hi: float) -> np.ndarray:
    u = (u64(key, n) >> np.uint64(40)).astype(np.float32) * np.float32(2.0 ** -24)
    return (np.float32(lo) + np.float32(hi - lo) * u).astype(np.float32)


def uniform_int(key: int, n: int, lo: int, hi: int) -> np.ndarray:
    span = np.uint64(hi - lo + 1)
    return ((u64(key, n) >> np.uint64(32)) % span).astype(np.int64) + lo


def normal_f32(key: int, n: int, sigma: float = 1.0, mu: float = 0.0) -> np.ndarray:
    z = u64(key, 2 * n)
    u1 = ((z[0::2] >> np.uint64(11)).astype(np.float64) + 1.0) * (2.0 ** -53)
    u2 = (z[1::2] >> np.uint64(11)).astype(np.float64) * (2.0 ** -53)
    g = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
    return (mu + sigma * g).astype(np.float32)


def _f16_bytes(vals: np.ndarray) -> np.ndarray:
    return vals.astype(np.float16).view(np.uint8).reshape(-1, 2)


def pack_k_scales(sc: np.ndarray, mn: np.ndarray) -> np.ndarray:
    """Inverse of the Q4_K/Q5_K 6-bit scale unpack (src/kq_numeric.c:161-174).

    sc, mn: [blocks, 8] in 0..63 -> [blocks, 12] packed bytes."""
    sc = sc.astype(np.uint8)
    mn = mn.astype(np.uint8)
    q = np.zeros((sc.shape[0], 12), dtype=np.uint8)
    for j in range(4):
        q[:, j] = sc[:, j] | ((sc[:, j + 4] >> 4) << 6)
        q[:, j + 4] = mn[:, j] | ((mn[:, j + 4] >> 4) << 6)
        q[:, j + 8] = (sc[:, j + 4] & 15) | ((mn[:, j + 4] & 15) << 4)
    return q


def q4k_blocks(key: int, blocks: int) -> np.ndarray:
    out = np.empty((blocks, Q4_K_BYTES), dtype=np.uint8)
    out[:, 0:2] = _f16_bytes(uniform_f32(key ^ 1, blocks, 1e-3, 2e-2))
    out[:, 2:4] = _f16_bytes(uniform_f32(key ^ 2, blocks, 0.0, 1e-2))
    sm = uniform_int(key ^ 3, blocks * 16, 0, 63).reshape(blocks, 16)
    out[:, 4:16] = pack_k_scales(sm[:, :8], sm[:, 8:])
    out[:, 16:] = random_bytes(key ^ 4, blocks * 128).reshape(blocks, 128)
    return out


def q8_0_blocks(key: int, blocks: int) -> np.ndarray:
    out = np.empty((blocks, Q8_0_BYTES), dtype=np.uint8)
    out[:, 0:2] = _f16_bytes(uniform_f32(key ^ 1, blocks, 1e-3, 2e-2))
    out[:, 2:] = uniform_int(key ^ 2, blocks * 32, -127, 127).astype(np.int8).view(
        np.uint8).reshape(blocks, 32)
    return out


def q6k_blocks(key: int, blocks: int) -> np.ndarray:
    out = np.empty((blocks, Q6_K_BYTES), dtype=np.uint8)
    out[:, 0:192] = random_bytes(key ^ 1, blocks * 192).reshape(blocks, 192)
    out[:, 192:208] = uniform_int(key ^ 2, blocks * 16, -32, 31).astype(np.int8).view(
        np.uint8).reshape(blocks, 16)
    out[:, 208:210] = _f16_bytes(uniform_f32(key ^ 3, blocks, 1e-4, 2e-3))
    return out


def q5k_blocks(key: int, blocks: int) -> np.ndarray:
    out = np.empty((blocks, Q5_K_BYTES), dtype=np.uint8)
    out[:, 0:2] = _f16_bytes(uniform_f32(key ^ 1, blocks, 1e-3, 2e-2))
    out[:, 2:4] = _f16_bytes(uniform_f32(key ^ 2, blocks, 0.0, 1e-2))
    sm = uniform_int(key ^ 3, blocks * 16, 0, 63).reshape(blocks, 16)
    out[:, 4:16] = pack_k_scales(sm[:, :8], sm[:, 8:])
    out[:, 16:] = random_bytes(key ^ 4, blocks * 160).reshape(blocks, 160)
    return out


def q5_1_blocks(key: int, blocks: int) -> np.ndarray:
    out = np.empty((blocks, Q5_1_BYTES), dtype=np.uint8)
    out[:, 0:2] = _f16_bytes(uniform_f32(key ^ 1, blocks, 1e-3, 2e-2))
    out[:, 2:4] = _f16_bytes(uniform_f32(key ^ 2, blocks, -1e-2, 1e-2))
    out[:, 4:] = random_bytes(key ^ 3, blocks * 20).reshape(blocks, 20)
    return out


def iq4_nl_blocks(key: int, blocks: int) -> np.ndarray:
    out = np.empty((blocks, IQ4_NL_BYTES), dtype=np.uint8)
    out[:, 0:2] = _f16_bytes(uniform_f32(key ^ 1, blocks, 1e-4, 2e-3))
    out[:, 2:] = random_bytes(key ^ 2, blocks * 16).reshape(blocks, 16)
    return out


BLOCK_GEN = {"Q4_K": (q4k_blocks, 256, Q4_K_BYTES),
             "Q8_0": (q8_0_blocks, 32, Q8_0_BYTES),
             "Q6_K": (q6k_blocks, 256, Q6_K_BYTES),
             "Q5_K": (q5k_blocks, 256, Q5_K_BYTES),
             "Q5_1": (q5_1_blocks, 32, Q5_1_BYTES),
             "IQ4_NL": (iq4_nl_blocks, 32, IQ4_NL_BYTES)}


def quant_matrix(fmt: str, key: int, rows: int, cols: int) -> np.ndarray:
    """Packed [rows, cols] matrix as a flat uint8 array (rows contiguous)."""
    gen, qk, _ = BLOCK_GEN[fmt]
    assert cols % qk == 0
    return gen(key, rows * (cols // qk)).reshape(-1)


def moe_weights(workload: int, hidden: int, experts: int, inter: int, shared_inter: int,
                gate_fmt: str = "Q4_K", down_fmt: str = "Q6_K", shared_gate_fmt: str = None,
                shared_down_fmt: str = None) -> dict:
    """MoE layer weights: fp32 router ~N(0,0.02), per-expert gate/up
    [inter, hidden] and down [hidden, inter] packed matrices stored back to
    back, a shared expert (of the routed formats unless given) and an fp32
    shared gate vector ~N(0, 0.02)."""
    w = {"router": normal_f32(stream_key(workload, R_ROUTER), experts * hidden, 0.02)}
    gate_gen, qk_g, _ = BLOCK_GEN[gate_fmt]
    down_gen, qk_d, _ = BLOCK_GEN[down_fmt]
    w["gate"] = np.concatenate([gate_gen(stream_key(workload, R_GATE, e), inter * hidden // qk_g)
                                .reshape(-1) for e in range(experts)])
    w["up"] = np.concatenate([gate_gen(stream_key(workload, R_UP, e), inter * hidden // qk_g)
                              .reshape(-1) for e in range(experts)])
    w["down"] = np.concatenate([down_gen(stream_key(workload, R_DOWN, e), hidden * inter // qk_d)
                                .reshape(-1) for e in range(experts)])
    sg_gen, qk_sg, _ = BLOCK_GEN[shared_gate_fmt or gate_fmt]
    sd_gen, qk_sd, _ = BLOCK_GEN[shared_down_fmt or down_fmt]
    w["shared_gate"] = sg_gen(stream_key(workload, R_SHARED_GATE),
                              shared_inter * hidden // qk_sg).reshape(-1)
    w["shared_up"] = sg_gen(stream_key(workload, R_SHARED_UP),
                            shared_inter * hidden // qk_sg).reshape(-1)
    w["shared_down"] = sd_gen(stream_key(workload, R_SHARED_DOWN),
                              hidden * shared_inter // qk_sd).reshape(-1)
    w["shared_gate_weight"] = normal_f32(stream_key(workload, R_SHARED_GATE_W), hidden, 0.02)
    return w


# ------------------------------------------------------------- GGUF writer

GGUF_UINT16, GGUF_UINT32, GGUF_INT32, GGUF_FLOAT32, GGUF_BOOL = 2, 4, 5, 6, 7
GGUF_STRING, GGUF_ARRAY, GGUF_UINT64 = 8, 9, 10


def _gguf_str(s) -> bytes:
    b = s.encode() if isinstance(s, str) else bytes(s)
    return len(b).to_bytes(8, "little") + b


def _gguf_value(vtype: int, value) -> bytes:
    if vtype == GGUF_STRING:
        return _gguf_str(value)
    if vtype == GGUF_ARRAY:
        etype, items = value
        body = b"".join(_gguf_value(etype, v) for v in items)
        return etype.to_bytes(4, "little") + len(items).to_bytes(8, "little") + body
    if vtype == GGUF_FLOAT32:
        return np.float32(value).tobytes()
    # GGUF value types 0..12: u8 i8 u16 i16 u32 i32 f32 bool str arr u64 i64 f64
    width = {0: 1, 1: 1, 2: 2, 3: 2, 4: 4, 5: 4, 7: 1, 10: 8, 11: 8, 12: 8}[vtype]
    return int(value).to_bytes(width, "little", signed=vtype in (1, 3, 5, 11))


def gguf_bytes(tensors, metadata, alignment: int = 32) -> bytes:
    """A GGUF v3 file image. tensors: (name, type_id, dims innermost first,
    packed payload bytes); metadata: (key, value type, value), arrays as
    (element type, items). Payloads are placed in order at aligned offsets
    from relative 0; a general.alignment entry is the caller's to add."""
    out = bytearray(b"GGUF")
    out += (3).to_bytes(4, "little") + len(tensors).to_bytes(8, "little")
    out += len(metadata).to_bytes(8, "little")
    for key, vtype, value in metadata:
        out += _gguf_str(key) + vtype.to_bytes(4, "little") + _gguf_value(vtype, value)
    rel, offsets = 0, []
    for name, type_id, dims, payload in tensors:
        offsets.append(rel)
        out += _gguf_str(name) + len(dims).to_bytes(4, "little")
        out += b"".join(int(d).to_bytes(8, "little") for d in dims)
        out += type_id.to_bytes(4, "little") + rel.to_bytes(8, "little")
        rel = (rel + len(payload) + alignment - 1) // alignment * alignment
    out += bytes(-len(out) % alignment)
    base = len(out)
    for (_, _, _, payload), off in zip(tensors, offsets):
        out += bytes(base + off - len(out))
        out += bytes(payload)
    return bytes(out)
