"""The oracle against the reference's own code (CPU).

oracle/_ref/libkq_ref.so is the reference's src/kq_numeric.c, kq_moe.c,
kq_moe_qwen38.c (and the files they need) compiled from their sources with
the reference's fp flags (oracle/Makefile, target `ref`). Every check below
feeds both the same inputs and asks for identical bits (or the identical
status on rejected input). Skipped where the reference sources are absent.
"""
import numpy as np
import pytest

import kq_oracle as O
import kq_ref as R
import kq_synth as S

pytestmark = pytest.mark.skipif(not R.available(),
                                reason="oracle/_ref not built (make -C oracle ref)")

# (type id, block bytes, block elements, byte offsets of f16 scale fields)
FORMATS = {
    "Q8_0": (O.Q8_0, 34, 32, (0,)),
    "Q4_K": (O.Q4_K, 144, 256, (0, 2)),
    "Q5_1": (O.Q5_1, 24, 32, (0, 2)),
    "Q5_K": (O.Q5_K, 176, 256, (0, 2)),
    "IQ4_NL": (O.IQ4_NL, 18, 32, (0,)),
}


def random_blocks(fmt: str, blocks: int, seed: int) -> np.ndarray:
    """Uniform random bytes with every f16 scale made finite (exponent < 31)."""
    _, nb, _, scale_offsets = FORMATS[fmt]
    rng = np.random.default_rng(seed)
    b = rng.integers(0, 256, size=(blocks, nb), dtype=np.uint8)
    for o in scale_offsets:
        b[:, o + 1] &= 0xBF
    return b.reshape(-1)


def same_bits(a, b):
    a = np.atleast_1d(np.asarray(a, np.float32)).view(np.uint32)
    b = np.atleast_1d(np.asarray(b, np.float32)).view(np.uint32)
    assert a.shape == b.shape
    bad = np.nonzero(a != b)[0]
    assert bad.size == 0, f"{bad.size} differ, first at {bad[:5]}: {a[bad[:5]]} vs {b[bad[:5]]}"


@pytest.mark.parametrize("fmt", sorted(FORMATS))
def test_dequantize_matches_reference(fmt):
    t, nb, qk, _ = FORMATS[fmt]
    packed = random_blocks(fmt, 4096, 11)
    same_bits(O.dequantize(t, packed), R.dequantize(t, packed, 4096 * qk))


@pytest.mark.parametrize("fmt", ["BF16", "F32"])
def test_dequantize_plain_matches_reference(fmt):
    rng = np.random.default_rng(12)
    v = rng.standard_normal(8192).astype(np.float32) * 3
    t = O.TYPE_IDS[fmt]
    packed = (v.view(np.uint32) >> 16).astype(np.uint16) if fmt == "BF16" else v
    same_bits(O.dequantize(t, packed.view(np.uint8)), R.dequantize(t, packed, 8192))


@pytest.mark.parametrize("fmt", ["Q8_0", "Q4_K", "Q5_K"])
def test_malformed_scale_status_matches_reference(fmt):
    t, nb, qk, offs = FORMATS[fmt]
    packed = random_blocks(fmt, 8, 13).reshape(8, nb)
    packed[5, offs[0] + 1] = 0x7C  # +Inf scale
    with pytest.raises(O.OracleError) as eo:
        O.dequantize(t, packed.reshape(-1))
    with pytest.raises(R.RefError) as er:
        R.dequantize(t, packed.reshape(-1), 8 * qk)
    assert eo.value.status == er.value.status == 38  # MALFORMED_QUANTIZED_DATA


def test_reference_has_no_q6k():
    # The Q6_K decode is restated from the GGML layout; the reference rejects
    # the type, so its parity rests on the oracle's own layout checks.
    with pytest.raises(R.RefError) as er:
        R.dequantize(O.Q6_K, np.zeros(210, np.uint8), 256)
    assert er.value.status == 12  # UNSUPPORTED_TENSOR_TYPE


@pytest.mark.parametrize("fmt", ["Q8_0", "Q4_K", "Q5_1", "Q5_K", "IQ4_NL"])
def test_row_dot_matches_reference(fmt):
    t, nb, qk, _ = FORMATS[fmt]
    cols = 2048
    rows = 48
    packed = random_blocks(fmt, rows * cols // qk, 21).reshape(rows, -1)
    rng = np.random.default_rng(22)
    for r in range(rows):
        x = rng.standard_normal(cols).astype(np.float32)
        same_bits(np.float32(O.row_dot(t, packed[r], x)), R.row_dot(t, packed[r], x)[0])


def test_matvec_rows_match_reference_row_dot():
    # the oracle's (threaded) matvec is the reference's row dot per row
    rows, cols = 256, 2048
    w = S.quant_matrix("Q4_K", S.stream_key(S.W_MATVEC_Q4K, S.R_WEIGHT, 99), rows, cols)
    x = S.normal_f32(S.stream_key(S.W_MATVEC_Q4K, S.R_X, 99), cols)
    y = O.matvec(O.Q4_K, w, rows, cols, x[None, :], threads=4)[0]
    rb = w.reshape(rows, -1)
    same_bits(y, np.array([R.row_dot(O.Q4_K, rb[r], x)[0] for r in range(rows)], np.float32))


def test_primitives_match_reference():
    rng = np.random.default_rng(31)
    a = (rng.standard_normal(4096) * 4).astype(np.float32)
    b = (rng.standard_normal(4096) * 4).astype(np.float32)
    for name in ("sigmoid", "silu", "softmax"):
        same_bits(O.unary(name, a), R.unary(name, a))
    for name in ("add", "multiply", "swiglu"):
        same_bits(O.binary(name, a, b), R.binary(name, a, b))
    same_bits(O.scale(a, np.float32(0.37)), R.scale(a, np.float32(0.37)))
    same_bits(np.float32(O.dot(a, b)), R.dot(a, b)[0])
    same_bits(O.rms_norm(a, b, 1e-6), R.rms_norm(a, b, 1e-6))
    oi, ov = O.stable_top_k(a, 10)
    ri, rv = R.stable_top_k(a, 10)
    assert list(oi) == list(ri)
    same_bits(ov, rv)


def route_both(H, E, K, router, x):
    cfg = R.MoeConfig(H, E, K, 8, 8)
    got_r = cfg.route(router, x)
    cfg.close()
    dims = dict(hidden=H, experts=E, top_k=K, inter=8, shared_inter=8)
    got_o = O.moe_route(dims, (O.F32, router), x)
    return got_o, got_r


@pytest.mark.parametrize("seed", range(3))
def test_route_512x2048_matches_reference(seed):
    H, E, K = 2048, 512, 10
    router = S.normal_f32(S.stream_key(S.W_MOE, S.R_ROUTER, 500 + seed), E * H, 0.02)
    x = S.normal_f32(S.stream_key(S.W_MOE, S.R_HIDDEN, 500 + seed), H)
    (ol, op, oi, ow), (rl, rp, ri, rw) = route_both(H, E, K, router, x)
    assert list(oi) == list(ri)
    for a, b in ((ol, rl), (op, rp), (ow, rw)):
        same_bits(a, b)


@pytest.mark.parametrize("pattern", ["duplicate-rows", "zero-router", "quantised-logits"])
def test_route_ties_match_reference(pattern):
    H, E, K = 64, 512, 10
    rng = np.random.default_rng({"duplicate-rows": 41, "zero-router": 42,
                                 "quantised-logits": 43}[pattern])
    if pattern == "duplicate-rows":
        router = rng.standard_normal((8, H)).astype(np.float32)[rng.integers(0, 8, E)]
    elif pattern == "zero-router":
        router = np.zeros((E, H), np.float32)
    else:
        router = (np.round(rng.standard_normal((E, H)) * 2) / 8).astype(np.float32)
    x = np.round(rng.standard_normal(H) * 4).astype(np.float32)
    (ol, op, oi, ow), (rl, rp, ri, rw) = route_both(H, E, K, router.reshape(-1), x)
    assert list(oi) == list(ri)
    for a, b in ((ol, rl), (op, rp), (ow, rw)):
        same_bits(a, b)


@pytest.mark.parametrize("shape,down_fmt", [((512, 32, 4, 256), "Q4_K"),
                                            ((2048, 64, 10, 512), "Q6_K")])
def test_execute_matches_reference_f32(shape, down_fmt):
    # The oracle's quantized MoE layer equals the reference's F32 layer run on
    # the oracle's dequantized weights, bit for bit (per-row sums are the same
    # left-to-right chains; the combine order is the reference's).
    H, E, K, I = shape
    w = S.moe_weights(S.W_MOE + 100, H, E, I, I, down_fmt=down_fmt)
    gt, dt = O.Q4_K, O.TYPE_IDS[down_fmt]
    roles = {"router": O.F32, "gate": gt, "up": gt, "down": dt, "shared_gate": gt,
             "shared_up": gt, "shared_down": dt, "shared_gate_weight": O.F32}
    dims = dict(hidden=H, experts=E, top_k=K, inter=I, shared_inter=I)
    x = S.normal_f32(S.stream_key(S.W_MOE + 100, S.R_HIDDEN, 3), 3 * H).reshape(3, H)
    got = O.moe_execute(dims, {k: (t, w[k]) for k, t in roles.items()}, x,
                        threads=O.cpu_threads())
    f32 = {"router": w["router"], "shared_gate_weight": w["shared_gate_weight"]}
    for ours, theirs in (("gate", "routed_gate"), ("up", "routed_up"),
                         ("down", "routed_down"), ("shared_gate", "shared_gate"),
                         ("shared_up", "shared_up"), ("shared_down", "shared_down")):
        f32[theirs] = O.dequantize(roles[ours], w[ours])
    cfg = R.MoeConfig(H, E, K, I, I)
    ref = cfg.execute(f32, x)
    cfg.close()
    same_bits(got, ref)


@pytest.mark.parametrize("B,H,rank,seed", [(4, 8, 4, 1), (4, 256, 32, 2), (2, 100, 7, 3),
                                           (4, 2560, 320, 4)])
def test_gated_residual_read_bit_exact(B, H, rank, seed):
    # the reference's src/kq_layer_qwen38.c (kq_layer_gr_read_f32) against
    # the oracle's kqo_gr_read on F32 projections: every output bit for bit
    W = B * H
    key = lambda i: S.stream_key(S.W_MOE + 600 + seed, 90, i)
    norm = S.normal_f32(key(1), W, 0.1)
    down = S.normal_f32(key(2), rank * W, 0.05)
    up = S.normal_f32(key(3), W * rank, 0.05)
    inject = S.normal_f32(key(4), B * W, 0.01)
    x = S.normal_f32(key(5), W)
    want = R.gr_read_f32(x, H, rank, 1e-6, norm, down, up, inject)
    got = O.gr_read(x, H, rank, 1e-6, norm, (O.F32, down), (O.F32, up), inject)
    for k in ("normalized", "read_gate", "mixed", "rank", "write_gate"):
        same_bits(got[k], want[k])


@pytest.mark.parametrize("H,I,scale", [(2048, 512, 1.0), (96, 40, 3.0), (7, 3, 0.01)])
def test_routed_expert_matches_reference(H, I, scale):
    # kq_moe_execute_routed_expert_f32 (src/kq_moe_qwen38.c:461-566): the
    # oracle's restatement bit for bit against the reference's own function
    rng = np.random.default_rng(H + I)
    g = (rng.standard_normal((I, H)) * 0.05 * scale).astype(np.float32)
    u = (rng.standard_normal((I, H)) * 0.05 * scale).astype(np.float32)
    d = (rng.standard_normal((H, I)) * 0.05 * scale).astype(np.float32)
    x = rng.standard_normal(H).astype(np.float32)
    cfg = R.MoeConfig(H, 8, 2, I, 4)
    want = cfg.routed_expert(g, u, d, 5, x)
    cfg.close()
    same_bits(O.moe_routed_expert(g, u, d, x), want)
