"""Pins the CPU oracle's numeric core against the reference's golden vectors
and against what the mathematics fixes. CPU only."""
import numpy as np
import pytest

from conftest import bits_f32, load_golden, oracle_threads, ulp_distance

NUM = load_golden("numeric_vectors.json")
PRIM = load_golden("primitive_vectors.json")


@pytest.mark.parametrize("case", NUM["cases"], ids=lambda c: c["id"])
def test_dequant_golden_exact_bits(oracle, case):
    # research/numerics/.../dequant-vectors.json: llama.cpp 90c26fcd to_float,
    # EXACT_BITS (tools/validate-native-numerics.py:63-93).
    packed = np.frombuffer(bytes.fromhex(case["packed_hex"]), np.uint8)
    got = oracle.dequantize(oracle.TYPE_IDS[case["type"]], packed)
    want = bits_f32(case["expected_f32_bits"])
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("case", NUM["row_dot_cases"], ids=lambda c: c["id"])
def test_row_dot_golden_exact_bits(oracle, case):
    src = {c["id"]: c for c in NUM["cases"]}[case["source_case_id"]]
    packed = np.frombuffer(bytes.fromhex(src["packed_hex"]), np.uint8)
    x = bits_f32(case["activation_f32_bits"])
    got = np.float32(oracle.row_dot(oracle.TYPE_IDS[case["type"]], packed, x))
    assert got.view(np.uint32) == bits_f32(case["expected_f32_bits"]).view(np.uint32)[0]


def test_f16_exhaustive(oracle):
    # Every binary16 pattern against numpy's independent conversion, bit for
    # bit (subnormals normalised exactly, Inf/NaN payload kept).
    got = oracle.f16_to_f32_array(np.arange(65536, dtype=np.uint16))
    want = np.arange(65536, dtype=np.uint16).view(np.float16).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_reference_unit_decode_cases(oracle):
    # tests/numeric_test.c:60-111 known answers.
    q8 = np.zeros(34, np.uint8)
    q8[0:2] = [0x00, 0x3C]
    q8[2:] = (np.arange(32) - 16).astype(np.int8).view(np.uint8)
    y = oracle.dequantize(oracle.Q8_0, q8)
    assert y[0] == -16.0 and y[31] == 15.0
    q4 = np.zeros(144, np.uint8)
    q4[0:2] = [0x00, 0x3C]
    q4[4] = 1
    q4[16] = 0x21
    y = oracle.dequantize(oracle.Q4_K, q4)
    assert y[0] == 1.0 and y[32] == 0.0
    q5 = np.zeros(24, np.uint8)
    q5[0:2] = [0x00, 0x3C]
    q5[2:4] = [0x00, 0xBC]
    q5[4] = 1
    q5[8] = 0x21
    y = oracle.dequantize(oracle.Q5_1, q5)
    assert y[0] == 16.0 and y[16] == 1.0
    row = np.zeros(34, np.uint8)
    row[0:2] = [0x00, 0x3C]
    row[2:] = 1
    assert oracle.row_dot(oracle.Q8_0, row, np.ones(32, np.float32)) == 32.0


def test_non_finite_scale_fails_closed(oracle):
    q8 = np.zeros(34, np.uint8)
    q8[0:2] = [0x00, 0x7C]  # +Inf
    with pytest.raises(oracle.OracleError) as e:
        oracle.dequantize(oracle.Q8_0, q8)
    assert e.value.status == 38
    q6 = np.zeros(210, np.uint8)
    q6[208:210] = [0x00, 0x7E]  # NaN
    with pytest.raises(oracle.OracleError):
        oracle.dequantize(oracle.Q6_K, q6)


# ---- Q6_K: the reference has no Q6_K; pinned by the public layout ----

def _q6k_block(d=1.0, sc=None, ql=None, qh=None):
    b = np.zeros(210, np.uint8)
    if ql is not None:
        b[0:128] = ql
    if qh is not None:
        b[128:192] = qh
    b[192:208] = (np.ones(16, np.int8) if sc is None else np.asarray(sc, np.int8)).view(np.uint8)
    b[208:210] = np.array([d], np.float16).view(np.uint8)
    return b


def test_q6k_all_zero_codes(oracle):
    # q = 0 everywhere -> every weight is (d*sc)*(-32); sc = 0 gives -0.0.
    y = oracle.dequantize(oracle.Q6_K, _q6k_block(d=0.5, sc=np.arange(16) - 8))
    want = np.repeat((np.float32(0.5) * (np.arange(16) - 8).astype(np.float32)) *
                     np.float32(-32.0), 16).astype(np.float32)
    assert np.array_equal(y.view(np.uint32), want.view(np.uint32))


def _q6k_bit_to_output():
    """Expected (output index, code bit) for each ql/qh bit, from the GGML
    block_q6_K description: ql byte j of half n holds the low nibble of
    output 128n+j (j<64) and the low nibble of output 128n+64+j in its high
    nibble; qh byte l of half n holds the 2 high bits of outputs
    128n+l, +32, +64, +96 in bit pairs 0-1, 2-3, 4-5, 6-7."""
    table = {}
    for n in range(2):
        for j in range(64):
            for bit in range(8):
                out = 128 * n + j + (64 if bit >= 4 else 0)
                table[("ql", 64 * n + j, bit)] = (out, bit % 4)
        for l in range(32):
            for bit in range(8):
                out = 128 * n + l + 32 * (bit // 2)
                table[("qh", 32 * n + l, bit)] = (out, 4 + bit % 2)
    return table


def test_q6k_single_bit_toggles(oracle):
    # Flipping one code bit changes exactly one weight by (d*sc)*2^k, and the
    # sub-scale used is sc[out // 16].
    sc = (np.arange(16) * 3 - 20).astype(np.int8)
    base = oracle.dequantize(oracle.Q6_K, _q6k_block(d=0.25, sc=sc))
    table = _q6k_bit_to_output()
    rng = np.random.default_rng(7)
    keys = list(table.keys())
    for idx in rng.choice(len(keys), 160, replace=False):
        field, byte, bit = keys[idx]
        ql = np.zeros(128, np.uint8)
        qh = np.zeros(64, np.uint8)
        (ql if field == "ql" else qh)[byte] = 1 << bit
        y = oracle.dequantize(oracle.Q6_K, _q6k_block(d=0.25, sc=sc, ql=ql, qh=qh))
        changed = np.nonzero(y != base)[0]
        out, code_bit = table[(field, byte, bit)]
        scale = np.float32(0.25) * np.float32(sc[out // 16])
        if scale == 0:
            assert changed.size == 0
            continue
        assert list(changed) == [out], (field, byte, bit)
        assert y[out] == scale * np.float32((1 << code_bit) - 32)


def test_q6k_pack_round_trip_and_closed_form(oracle):
    # Pack known 6-bit codes with an encoder written from the layout, decode,
    # and compare with (d*sc)*(q-32) rounded per step in binary32.
    rng = np.random.default_rng(11)
    for _ in range(8):
        q = rng.integers(0, 64, 256)
        sc = rng.integers(-32, 32, 16).astype(np.int8)
        d = np.float16(rng.uniform(1e-4, 2e-3))
        ql = np.zeros(128, np.uint8)
        qh = np.zeros(64, np.uint8)
        for o in range(256):
            n, r = divmod(o, 128)
            quarter, l = divmod(r, 32)
            lo, hi = q[o] & 15, q[o] >> 4
            j = 64 * n + l + (32 if quarter in (1, 3) else 0)
            ql[j] |= lo << (4 if quarter >= 2 else 0)
            qh[32 * n + l] |= hi << (2 * quarter)
        y = oracle.dequantize(oracle.Q6_K, _q6k_block(d=float(d), sc=sc, ql=ql, qh=qh))
        ds = np.float32(d) * np.repeat(sc.astype(np.float32), 16)
        want = (ds.astype(np.float32) * (q - 32).astype(np.float32)).astype(np.float32)
        assert np.array_equal(y.view(np.uint32), want.view(np.uint32))


# ---- Q4_K / Q8_0 against the closed form on random blocks ----

def test_q4k_closed_form_random(oracle):
    import kq_synth
    blocks = kq_synth.q4k_blocks(kq_synth.stream_key(99, 1), 64)
    y = oracle.dequantize(oracle.Q4_K, blocks.reshape(-1)).reshape(64, 256)
    for b in range(64):
        blk = blocks[b]
        d = np.float32(blk[0:2].view(np.float16)[0])
        dmin = np.float32(blk[2:4].view(np.float16)[0])
        s = blk[4:16]
        sc = [s[j] & 63 if j < 4 else (s[j + 4] & 15) | ((s[j - 4] >> 6) << 4) for j in range(8)]
        mn = [s[j + 4] & 63 if j < 4 else (s[j + 4] >> 4) | ((s[j] >> 6) << 4) for j in range(8)]
        qs = blk[16:]
        for g in range(4):
            lo = (qs[32 * g:32 * g + 32] & 15).astype(np.float32)
            hi = (qs[32 * g:32 * g + 32] >> 4).astype(np.float32)
            wl = np.float32(d * np.float32(sc[2 * g])) * lo - np.float32(dmin * np.float32(mn[2 * g]))
            wh = np.float32(d * np.float32(sc[2 * g + 1])) * hi - np.float32(
                dmin * np.float32(mn[2 * g + 1]))
            assert np.array_equal(y[b, 64 * g:64 * g + 32].view(np.uint32),
                                  wl.astype(np.float32).view(np.uint32))
            assert np.array_equal(y[b, 64 * g + 32:64 * g + 64].view(np.uint32),
                                  wh.astype(np.float32).view(np.uint32))


def test_synth_scale_pack_inverts_unpack(oracle):
    import kq_synth
    rng = np.random.default_rng(3)
    sc = rng.integers(0, 64, (50, 8))
    mn = rng.integers(0, 64, (50, 8))
    packed = kq_synth.pack_k_scales(sc, mn)
    blocks = np.zeros((50, 144), np.uint8)
    blocks[:, 0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    blocks[:, 2:4] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    blocks[:, 4:16] = packed
    # all quant nibbles zero -> weight = -(dmin*m) = -m per sub-block
    y = oracle.dequantize(oracle.Q4_K, blocks.reshape(-1)).reshape(50, 8, 32)
    assert np.array_equal(-y[:, :, 0], mn.astype(np.float32))
    blocks[:, 16:] = 0x11  # code 1 in both nibbles -> s - m
    y = oracle.dequantize(oracle.Q4_K, blocks.reshape(-1)).reshape(50, 8, 32)
    assert np.array_equal(y[:, :, 0], (sc - mn).astype(np.float32))


def test_row_dot_is_sequential_sum(oracle):
    # Brute force: one binary32 accumulator, left to right over the row.
    import kq_synth
    w = kq_synth.q4k_blocks(kq_synth.stream_key(98, 1), 4).reshape(-1)
    x = kq_synth.normal_f32(kq_synth.stream_key(98, 2), 1024)
    dq = oracle.dequantize(oracle.Q4_K, w)
    acc = np.float32(0)
    for a, b in zip(dq, x):
        acc = np.float32(acc + np.float32(a * b))
    assert np.float32(oracle.row_dot(oracle.Q4_K, w, x)).view(np.uint32) == acc.view(np.uint32)
    y = oracle.matvec(oracle.Q4_K, w, 1, 1024, x[None, :], threads=oracle_threads())
    assert y[0, 0].view(np.uint32) == acc.view(np.uint32)


def test_matvec_threads_identical(oracle):
    import kq_synth
    w = kq_synth.q6k_blocks(kq_synth.stream_key(97, 1), 64 * 4).reshape(-1)
    x = kq_synth.normal_f32(kq_synth.stream_key(97, 2), 2 * 1024).reshape(2, 1024)
    a = oracle.matvec(oracle.Q6_K, w, 64, 1024, x, threads=1)
    b = oracle.matvec(oracle.Q6_K, w, 64, 1024, x, threads=4)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_argmax_first_maximum(oracle):
    v = np.array([1.0, 3.0, 2.0, 3.0, -1.0], np.float32)
    assert oracle.argmax(v) == 1
    v = np.random.default_rng(5).standard_normal(10000).astype(np.float32)
    assert oracle.argmax(v) == int(np.argmax(v))
    with pytest.raises(oracle.OracleError):
        oracle.argmax(np.array([0.0, np.nan], np.float32))


def test_expf_equals_libm_all_inputs(oracle):
    # The restated expf against this process's libm expf on every 2^32 pattern.
    bad = oracle.lib().kqo_expf_libm_mismatches(0, 1 << 32, oracle_threads())
    assert bad == 0


# ---- primitives: primitive-calibration/holdout.json ----

PRIM_CASES = PRIM["calibration"] + PRIM["holdout"]


@pytest.mark.parametrize("case", PRIM_CASES, ids=lambda c: c["id"])
def test_primitive_vectors(oracle, case):
    op = case["operation"]
    left = bits_f32(case["input_left_f32_bits"])
    right = bits_f32(case.get("input_right_f32_bits", [])) if "input_right_f32_bits" in case else None
    if op == "topk":
        idx, val = oracle.stable_top_k(left, case["k"])
        assert list(idx) == case["expected_indices"]
        assert np.array_equal(val.view(np.uint32),
                              bits_f32(case["expected_f32_bits"]).view(np.uint32))
        return
    if op in ("add", "multiply", "swiglu"):
        got = oracle.binary(op, left, right)
    elif op in ("sigmoid", "silu", "softmax", "renormalize"):
        got = oracle.unary(op, left)
    elif op == "scale":
        got = oracle.scale(left, float(right[0]))
    elif op == "dot":
        got = np.array([oracle.dot(left, right)], np.float32)
    elif op == "rmsnorm":
        eps = bits_f32([case["epsilon_f32_bits"]])[0]
        got = oracle.rms_norm(left, right, float(eps))
    else:
        raise AssertionError(op)
    want = bits_f32(case["expected_f32_bits"])
    limit = PRIM["contracts"][op]["ulp_limit"]
    assert int(ulp_distance(got, want).max()) <= limit


def test_reference_unit_primitives(oracle):
    # tests/numeric_test.c:136-174.
    left = np.array([1.0, -2.0, 3.0, 4.0], np.float32)
    right = np.array([2.0, 3.0, -1.0, 0.5], np.float32)
    assert oracle.dot(left, right) == -5.0
    idx, _ = oracle.stable_top_k(np.array([3.0, 1.0, 3.0, 2.0], np.float32), 3)
    assert list(idx) == [0, 2, 3]
    assert oracle.unary("renormalize", np.array([0.2, 0.3, 0.5], np.float32))[2] == 0.5
    sm = oracle.unary("softmax", left)
    assert sm[3] > sm[2]
