"""Device parity for the numeric core, through the C ABI, against the CPU
oracle on identical seeded inputs.

Bars: dequantized weights bit-exact; matvec / LM-head outputs per element
within 1e-4 absolute or 1e-3 relative of the oracle (fp32 accumulation in a
different order, conftest.assert_close), or of the binary64 value where the
oracle's own sequential sum is off by more (tests/exact.py); argmax token
ids exact; device expf bit-exact on all 2^32 inputs."""
import numpy as np
import pytest

from conftest import assert_close, bits_f32, load_golden, oracle_threads

import exact

import kq_hip
import kq_oracle
import kq_synth as S

pytestmark = pytest.mark.gpu

RTOL, ATOL = 1e-3, 1e-4
NUM = load_golden("numeric_vectors.json")
FMTS = {"Q4_K": kq_hip.TYPE_Q4_K, "Q8_0": kq_hip.TYPE_Q8_0, "Q6_K": kq_hip.TYPE_Q6_K,
        "Q5_K": kq_hip.TYPE_Q5_K, "Q5_1": kq_hip.TYPE_Q5_1, "IQ4_NL": kq_hip.TYPE_IQ4_NL}
# decode-only element types (no device products)
ELEM = {"F32": kq_hip.TYPE_F32, "BF16": kq_hip.TYPE_BF16}
ALL_FMTS = sorted(FMTS)


@pytest.fixture(scope="module")
def ctx():
    c = kq_hip.Context(0)
    yield c
    c.close()


def say(*a):
    print(*a, flush=True)


def gpu_dequant(ctx, type_id, packed):
    be, bb = kq_hip.geometry(type_id)
    n = packed.size // bb * be
    dp = ctx.upload(packed)
    do = ctx.alloc(n * 4)
    cnt = ctx.dequantize(type_id, dp, packed.size, do, n)
    assert cnt == n
    out = ctx.download(do, np.float32, n)
    dp.close()
    do.close()
    return out


@pytest.mark.parametrize("case", [c for c in NUM["cases"] if c["type"] in FMTS or c["type"] in ELEM],
                         ids=lambda c: c["id"])
def test_dequant_golden_vectors(ctx, case):
    packed = np.frombuffer(bytes.fromhex(case["packed_hex"]), np.uint8).copy()
    got = gpu_dequant(ctx, {**FMTS, **ELEM}[case["type"]], packed)
    want = bits_f32(case["expected_f32_bits"])
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("fmt", ALL_FMTS)
def test_dequant_64m_weights_bit_exact(ctx, fmt):
    # 67,108,864 weights per format, same seeded blocks as the oracle.
    gen, qk, bb = S.BLOCK_GEN[fmt]
    blocks = (1 << 26) // qk
    say(f"dequant {fmt}: {blocks} blocks")
    packed = gen(S.stream_key(S.W_DEQUANT, S.R_WEIGHT, FMTS[fmt]), blocks).reshape(-1)
    got = gpu_dequant(ctx, FMTS[fmt], packed)
    want = kq_oracle.dequantize(FMTS[fmt], packed)
    bad = np.nonzero(got.view(np.uint32) != want.view(np.uint32))[0]
    assert bad.size == 0, f"{bad.size} mismatches, first at {bad[:5]}"


@pytest.mark.parametrize("fmt", ALL_FMTS)
def test_dequant_ragged_block_counts(ctx, fmt):
    # Every wave takes four steps (a K-quant block or eight 32-weight
    # blocks) at a time: counts that end inside a step, inside a group of
    # four steps and on the buffer's last dword, each bit-exact.
    gen, qk, bb = S.BLOCK_GEN[fmt]
    for n in (1, 2, 3, 7, 9, 31, 33, 257, 1025):
        packed = gen(S.stream_key(S.W_DEQUANT, 60, FMTS[fmt], n), n).reshape(-1)
        got = gpu_dequant(ctx, FMTS[fmt], packed)
        want = kq_oracle.dequantize(FMTS[fmt], packed)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (fmt, n)


def test_dequant_subnormal_and_edge_scales(ctx):
    # Q4_K blocks whose d/dmin are fp16 subnormals, zero, negative zero and
    # the largest finite half; Q6_K/Q8_0 with subnormal d.
    blocks = S.q4k_blocks(S.stream_key(S.W_DEQUANT, 50), 64)
    halves = np.array([0x0001, 0x03FF, 0x8001, 0x0000, 0x8000, 0x7BFF, 0xFBFF, 0x0400],
                      np.uint16)
    for i in range(64):
        blocks[i, 0:2] = np.frombuffer(halves[i % 8].tobytes(), np.uint8)
        blocks[i, 2:4] = np.frombuffer(halves[(i // 8) % 8].tobytes(), np.uint8)
    p = blocks.reshape(-1)
    assert np.array_equal(gpu_dequant(ctx, kq_hip.TYPE_Q4_K, p).view(np.uint32),
                          kq_oracle.dequantize(kq_oracle.Q4_K, p).view(np.uint32))
    q6 = S.q6k_blocks(S.stream_key(S.W_DEQUANT, 51), 8)
    q8 = S.q8_0_blocks(S.stream_key(S.W_DEQUANT, 52), 8)
    for i in range(8):
        q6[i, 208:210] = np.frombuffer(halves[i].tobytes(), np.uint8)
        q8[i, 0:2] = np.frombuffer(halves[i].tobytes(), np.uint8)
    for t, b in ((kq_hip.TYPE_Q6_K, q6), (kq_hip.TYPE_Q8_0, q8)):
        p = b.reshape(-1)
        assert np.array_equal(gpu_dequant(ctx, t, p).view(np.uint32),
                              kq_oracle.dequantize(t, p).view(np.uint32))


# (format, byte offset of a binary16 scale field in the block)
SCALE_FIELDS = [("Q8_0", 0), ("Q4_K", 0), ("Q4_K", 2), ("Q5_K", 0), ("Q5_K", 2), ("Q6_K", 208),
                ("Q5_1", 0), ("Q5_1", 2), ("IQ4_NL", 0)]
HALF_ALL = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
HALF_FINITE = HALF_ALL[(HALF_ALL & 0x7C00) != 0x7C00]      # 63,488 patterns
HALF_NONFINITE = HALF_ALL[(HALF_ALL & 0x7C00) == 0x7C00]   # +-Inf and the NaNs: 2,048


@pytest.mark.parametrize("fmt,field", SCALE_FIELDS, ids=[f"{f}@{o}" for f, o in SCALE_FIELDS])
def test_f16_scale_every_finite_pattern(ctx, fmt, field):
    # Every finite binary16 pattern, subnormals and both zeros included, as
    # this scale field of one block each (the other fields seeded): the
    # device decode is bit-exact with the oracle's on all 63,488 of them.
    gen, qk, bb = S.BLOCK_GEN[fmt]
    blocks = gen(S.stream_key(S.W_DEQUANT, 70, FMTS[fmt], field), HALF_FINITE.size)
    blocks[:, field:field + 2] = HALF_FINITE.view(np.uint8).reshape(-1, 2)
    if fmt == "Q8_0":
        blocks[:, 2] = 1  # code 1: the first output is the scale itself
    p = blocks.reshape(-1)
    got = gpu_dequant(ctx, FMTS[fmt], p)
    want = kq_oracle.dequantize(FMTS[fmt], p)
    bad = np.nonzero(got.view(np.uint32) != want.view(np.uint32))[0]
    assert bad.size == 0, f"{bad.size} mismatches, first blocks {bad[:5] // qk}"
    if fmt == "Q8_0":
        # and against numpy's binary16 -> binary32 conversion directly
        ref = HALF_FINITE.view(np.float16).astype(np.float32)
        assert np.array_equal(got[0::32].view(np.uint32), ref.view(np.uint32))


@pytest.mark.parametrize("fmt,field", SCALE_FIELDS, ids=[f"{f}@{o}" for f, o in SCALE_FIELDS])
def test_f16_scale_nonfinite_patterns_fail_closed(ctx, fmt, field):
    # A non-finite scale is MALFORMED_QUANTIZED_DATA (src/kq_numeric.c:194,
    # :212, :235, :281). Q8_0's scale field: every one of the 2,048
    # non-finite patterns alone in a three-block buffer; the other fields:
    # the infinities and NaNs with the smallest, largest and a middle
    # payload, of both signs.
    gen, qk, bb = S.BLOCK_GEN[fmt]
    pats = HALF_NONFINITE if (fmt, field) == ("Q8_0", 0) else np.array(
        [0x7C00, 0xFC00, 0x7C01, 0xFC01, 0x7E00, 0xFE00, 0x7FFF, 0xFFFF, 0x7D55], np.uint16)
    base = gen(S.stream_key(S.W_DEQUANT, 71, FMTS[fmt], field), 3)
    dp = ctx.alloc(base.size)
    do = ctx.alloc(3 * qk * 4)
    for h in pats:
        b = base.copy()
        b[1, field:field + 2] = np.frombuffer(np.uint16(h).tobytes(), np.uint8)
        d = kq_hip.Diagnostic()
        kq_hip.check(kq_hip.lib().kq_hip_upload(ctx._h, kq_hip.C.c_void_p(dp.ptr),
                                                b.ctypes.data, b.nbytes, kq_hip.C.byref(d)), d)
        with pytest.raises(kq_hip.KqError) as e:
            ctx.dequantize(FMTS[fmt], dp, b.nbytes, do, 3 * qk)
        assert e.value.name == "MALFORMED_QUANTIZED_DATA", hex(int(h))
    # and the context still decodes a good buffer
    ok = base.reshape(-1)
    assert np.array_equal(gpu_dequant(ctx, FMTS[fmt], ok).view(np.uint32),
                          kq_oracle.dequantize(FMTS[fmt], ok).view(np.uint32))
    dp.close()
    do.close()


def test_matvec_f16_scale_every_finite_pattern(ctx):
    # The matvec path converts block scales with the hardware instruction:
    # a Q8_0 matrix of one-block rows whose scales are every finite binary16
    # pattern, against the oracle (the products of huge scales stay finite).
    rows, cols = HALF_FINITE.size, 32
    w = S.q8_0_blocks(S.stream_key(S.W_MATVEC_Q8_0, 72), rows)
    w[:, 0:2] = HALF_FINITE.view(np.uint8).reshape(-1, 2)
    x = S.normal_f32(S.stream_key(S.W_MATVEC_Q8_0, 73), 2 * cols).reshape(2, cols)
    w = w.reshape(-1)
    dw, dx, dy = ctx.upload(w), ctx.upload(x), ctx.alloc(rows * 2 * 4)
    ctx.matvec(kq_hip.TYPE_Q8_0, dw, rows, cols, dx, 2, dy)
    got = ctx.download(dy, np.float32, rows * 2).reshape(2, rows)
    want = kq_oracle.matvec(kq_oracle.Q8_0, w, rows, cols, x)
    # The integer-dot lane stages each activation as a 22-bit integer of its
    # 16-column group's largest magnitude m (error <= 2^-22 m), so at a
    # near-cancellation the error is bounded by 2^-22 sum|w| m rather than
    # by a multiple of u sum|w x|: 1.7e-7 S measured on this sweep of every
    # binary16 scale, against 7.5e-9 S at most anywhere else. The stage-3
    # bar here is 2^-21 S (a missing 32-column term is about S / 32).
    assert_close(got, want, exact=exact.matvec(kq_oracle.Q8_0, w, rows, cols, x),
                 cond_tol=2.0 ** -21)
    for b in (dw, dx, dy):
        b.close()


def test_dequant_fails_closed(ctx):
    q8 = S.q8_0_blocks(S.stream_key(S.W_DEQUANT, 53), 4)
    q8[2, 0:2] = [0x00, 0x7C]  # +Inf scale
    with pytest.raises(kq_hip.KqError) as e:
        gpu_dequant(ctx, kq_hip.TYPE_Q8_0, q8.reshape(-1))
    assert e.value.name == "MALFORMED_QUANTIZED_DATA"
    dp = ctx.upload(np.zeros(144 * 2, np.uint8))
    do = ctx.alloc(256 * 4)
    with pytest.raises(kq_hip.KqError) as e:
        ctx.dequantize(kq_hip.TYPE_Q4_K, dp, 288, do, 256)  # room for one block only
    assert e.value.name == "BUFFER_TOO_SMALL"
    with pytest.raises(kq_hip.KqError) as e:
        ctx.dequantize(kq_hip.TYPE_Q4_K, dp, 200, do, 256)  # partial block
    assert e.value.name == "MALFORMED_QUANTIZED_DATA"
    # the context stays usable after device-detected failures
    ok = S.q8_0_blocks(S.stream_key(S.W_DEQUANT, 54), 2).reshape(-1)
    assert np.array_equal(gpu_dequant(ctx, kq_hip.TYPE_Q8_0, ok).view(np.uint32),
                          kq_oracle.dequantize(kq_oracle.Q8_0, ok).view(np.uint32))


def test_expf_bit_exact_all_inputs(ctx):
    # Device expf against the oracle's (which equals libm expf on every
    # pattern, see test_oracle_numeric) over all 2^32 bit patterns.
    chunk = 1 << 27
    din = ctx.alloc(chunk * 4)
    dout = ctx.alloc(chunk * 4)
    th = oracle_threads()
    for start in range(0, 1 << 32, chunk):
        if start % (1 << 30) == 0:
            say(f"expf chunk at {start:#x}")
        x = np.arange(start, start + chunk, dtype=np.uint64).astype(np.uint32).view(np.float32)
        d = kq_hip.Diagnostic()
        kq_hip.check(kq_hip.lib().kq_hip_upload(ctx._h, kq_hip.C.c_void_p(din.ptr),
                                                x.ctypes.data, x.nbytes, kq_hip.C.byref(d)), d)
        ctx.expf(din, chunk, dout)
        got = ctx.download(dout, np.float32, chunk)
        want = kq_oracle.expf_array(x, th)
        gb, wb = got.view(np.uint32), want.view(np.uint32)
        diff = gb != wb
        if diff.any():
            both_nan = np.isnan(got) & np.isnan(want)
            diff &= ~both_nan
        assert not diff.any(), f"expf mismatch at {x[diff][:4]}"


def matvec_case(ctx, fmt, rows, cols, batch, key):
    t = FMTS[fmt]
    w = S.quant_matrix(fmt, key, rows, cols)
    x = S.normal_f32(key ^ 0x55, batch * cols).reshape(batch, cols)
    dw, dx = ctx.upload(w), ctx.upload(x)
    dy = ctx.alloc(rows * batch * 4)
    ctx.matvec(t, dw, rows, cols, dx, batch, dy)
    got = ctx.download(dy, np.float32, rows * batch).reshape(batch, rows)
    want = kq_oracle.matvec(t, w, rows, cols, x, threads=oracle_threads())
    for b in (dw, dx, dy):
        b.close()
    return got, want, exact.matvec(t, w, rows, cols, x)


@pytest.mark.parametrize("fmt", ALL_FMTS)
def test_matvec_4096x2048_batch1(ctx, fmt):
    got, want, ex = matvec_case(ctx, fmt, 4096, 2048, 1, S.stream_key(S.W_MATVEC_Q4K, S.R_WEIGHT))
    assert_close(got, want, exact=ex)


@pytest.mark.parametrize("fmt", ALL_FMTS)
@pytest.mark.parametrize("rows,cols,batch", [(1, 256, 1), (7, 512, 2), (33, 1024, 3),
                                             (4097, 2048, 4), (5, 2048, 8), (300, 256, 4)])
def test_matvec_shapes(ctx, fmt, rows, cols, batch):
    got, want, ex = matvec_case(ctx, fmt, rows, cols, batch,
                            S.stream_key(S.W_MATVEC_Q6K, rows, cols, batch))
    assert_close(got, want, exact=ex)


@pytest.mark.parametrize("fmt", ALL_FMTS)
@pytest.mark.parametrize("rows,cols,batch", [(37, 2304, 1), (300, 2560, 2), (5, 4096, 1),
                                             (129, 6144, 1), (64, 10240, 1), (17, 6144, 2),
                                             (9, 4352, 3), (4100, 2560, 1), (3, 12288, 1),
                                             (16500, 2560, 1)])
def test_matvec_wide_rows(ctx, fmt, rows, cols, batch):
    # Rows wider than 2048 columns run as one launch over 2048-column chunks
    # (the last one shorter: 256 .. 2048 columns), or as column segments
    # where no chunk count has an instance (12288 columns, 3 x 4352):
    # every format against the oracle
    got, want, ex = matvec_case(ctx, fmt, rows, cols, batch,
                                S.stream_key(S.W_MATVEC_Q6K, 77, rows * 64 + batch, cols // 256))
    assert_close(got, want, exact=ex)


@pytest.mark.parametrize("fmt", ["Q8_0", "Q4_K"])
def test_lm_head_wide_rows_argmax(ctx, fmt):
    # the LM head's argmax partials from the one-launch wide path
    rows, cols, batch = 9000, 2560, 2
    t = FMTS[fmt]
    w = S.quant_matrix(fmt, S.stream_key(S.W_LM_HEAD, 78, t), rows, cols)
    h = S.normal_f32(S.stream_key(S.W_LM_HEAD, 79, t), batch * cols).reshape(batch, cols)
    dw, dh, dl, di = ctx.upload(w), ctx.upload(h), ctx.alloc(rows * batch * 4), ctx.alloc(batch * 4)
    ctx.lm_head(t, dw, rows, cols, dh, batch, dl, di)
    logits = ctx.download(dl, np.float32, rows * batch).reshape(batch, rows)
    ids = ctx.download(di, np.uint32, batch)
    want = kq_oracle.matvec(t, w, rows, cols, h, threads=oracle_threads())
    assert_close(logits, want, exact=exact.matvec(t, w, rows, cols, h))
    for b in range(batch):
        assert ids[b] == kq_oracle.argmax(logits[b])
    for buf in (dw, dh, dl, di):
        buf.close()


@pytest.mark.parametrize("fmt", ALL_FMTS)
def test_matvec_activation_magnitudes(ctx, fmt):
    # activations over many binades, inside 16-column groups too (the Q4_K
    # matvec scales each group of 16 by one power of two before its integer
    # dots): N(0,1) * 2^U(-20, 20) per element, then whole groups of zeros,
    # of subnormals, of one huge value among tiny ones, and at 2^100
    rows, cols, batch = 257, 2048, 2
    rng = np.random.default_rng(31)
    x = (rng.standard_normal((batch, cols)) *
         np.exp2(rng.uniform(-20, 20, (batch, cols)))).astype(np.float32)
    x[0, 0:16] = 0.0
    x[0, 16:32] = (rng.standard_normal(16) * 1e-40).astype(np.float32)
    x[0, 32:48] = np.float32(1e-30)
    x[0, 40] = np.float32(3e20)
    x[1, 256:272] = (rng.standard_normal(16) * 2.0 ** 100).astype(np.float32)
    x[1, 512:528] = np.float32(-2.0 ** -126)
    t = FMTS[fmt]
    w = S.quant_matrix(fmt, S.stream_key(S.W_MATVEC_Q4K, 31, t), rows, cols)
    dw, dx = ctx.upload(w), ctx.upload(x)
    dy = ctx.alloc(rows * batch * 4)
    ctx.matvec(t, dw, rows, cols, dx, batch, dy)
    got = ctx.download(dy, np.float32, rows * batch).reshape(batch, rows)
    want = kq_oracle.matvec(t, w, rows, cols, x, threads=oracle_threads())
    for b in (dw, dx, dy):
        b.close()
    assert np.isfinite(got).all()
    assert_close(got, want, exact=exact.matvec(t, w, rows, cols, x))


@pytest.mark.parametrize("fmt", ["Q8_0", "Q5_1", "IQ4_NL"])
@pytest.mark.parametrize("cols", [32, 64, 128])
def test_matvec_short_rows(ctx, fmt, cols):
    # 32-weight formats: rows of one to four blocks
    got, want, ex = matvec_case(ctx, fmt, 130, cols, 2, S.stream_key(S.W_MATVEC_Q8_0, cols, FMTS[fmt]))
    assert_close(got, want, exact=ex)


@pytest.mark.parametrize("fmt", ["Q8_0", "Q5_1", "IQ4_NL"])
@pytest.mark.parametrize("rows", [1, 3, 7])
def test_matvec_last_block_of_buffer(ctx, fmt, rows):
    # An odd number of 32-weight blocks: the buffer's last block ends off a
    # dword boundary, where no load may reach past the buffer.
    got, want, ex = matvec_case(ctx, fmt, rows, 32, 1, S.stream_key(S.W_MATVEC_Q8_0, rows, FMTS[fmt]))
    assert_close(got, want, exact=ex)


@pytest.mark.parametrize("fmt", ["F32", "BF16"])
def test_dequant_elements_bit_exact(ctx, fmt):
    # element types decode to their own bits (F32) or bits << 16 (BF16),
    # NaN and infinity patterns included
    n = 1_000_003
    raw = S.random_bytes(S.stream_key(S.W_DEQUANT, S.R_WEIGHT, ELEM[fmt]),
                         n * (4 if fmt == "F32" else 2))
    got = gpu_dequant(ctx, ELEM[fmt], raw)
    want = kq_oracle.dequantize(ELEM[fmt], raw)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("case", [c for c in NUM["row_dot_cases"] if c["type"] in FMTS],
                         ids=lambda c: c["id"])
def test_row_dot_golden(ctx, case):
    src = {c["id"]: c for c in NUM["cases"]}[case["source_case_id"]]
    packed = np.frombuffer(bytes.fromhex(src["packed_hex"]), np.uint8).copy()
    x = bits_f32(case["activation_f32_bits"])
    dp, dx, do = ctx.upload(packed), ctx.upload(x), ctx.alloc(4)
    ctx.row_dot(FMTS[case["type"]], dp, packed.size, dx, x.size, do)
    got = ctx.download(do, np.float32, 1)[0]
    want = bits_f32(case["expected_f32_bits"])[0]
    assert abs(float(got) - float(want)) <= ATOL + RTOL * abs(float(want))


def test_matvec_fails_closed(ctx):
    w = S.quant_matrix("Q4_K", S.stream_key(S.W_MATVEC_Q4K, 77), 16, 512)
    x = S.normal_f32(S.stream_key(S.W_MATVEC_Q4K, 78), 512)
    x_bad = x.copy()
    x_bad[100] = np.nan
    dw, dx, dxb, dy = ctx.upload(w), ctx.upload(x), ctx.upload(x_bad), ctx.alloc(16 * 4)
    with pytest.raises(kq_hip.KqError) as e:
        ctx.matvec(kq_hip.TYPE_Q4_K, dw, 16, 512, dxb, 1, dy)
    assert e.value.name == "NUMERIC_DOMAIN"
    w_bad = w.copy().reshape(-1, 144)
    w_bad[5, 0:2] = [0x00, 0xFC]  # -Inf d
    dwb = ctx.upload(w_bad.reshape(-1))
    with pytest.raises(kq_hip.KqError) as e:
        ctx.matvec(kq_hip.TYPE_Q4_K, dwb, 16, 512, dx, 1, dy)
    assert e.value.name == "MALFORMED_QUANTIZED_DATA"
    with pytest.raises(kq_hip.KqError) as e:
        ctx.matvec(kq_hip.TYPE_Q4_K, dw, 16, 512, dx, 1, dy, capacity=15)
    assert e.value.name == "BUFFER_TOO_SMALL"
    with pytest.raises(kq_hip.KqError) as e:
        ctx.matvec(kq_hip.TYPE_Q4_K, dw, 16, 500, dx, 1, dy)
    assert e.value.name == "DIMENSION_MISMATCH"
    with pytest.raises(kq_hip.KqError) as e:
        ctx.matvec(kq_hip.TYPE_Q4_K, dw, 16, 512, dw, 1, dw.ptr + 64)
    assert e.value.name == "ALIASING_VIOLATION"
    ctx.matvec(kq_hip.TYPE_Q4_K, dw, 16, 512, dx, 1, dy)  # still usable


@pytest.mark.parametrize("rows,cols,batch,scale", [
    (65536, 256, 2, 1.0), (70001, 2048, 3, 1.0), (65537, 4096, 4, 1e-30),
    (66000, 1024, 2, 1e6), (65600, 512, 4, 1.0), (65551, 2048, 4, 1.0)])
def test_matvec_q6k_batched_mfma(ctx, rows, cols, batch, scale):
    # Q6_K with 2..4 activation columns on at least 65,536 rows runs on
    # MFMA (exact fp16 codes, activation columns as fp16 hi + lo after a
    # power-of-two scaling): ragged last tiles, 1 .. 16 blocks per row, tiny
    # and large activations (compared relative to their scale)
    say(f"q6k mfma {rows}x{cols} batch {batch} scale {scale}")
    key = S.stream_key(S.W_MATVEC_Q6K, rows, cols, batch)
    w = S.quant_matrix("Q6_K", key, rows, cols)
    x = (S.normal_f32(key ^ 0x55, batch * cols) * np.float32(scale)).reshape(batch, cols)
    dw, dx, dy = ctx.upload(w), ctx.upload(x), ctx.alloc(rows * batch * 4)
    ctx.matvec(kq_hip.TYPE_Q6_K, dw, rows, cols, dx, batch, dy)
    got = ctx.download(dy, np.float32, rows * batch).reshape(batch, rows)
    want = kq_oracle.matvec(kq_oracle.Q6_K, w, rows, cols, x, threads=oracle_threads())
    ex = exact.matvec(kq_oracle.Q6_K, w, rows, cols, x)
    assert_close(got.astype(np.float64) / scale, want.astype(np.float64) / scale,
                 exact=lambda i: ex(i) / scale)
    for b in (dw, dx, dy):
        b.close()


@pytest.mark.parametrize("cols", [256, 2048])
def test_matvec_q6k_batched_mfma_fails_closed(ctx, cols):
    # 2,048 columns run on the tile-shared kernel, the other widths on the
    # per-wave block rings
    rows = 65536
    w = S.quant_matrix("Q6_K", S.stream_key(S.W_MATVEC_Q6K, 91), rows, cols)
    x = S.normal_f32(S.stream_key(S.W_MATVEC_Q6K, 92), 2 * cols).reshape(2, cols)
    x_bad = x.copy()
    x_bad[1, 17] = np.inf
    dw, dx, dxb, dy = ctx.upload(w), ctx.upload(x), ctx.upload(x_bad), ctx.alloc(rows * 2 * 4)
    with pytest.raises(kq_hip.KqError) as e:
        ctx.matvec(kq_hip.TYPE_Q6_K, dw, rows, cols, dxb, 2, dy)
    assert e.value.name == "NUMERIC_DOMAIN"
    w_bad = w.copy().reshape(-1, 210)
    w_bad[40000, 208:210] = [0x00, 0x7C]  # +Inf d
    dwb = ctx.upload(w_bad.reshape(-1))
    with pytest.raises(kq_hip.KqError) as e:
        ctx.matvec(kq_hip.TYPE_Q6_K, dwb, rows, cols, dx, 2, dy)
    assert e.value.name == "MALFORMED_QUANTIZED_DATA"
    ctx.matvec(kq_hip.TYPE_Q6_K, dw, rows, cols, dx, 2, dy)  # still usable
    got = ctx.download(dy, np.float32, rows * 2).reshape(2, rows)
    assert_close(got, kq_oracle.matvec(kq_oracle.Q6_K, w, rows, cols, x,
                                       threads=oracle_threads()),
                 exact=exact.matvec(kq_oracle.Q6_K, w, rows, cols, x))


def test_argmax_exact(ctx):
    rng = np.random.default_rng(9)
    v = rng.standard_normal((3, 151936)).astype(np.float32)
    v[1, 5000] = v[1, 90000] = v[1].max() + 1  # tie -> lower id
    v[2, :] = 0.0
    v[2, 77] = -0.0  # +0 and -0 compare equal: first occurrence wins
    dv, di = ctx.upload(v), ctx.alloc(3 * 4)
    ctx.argmax(dv, 151936, 3, di)
    got = ctx.download(di, np.uint32, 3)
    assert list(got) == [kq_oracle.argmax(v[b]) for b in range(3)] == [int(np.argmax(v[0])), 5000, 0]
    v[0, 10] = np.inf
    dv2 = ctx.upload(v)
    with pytest.raises(kq_hip.KqError) as e:
        ctx.argmax(dv2, 151936, 3, di)
    assert e.value.name == "NUMERIC_DOMAIN"


@pytest.mark.parametrize("batch", [1, 4])
def test_lm_head_q6k_151936x2048(ctx, batch):
    V, H = 151936, 2048
    say(f"lm head batch {batch}")
    w = S.quant_matrix("Q6_K", S.stream_key(S.W_LM_HEAD, S.R_WEIGHT), V, H)
    h = S.normal_f32(S.stream_key(S.W_LM_HEAD, S.R_HIDDEN, batch), batch * H).reshape(batch, H)
    dw, dh = ctx.upload(w), ctx.upload(h)
    dl, di = ctx.alloc(V * batch * 4), ctx.alloc(batch * 4)
    ctx.lm_head(kq_hip.TYPE_Q6_K, dw, V, H, dh, batch, dl, di)
    logits = ctx.download(dl, np.float32, V * batch).reshape(batch, V)
    ids = ctx.download(di, np.uint32, batch)
    ref = kq_oracle.matvec(kq_oracle.Q6_K, w, V, H, h, threads=oracle_threads())
    assert_close(logits, ref, exact=exact.matvec(kq_oracle.Q6_K, w, V, H, h))
    for b in range(batch):
        # exact on the device's own logits; equal to the CPU's where the
        # CPU top-2 margin exceeds the tolerance
        assert ids[b] == int(np.argmax(logits[b]))
        top2 = np.sort(ref[b])[-2:]
        if top2[1] - top2[0] > ATOL + RTOL * abs(top2[1]):
            assert ids[b] == kq_oracle.argmax(ref[b])


@pytest.mark.parametrize("fmt,rows,cols,batch", [
    ("Q8_0", 300, 2560, 1), ("Q8_0", 257, 6144, 2), ("Q8_0", 65, 10240, 1),
    ("Q8_0", 1000, 320, 3), ("Q8_0", 640, 640, 1), ("Q5_1", 300, 640, 2),
    ("IQ4_NL", 300, 2560, 1), ("Q4_K", 640, 2560, 1), ("Q5_K", 640, 2560, 4),
    ("Q6_K", 129, 6144, 1), ("Q4_K", 33, 2304, 3)])
def test_matvec_long_rows(ctx, fmt, rows, cols, batch):
    # Rows of the reference model's widths (hidden 2560, expert 640, the
    # 6144- and 10240-wide GDN and hyper-connection projections, 320): the
    # row runs as column segments of supported widths, each one launch
    # adding to the previous segments' sums.
    got, want, ex = matvec_case(ctx, fmt, rows, cols, batch,
                            S.stream_key(S.W_MATVEC_Q8_0, rows, cols, FMTS[fmt]))
    assert_close(got, want, exact=ex)


def test_lm_head_q8_0_248320x2560(ctx):
    # The reference model's LM head (Q8_0, vocabulary 248,320, hidden 2560):
    # two segments, the argmax taken over the finished sums.
    V, H = 248320, 2560
    say("lm head q8_0 248320x2560")
    w = S.quant_matrix("Q8_0", S.stream_key(S.W_LM_HEAD, S.R_WEIGHT, 8), V, H)
    h = S.normal_f32(S.stream_key(S.W_LM_HEAD, S.R_HIDDEN, 8), H)[None, :]
    dw, dh = ctx.upload(w), ctx.upload(h)
    dl, di = ctx.alloc(V * 4), ctx.alloc(4)
    ctx.lm_head(kq_hip.TYPE_Q8_0, dw, V, H, dh, 1, dl, di)
    logits = ctx.download(dl, np.float32, V)[None, :]
    ids = ctx.download(di, np.uint32, 1)
    ref = kq_oracle.matvec(kq_oracle.Q8_0, w, V, H, h, threads=oracle_threads())
    assert_close(logits, ref, exact=exact.matvec(kq_oracle.Q8_0, w, V, H, h))
    assert ids[0] == int(np.argmax(logits[0]))
    top2 = np.sort(ref[0])[-2:]
    if top2[1] - top2[0] > ATOL + RTOL * abs(top2[1]):
        assert ids[0] == kq_oracle.argmax(ref[0])
    for b in (dw, dh, dl, di):
        b.close()


@pytest.mark.parametrize("V,batch", [(40000, 5), (40000, 6), (40000, 8), (65600, 5)])
def test_lm_head_batch_spans_launches(ctx, V, batch):
    # batches over 4 run as several launches whose wave counts differ (at
    # 65,600 rows the first four columns run on MFMA, the fifth on the row
    # engine); the argmax partials of every batch row must still merge to
    # the first max
    H = 2048
    say(f"lm head {V}x{H} batch {batch}")
    w = S.quant_matrix("Q6_K", S.stream_key(S.W_LM_HEAD, S.R_WEIGHT, 7), V, H)
    h = S.normal_f32(S.stream_key(S.W_LM_HEAD, S.R_HIDDEN, 70 + batch), batch * H).reshape(batch, H)
    dw, dh = ctx.upload(w), ctx.upload(h)
    dl, di = ctx.alloc(V * batch * 4), ctx.alloc(batch * 4)
    ctx.lm_head(kq_hip.TYPE_Q6_K, dw, V, H, dh, batch, dl, di)
    logits = ctx.download(dl, np.float32, V * batch).reshape(batch, V)
    ids = ctx.download(di, np.uint32, batch)
    ref = kq_oracle.matvec(kq_oracle.Q6_K, w, V, H, h, threads=oracle_threads())
    assert_close(logits, ref, exact=exact.matvec(kq_oracle.Q6_K, w, V, H, h))
    for b in range(batch):
        assert ids[b] == int(np.argmax(logits[b]))
