"""Device tensor views and GDN canonical-order copies, through the C ABI.

Bars: block-range dequant of a view bit-exact with the oracle's decode of
the same blocks (kq_dequantize_view_blocks_f32, src/kq_numeric.c:361-418),
with the reference's statuses; the canonical copy of a GDN tensor equal byte
for byte to the numpy re-layout of the stored tensor; the matvec on that
copy per element within 1e-4 absolute or 1e-3 relative of the oracle's
restatement of the provider's GDN linear on the stored tensor
(physical_row_for, the GDN_OUT activation permutation,
src/kq_weight_provider.c:205-248, :438-475), or of the binary64 value, at
the reference model's full shapes."""
import numpy as np
import pytest

from conftest import assert_close, oracle_threads

import exact
import kq_hip
import kq_oracle
import kq_synth as S

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def ctx():
    c = kq_hip.Context(0)
    yield c
    c.close()


FMTS = ["Q4_K", "Q5_K", "Q6_K", "Q8_0", "Q5_1", "IQ4_NL"]


@pytest.mark.parametrize("fmt", FMTS)
def test_view_block_ranges_bit_exact(ctx, fmt):
    # ranges starting on odd blocks (off the decoder's alignment for the
    # 34-, 18- and 210-byte formats), in the middle, and the last block
    t = kq_hip.TYPE_IDS[fmt]
    gen, qk, bb = S.BLOCK_GEN[fmt]
    nblk = 1001
    packed = gen(S.stream_key(S.W_DEQUANT, 80, t), nblk).reshape(-1)
    buf = ctx.upload(packed)
    view = kq_hip.tensor_view(t, buf, packed.size)
    out = ctx.alloc(nblk * qk * 4)
    for first, count in [(0, 1), (1, 1), (3, 17), (500, 501), (1000, 1), (7, 994)]:
        n = ctx.dequantize_view(view, first, count, kq_hip.CANONICAL_ORDER, out, count * qk)
        assert n == count * qk
        got = ctx.download(out, np.float32, n)
        want = kq_oracle.dequantize(t, packed[first * bb:(first + count) * bb])
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (first, count)
    buf.close()
    out.close()


def test_view_statuses(ctx):
    t = kq_hip.TYPE_Q8_0
    packed = S.q8_0_blocks(S.stream_key(S.W_DEQUANT, 81), 16).reshape(-1)
    buf, out = ctx.upload(packed), ctx.alloc(16 * 32 * 4)
    tv = kq_hip.tensor_view(t, buf, packed.size, kq_hip.LAYOUT_TRANSFORMED)
    # a transformed (GDN) view decodes in physical order only
    assert ctx.dequantize_view(tv, 2, 3, kq_hip.PHYSICAL_ORDER, out, 96) == 96
    with pytest.raises(kq_hip.KqError) as e:
        ctx.dequantize_view(tv, 2, 3, kq_hip.CANONICAL_ORDER, out, 96)
    assert e.value.name == "TENSOR_LAYOUT_MISMATCH"
    cv = kq_hip.tensor_view(t, buf, packed.size)
    for first, count in [(15, 2), (16, 1), (2 ** 64 - 1, 2)]:
        with pytest.raises(kq_hip.KqError) as e:
            ctx.dequantize_view(cv, first, count, kq_hip.PHYSICAL_ORDER, out, 512)
        assert e.value.name == "SPAN_OUT_OF_RANGE"
    with pytest.raises(kq_hip.KqError) as e:
        ctx.dequantize_view(cv, 0, 3, 7, out, 96)
    assert e.value.name == "INVALID_ARGUMENT"
    with pytest.raises(kq_hip.KqError) as e:  # capacity for two blocks only
        ctx.dequantize_view(cv, 1, 3, kq_hip.PHYSICAL_ORDER, out, 64)
    assert e.value.name == "BUFFER_TOO_SMALL"
    broken = kq_hip.tensor_view(t, buf, packed.size)
    broken.bytes_per_block = 18
    with pytest.raises(kq_hip.KqError) as e:
        ctx.dequantize_view(broken, 0, 1, kq_hip.PHYSICAL_ORDER, out, 32)
    assert e.value.name == "TENSOR_OWNERSHIP_MISMATCH"
    buf.close()
    out.close()


def relayout(packed, fmt, layout, rows, cols):
    """The canonical copy by numpy: rows (or 128-column units) gathered by
    the reshape/transpose form of the GDN order."""
    gen, qk, bb = S.BLOCK_GEN[fmt]
    rb = cols // qk * bb
    m = packed.reshape(rows, rb)
    tiled = lambda w: np.arange(48 * w).reshape(3, 16, w).transpose(1, 0, 2).reshape(-1)
    if layout == "out":
        ub = 128 // qk * bb
        u = m.reshape(rows, 48, ub)
        return np.ascontiguousarray(u[:, tiled(1), :]).reshape(-1)
    prefix = 4096 if layout in ("qkv", "conv") else 0
    w = 1 if layout in ("alpha", "beta") else 128
    order = np.concatenate([np.arange(prefix), prefix + tiled(w)])
    return np.ascontiguousarray(m[order]).reshape(-1)


# the reference model's GDN tensors (research/model-gguf inventory: Q8_0)
GDN = [("qkv", "Q8_0", 10240, 2560), ("gate", "Q8_0", 6144, 2560), ("out", "Q8_0", 2560, 6144),
       ("alpha", "Q8_0", 48, 2560), ("beta", "Q8_0", 48, 2560), ("out", "IQ4_NL", 300, 6144),
       ("gate", "Q4_K", 6144, 512), ("qkv", "Q6_K", 10240, 256)]


@pytest.mark.parametrize("layout,fmt,rows,cols", GDN, ids=[f"{g[0]}-{g[1]}-{g[2]}x{g[3]}" for g in GDN])
def test_gdn_canonical_matvec(ctx, layout, fmt, rows, cols):
    t = kq_hip.TYPE_IDS[fmt]
    key = S.stream_key(S.W_MATVEC_Q8_0, 90, rows, cols)
    packed = S.quant_matrix(fmt, key, rows, cols)
    x = S.normal_f32(key ^ 0x77, cols)
    dp, dc = ctx.upload(packed), ctx.alloc(packed.size)
    ctx.gdn_canonicalize(layout, t, dp, rows, cols, dc, packed.size)
    canon = ctx.download(dc, np.uint8, packed.size)
    assert np.array_equal(canon, relayout(packed, fmt, layout, rows, cols))
    dx, dy = ctx.upload(x), ctx.alloc(rows * 4)
    ctx.matvec(t, dc, rows, cols, dx, 1, dy)
    got = ctx.download(dy, np.float32, rows)[None, :]
    want = kq_oracle.gdn_linear(layout, t, packed, rows, cols, x, threads=oracle_threads())
    assert_close(got, want[None, :], exact=exact.matvec(t, canon, rows, cols, x))
    for b in (dp, dc, dx, dy):
        b.close()


def test_gdn_canonicalize_statuses(ctx):
    t = kq_hip.TYPE_Q8_0
    packed = S.quant_matrix("Q8_0", S.stream_key(S.W_MATVEC_Q8_0, 91), 48, 256)
    dp, dc = ctx.upload(packed), ctx.alloc(packed.size)
    with pytest.raises(kq_hip.KqError) as e:  # 48 rows are not the gate's 6144
        ctx.gdn_canonicalize("gate", t, dp, 48, 256, dc, packed.size)
    assert e.value.name == "TENSOR_LAYOUT_MISMATCH"
    with pytest.raises(kq_hip.KqError) as e:
        ctx.gdn_canonicalize("alpha", t, dp, 48, 256, dc, packed.size - 1)
    assert e.value.name == "BUFFER_TOO_SMALL"
    with pytest.raises(kq_hip.KqError) as e:
        ctx.gdn_canonicalize("alpha", t, dp, 48, 256, dp, packed.size)
    assert e.value.name == "ALIASING_VIOLATION"
    q4 = S.quant_matrix("Q4_K", S.stream_key(S.W_MATVEC_Q8_0, 92), 2, 6144)
    d4, c4 = ctx.upload(q4), ctx.alloc(q4.size)
    with pytest.raises(kq_hip.KqError) as e:  # 256-element blocks span two units
        ctx.gdn_canonicalize("out", kq_hip.TYPE_Q4_K, d4, 2, 6144, c4, q4.size)
    assert e.value.name == "UNSUPPORTED_TENSOR_TYPE"
    # no layout: a plain copy
    ctx.gdn_canonicalize("none", t, dp, 48, 256, dc, packed.size)
    assert np.array_equal(ctx.download(dc, np.uint8, packed.size), packed)
    for b in (dp, dc, d4, c4):
        b.close()
