"""Host-side layout arithmetic of the C ABI, on the CPU: element ranges to
blocks against the reference's own kq_quant_element_to_block /
kq_quant_range_to_blocks (oracle/_ref, where it is built), the GDN row and
column maps against the oracle's restatement of physical_row_for /
grouped_to_tiled (src/kq_weight_provider.c:205-248) and an independent
reshape/transpose form, and tensor-view set-up. Nothing here launches
device work."""
import numpy as np
import pytest

import kq_hip
import kq_oracle
import kq_ref as R

TYPES = [kq_hip.TYPE_Q4_K, kq_hip.TYPE_Q8_0, kq_hip.TYPE_Q6_K, kq_hip.TYPE_Q5_1,
         kq_hip.TYPE_Q5_K, kq_hip.TYPE_IQ4_NL, kq_hip.TYPE_F32, kq_hip.TYPE_BF16]
SPAN = ("requested_element_offset", "requested_element_count", "first_block", "block_count",
        "physical_byte_offset", "physical_byte_length", "leading_elements",
        "trailing_elements")


def ours_range(t, total, off, cnt):
    try:
        sp = kq_hip.range_to_blocks(t, total, off, cnt)
        return 0, tuple(getattr(sp, n) for n in SPAN)
    except kq_hip.KqError as e:
        return e.status, (0,) * 8


def ours_elem(t, total, i):
    try:
        b, w = kq_hip.element_to_block(t, total, i)
        return 0, b, w
    except kq_hip.KqError as e:
        return e.status, 0, 0


@pytest.mark.skipif(not R.available(), reason="oracle/_ref not built (needs the reference sources)")
def test_ranges_match_reference():
    rng = np.random.default_rng(5)
    cases = [(kq_hip.TYPE_Q4_K, 4096, 0, 4096), (kq_hip.TYPE_Q4_K, 4096, 255, 2),
             (kq_hip.TYPE_Q8_0, 64, 63, 1), (kq_hip.TYPE_Q8_0, 64, 64, 1),
             (kq_hip.TYPE_Q8_0, 64, 10, 0), (kq_hip.TYPE_Q6_K, 100, 0, 1),
             (kq_hip.TYPE_Q8_0, 2 ** 64 - 32, 2 ** 64 - 40, 16), (2, 256, 0, 1)]
    for _ in range(4000):
        t = TYPES[rng.integers(len(TYPES))]
        be = kq_hip.GEOMETRY[t][0]
        total = int(rng.integers(1, 64)) * be + (be // 2 if rng.random() < 0.1 else 0)
        off = int(rng.integers(0, total + 2))
        cnt = int(rng.integers(0, total + 2 - min(off, total)))
        cases.append((t, total, off, cnt))
    for t, total, off, cnt in cases:
        if t == kq_hip.TYPE_Q6_K:
            continue  # the reference has no Q6_K: closed form below
        assert ours_range(t, total, off, cnt) == R.range_to_blocks(t, total, off, cnt), \
            (t, total, off, cnt)
        assert ours_elem(t, total, off) == R.element_to_block(t, total, off), (t, total, off)


def test_q6k_ranges_closed_form():
    # 256-element blocks of 210 bytes
    for total, off, cnt in [(256 * 9, 300, 700), (256, 0, 256), (512, 511, 1)]:
        st, sp = ours_range(kq_hip.TYPE_Q6_K, total, off, cnt)
        first, last = off // 256, (off + cnt - 1) // 256 + 1
        assert st == 0 and sp == (off, cnt, first, last - first, 210 * first,
                                  210 * (last - first), off - 256 * first,
                                  256 * last - off - cnt)
    assert ours_range(kq_hip.TYPE_Q6_K, 300, 0, 1)[0] == 25  # not whole blocks


# canonical index -> physical index of a 48-unit region of width w: the
# canonical order is [16 key heads][3 repeats][w], the physical one
# [3 repeats][16 key heads][w]
def tiled(w):
    return np.arange(48 * w).reshape(3, 16, w).transpose(1, 0, 2).reshape(-1)


@pytest.mark.parametrize("layout,n,prefix,w,columns", [
    ("qkv", 10240, 4096, 128, False), ("conv", 10240, 4096, 128, False),
    ("gate", 6144, 0, 128, False), ("alpha", 48, 0, 1, False), ("beta", 48, 0, 1, False),
    ("out", 6144, 0, 128, True)])
def test_gdn_maps(layout, n, prefix, w, columns):
    want = np.concatenate([np.arange(prefix), prefix + tiled(w)])
    ours = np.array([kq_hip.gdn_physical_index(layout, n, i, columns) for i in range(n)])
    orc = np.array([(kq_oracle.gdn_physical_column if columns else kq_oracle.gdn_physical_row)
                    (layout, i) for i in range(n)])
    assert np.array_equal(ours, want) and np.array_equal(orc, want)
    assert np.array_equal(np.sort(want), np.arange(n))  # a permutation
    # a few values by hand: value row 128 of attn_qkv is the second repeat
    # of key head 0, stored after all 16 key heads' first repeats
    if layout == "qkv":
        assert ours[4096] == 4096 and ours[4096 + 128] == 4096 + 16 * 128
        assert ours[4096 + 384] == 4096 + 128 and ours[4095] == 4095
    # a geometry the layout does not map onto itself is refused
    with pytest.raises(kq_hip.KqError) as e:
        kq_hip.gdn_physical_index(layout, n + (1 if w == 1 else 128), 0, columns)
    assert e.value.name == "TENSOR_LAYOUT_MISMATCH"
    # the other axis is untouched
    assert kq_hip.gdn_physical_index(layout, 12345, 777, not columns) == 777


def test_tensor_view_init():
    v = kq_hip.tensor_view(kq_hip.TYPE_Q6_K, 0x10000, 210 * 7)
    assert (v.block_count, v.block_elements, v.bytes_per_block, v.canonical_contiguous) == \
        (7, 256, 210, 1)
    v = kq_hip.tensor_view(kq_hip.TYPE_Q8_0, 0x10000, 34 * 4, kq_hip.LAYOUT_TRANSFORMED)
    assert v.canonical_contiguous == 0
    with pytest.raises(kq_hip.KqError) as e:
        kq_hip.tensor_view(kq_hip.TYPE_Q8_0, 0x10000, 35)
    assert e.value.name == "MALFORMED_QUANTIZED_DATA"
    with pytest.raises(kq_hip.KqError) as e:
        kq_hip.tensor_view(2, 0x10000, 18)
    assert e.value.name == "UNSUPPORTED_TENSOR_TYPE"
