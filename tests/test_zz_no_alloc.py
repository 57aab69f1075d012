"""The allocation-free LM head (kq_hip_lm_head_greedy_f32_noalloc) against
kq_hip_lm_head_greedy_f32, through the C ABI: the same kernels with the
argmax partials in the library's static device array instead of the
context's, so logits and token ids must be identical bit for bit. Two
calls in a row, the second smaller, so stale partials from the first call
would show in the second's ids."""
import numpy as np
import pytest

import kq_hip
import kq_synth as S

pytestmark = pytest.mark.gpu


def run(fmt, V, H, batch, seed, noalloc):
    t = kq_hip.TYPE_IDS[fmt]
    w = S.quant_matrix(fmt, S.stream_key(S.W_LM_HEAD, S.R_WEIGHT, seed), V, H)
    h = S.normal_f32(S.stream_key(S.W_LM_HEAD, S.R_HIDDEN, seed), batch * H)
    with kq_hip.Context(0) as ctx:
        dw, dh = ctx.upload(w), ctx.upload(h)
        dl, di = ctx.alloc(V * batch * 4), ctx.alloc(batch * 4)
        ctx.lm_head(t, dw, V, H, dh, batch, dl, di, noalloc=noalloc)
        logits = ctx.download(dl, np.float32, V * batch).reshape(batch, V)
        ids = ctx.download(di, np.uint32, batch)
    return logits, ids


# (format, vocab, hidden, batch, seed), each call smaller than the one
# before: the reference model's Q8_0 head at batch 8 (two launches of four
# columns on the row engine, the most partials any call here needs), the
# Q6_K head at batch 4 (MFMA path), then a small head at batch 2
CALLS = [("Q8_0", 248320, 2560, 8, 3), ("Q6_K", 151936, 2048, 4, 1),
         ("Q8_0", 40000, 2560, 2, 2)]


def test_noalloc_lm_head_matches_allocating_entry():
    print("noalloc lm head: three calls, each smaller than the one before", flush=True)
    got = []
    for fmt, V, H, batch, seed in CALLS:
        print(f"  noalloc {fmt} {V}x{H} batch {batch}", flush=True)
        got.append(run(fmt, V, H, batch, seed, True))
    for (fmt, V, H, batch, seed), (lg, ig) in zip(CALLS, got):
        print(f"  allocating {fmt} {V}x{H} batch {batch}", flush=True)
        lw, iw = run(fmt, V, H, batch, seed, False)
        assert np.array_equal(lg.view(np.uint32), lw.view(np.uint32)), fmt
        assert np.array_equal(ig, iw), (fmt, ig, iw)
        assert list(ig) == [int(np.argmax(lg[b])) for b in range(batch)]


def test_noalloc_lm_head_same_context():
    # the smaller two calls on one context, each entry point in turn; then a
    # batch above the matvec limit is refused before any launch. (The
    # static array's own LIMIT_EXCEEDED cannot be reached: no launch shape
    # needs more than 16,384 partials per column, 131,072 at 8 columns,
    # which is the array's size.)
    with kq_hip.Context(0) as ctx:
        outs = []
        for fmt, V, H, batch, seed in CALLS[1:]:
            t = kq_hip.TYPE_IDS[fmt]
            w = S.quant_matrix(fmt, S.stream_key(S.W_LM_HEAD, S.R_WEIGHT, seed), V, H)
            h = S.normal_f32(S.stream_key(S.W_LM_HEAD, S.R_HIDDEN, seed), batch * H)
            dw, dh = ctx.upload(w), ctx.upload(h)
            dl, di = ctx.alloc(V * batch * 4), ctx.alloc(batch * 4)
            ctx.lm_head(t, dw, V, H, dh, batch, dl, di, noalloc=True)
            a = (ctx.download(dl, np.float32, V * batch), ctx.download(di, np.uint32, batch))
            ctx.lm_head(t, dw, V, H, dh, batch, dl, di, noalloc=False)
            b = (ctx.download(dl, np.float32, V * batch), ctx.download(di, np.uint32, batch))
            assert np.array_equal(a[0].view(np.uint32), b[0].view(np.uint32))
            assert np.array_equal(a[1], b[1])
            outs.append((dw, dh, dl, di, t, V, H))
        dw, dh, dl, di, t, V, H = outs[-1]
        with pytest.raises(kq_hip.KqError) as e:
            ctx.lm_head(t, dw, V, H, dh, 9, dl, di, noalloc=True)
        assert e.value.name == "LIMIT_EXCEEDED"
