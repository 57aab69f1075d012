"""The C ABI's contracts at the reference's boundary, on the device:

- kq_hip_moe_route_f32's shape and capacity checks (include/kq_moe.h:128-141,
  src/kq_moe_qwen38.c:293-349): router weight count, output capacities in
  values with BUFFER_TOO_SMALL, overlapping outputs;
- kq_hip_moe_execute_routed_expert_f32 (include/kq_moe.h:143-152,
  src/kq_moe_qwen38.c:461-566): bit-identical to the oracle, which is
  itself checked bit for bit against the reference's own function
  (tests/test_oracle_vs_reference.py), plus its statuses;
- commit on success (src/kq_weight_provider.c:420, :480): a synchronous call
  that fails leaves its device outputs as they were."""
import numpy as np
import pytest

import kq_hip
import kq_oracle
import kq_synth as S

pytestmark = pytest.mark.gpu

SENTINEL = np.float32(-1234.5)


@pytest.fixture(scope="module")
def ctx():
    c = kq_hip.Context(0)
    yield c
    c.close()


def say(*a):
    print(*a, flush=True)


def filled(ctx, n, dtype=np.float32, value=SENTINEL):
    return ctx.upload(np.full(n, value, dtype))


def unchanged(ctx, buf, n, dtype=np.float32, value=SENTINEL):
    return np.array_equal(ctx.download(buf, dtype, n), np.full(n, value, dtype))


def status_of(fn):
    with pytest.raises(kq_hip.KqError) as e:
        fn()
    return e.value


# ---------------- route capacities ----------------

def test_route_capacities_and_shape(ctx):
    H, E, K, T = 2048, 512, 10, 2
    say(f"route capacities H={H} E={E} K={K} T={T}")
    router = S.normal_f32(S.stream_key(S.W_MOE, S.R_ROUTER, 71), E * H, 0.02)
    sgw = S.normal_f32(S.stream_key(S.W_MOE, S.R_ROUTER, 72), H, 0.02)
    x = S.normal_f32(S.stream_key(S.W_MOE, S.R_HIDDEN, 73), T * H)
    cfg = kq_hip.MoeConfig(H, E, K, 256, 256)
    n = cfg.scratch_bytes(T)
    dr, dsg, dx, ds = ctx.upload(router), ctx.upload(sgw), ctx.upload(x), ctx.alloc(n)
    dl, dp = filled(ctx, T * E + 8), filled(ctx, T * E + 8)
    di, dw = filled(ctx, T * K + 8, np.uint32, 7), filled(ctx, T * K + 8)

    def route(rc=None, caps=None, outs=(dl, dp, di, dw)):
        ctx.moe_route(cfg, dr, dsg, dx, T, *outs, ds, n, router_count=rc, caps=caps)

    full = (T * E, T * E, T * K, T * K)
    for i in range(4):
        caps = list(full)
        caps[i] -= 1
        e = status_of(lambda: route(caps=tuple(caps)))
        assert e.name == "BUFFER_TOO_SMALL"
        assert f"{T * E} values" in str(e) and f"{T * K}" in str(e)
    assert status_of(lambda: route(rc=E * H - 1)).name == "DIMENSION_MISMATCH"
    assert status_of(lambda: route(outs=(dl, dl, di, dw))).name == "ALIASING_VIOLATION"
    assert status_of(lambda: route(outs=(dl, dp, di, di))).name == "ALIASING_VIOLATION"
    assert status_of(lambda: route(outs=(dl, dp, dx, dw))).name == "ALIASING_VIOLATION"
    # every rejection came before any device work: the outputs are untouched
    assert unchanged(ctx, dl, T * E + 8) and unchanged(ctx, di, T * K + 8, np.uint32, 7)
    # larger capacities are accepted; the values past the tokens' stay as they were
    route(caps=(T * E + 8, T * E + 8, T * K + 8, T * K + 8))
    dims = dict(hidden=H, experts=E, top_k=K, inter=1, shared_inter=1)
    xs = x.reshape(T, H)
    want = [kq_oracle.moe_route(dims, (kq_oracle.F32, router), xs[t]) for t in range(T)]
    got_l = ctx.download(dl, np.float32, T * E + 8)
    got_i = ctx.download(di, np.uint32, T * K + 8)
    assert np.array_equal(got_l[:T * E].view(np.uint32),
                          np.concatenate([w[0] for w in want]).view(np.uint32))
    assert np.array_equal(got_i[:T * K], np.concatenate([w[2] for w in want]))
    assert np.all(got_l[T * E:] == SENTINEL) and np.all(got_i[T * K:] == 7)
    # a non-finite router weight: NUMERIC_DOMAIN, and no output is written
    bad = router.copy()
    bad[5 * H + 17] = np.nan
    dbad = ctx.upload(bad)
    dl2 = filled(ctx, T * E)
    e = status_of(lambda: ctx.moe_route(cfg, dbad, dsg, dx, T, dl2, dp, di, dw, ds, n))
    assert e.name == "NUMERIC_DOMAIN"
    assert unchanged(ctx, dl2, T * E)
    for b in (dr, dsg, dx, ds, dl, dp, di, dw, dbad, dl2):
        b.close()
    cfg.close()


# ---------------- one routed expert on F32 member matrices ----------------

@pytest.mark.parametrize("H,I", [(2048, 512), (2560, 640), (7, 3)])
def test_routed_expert_bit_exact(ctx, H, I):
    say(f"routed expert H={H} I={I}")
    rng = np.random.default_rng(H * 7 + I)
    g = (rng.standard_normal((I, H)) * 0.03).astype(np.float32)
    u = (rng.standard_normal((I, H)) * 0.03).astype(np.float32)
    d = (rng.standard_normal((H, I)) * 0.03).astype(np.float32)
    x = rng.standard_normal(H).astype(np.float32)
    cfg = kq_hip.MoeConfig(H, 16, 4, I, I)
    n = cfg.one_expert_scratch_bytes()
    assert n >= (3 * I + H) * 4
    dg, du, dd, dx, dout, ds = (ctx.upload(g), ctx.upload(u), ctx.upload(d), ctx.upload(x),
                                ctx.alloc(H * 4), ctx.alloc(n))
    ctx.moe_routed_expert_f32(cfg, dg, du, dd, 9, dx, dout, ds, n)
    got = ctx.download(dout, np.float32, H)
    want = kq_oracle.moe_routed_expert(g, u, d, x)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    for b in (dg, du, dd, dx, dout, ds):
        b.close()
    cfg.close()


def test_routed_expert_statuses(ctx):
    H, I = 256, 64
    rng = np.random.default_rng(5)
    g = (rng.standard_normal((I, H)) * 0.03).astype(np.float32)
    d = (rng.standard_normal((H, I)) * 0.03).astype(np.float32)
    x = rng.standard_normal(H).astype(np.float32)
    cfg = kq_hip.MoeConfig(H, 16, 4, I, I)
    n = cfg.one_expert_scratch_bytes()
    dg, dd, dx, ds = ctx.upload(g), ctx.upload(d), ctx.upload(x), ctx.alloc(n)
    dout = filled(ctx, H)
    call = lambda **kw: ctx.moe_routed_expert_f32(  # noqa: E731
        cfg, dg, dg, dd, kw.get("eid", 3), kw.get("x", dx), kw.get("out", dout), ds,
        kw.get("n", n), capacity=kw.get("cap"), counts=kw.get("counts"))
    assert status_of(lambda: call(eid=16)).name == "INVALID_ARGUMENT"
    assert status_of(lambda: call(cap=H - 1)).name == "BUFFER_TOO_SMALL"
    assert status_of(lambda: call(n=n - 4)).name == "BUFFER_TOO_SMALL"
    assert status_of(lambda: call(counts=(I * H, I * H, I * H - 1))).name == "DIMENSION_MISMATCH"
    assert status_of(lambda: call(out=dx)).name == "ALIASING_VIOLATION"
    assert status_of(lambda: call(out=ds)).name == "ALIASING_VIOLATION"
    bad = x.copy()
    bad[11] = np.inf
    dbad = ctx.upload(bad)
    assert status_of(lambda: call(x=dbad)).name == "NUMERIC_DOMAIN"
    assert unchanged(ctx, dout, H)  # written only on success
    call()
    want = kq_oracle.moe_routed_expert(g, g, d, x)
    assert np.array_equal(ctx.download(dout, np.float32, H).view(np.uint32), want.view(np.uint32))
    for b in (dg, dd, dx, ds, dout, dbad):
        b.close()
    cfg.close()


# ---------------- commit on success ----------------

def test_failed_matvec_and_lm_head_leave_outputs(ctx):
    rows, cols = 4096, 2048
    w = S.q4k_blocks(S.stream_key(S.W_MATVEC_Q4K, 301), rows * cols // 256).reshape(-1)
    x = S.normal_f32(S.stream_key(S.W_MATVEC_Q4K, 302), 2 * cols).copy()
    x[cols + 5] = np.nan
    dw, dx = ctx.upload(w), ctx.upload(x)
    dy, dl, di = filled(ctx, 2 * rows), filled(ctx, 2 * rows), filled(ctx, 2, np.uint32, 99)
    e = status_of(lambda: ctx.matvec(kq_hip.TYPE_Q4_K, dw, rows, cols, dx, 2, dy))
    assert e.name == "NUMERIC_DOMAIN"
    assert unchanged(ctx, dy, 2 * rows)
    e = status_of(lambda: ctx.lm_head(kq_hip.TYPE_Q4_K, dw, rows, cols, dx, 2, dl, di))
    assert e.name == "NUMERIC_DOMAIN"
    assert unchanged(ctx, dl, 2 * rows) and unchanged(ctx, di, 2, np.uint32, 99)
    # a malformed block scale: the dequantized output keeps its contents too
    q8 = S.q8_0_blocks(S.stream_key(S.W_DEQUANT, 303), 64)
    q8[40, 0:2] = [0x00, 0x7E]  # NaN scale
    dq, do = ctx.upload(q8.reshape(-1)), filled(ctx, 64 * 32)
    e = status_of(lambda: ctx.dequantize(kq_hip.TYPE_Q8_0, dq, q8.size, do, 64 * 32))
    assert e.name == "MALFORMED_QUANTIZED_DATA"
    assert unchanged(ctx, do, 64 * 32)
    # switched off, the call still fails; the outputs are then unspecified
    ctx.set_commit_on_success(False)
    try:
        e = status_of(lambda: ctx.matvec(kq_hip.TYPE_Q4_K, dw, rows, cols, dx, 2, dy))
        assert e.name == "NUMERIC_DOMAIN"
    finally:
        ctx.set_commit_on_success(True)
    # and a good call after the failures writes its result
    ctx.matvec(kq_hip.TYPE_Q4_K, dw, rows, cols, dx, 1, dy)
    got = ctx.download(dy, np.float32, rows)
    assert np.isfinite(got).all() and not np.any(got == SENTINEL)
    for b in (dw, dx, dy, dl, di, dq, do):
        b.close()


@pytest.mark.parametrize("T", [1, 3])
def test_failed_moe_execute_leaves_outputs(ctx, T):
    H, E, K, I = 512, 32, 4, 256
    say(f"moe commit T={T}")
    w = S.moe_weights(S.W_MOE + 411, H, E, I, I)
    bufs = {k: ctx.upload(v) for k, v in w.items()}
    cfg = kq_hip.MoeConfig(H, E, K, I, I)
    x = S.normal_f32(S.stream_key(S.W_MOE + 411, S.R_HIDDEN), T * H).copy()
    x[(T - 1) * H + 9] = np.inf
    n = cfg.scratch_bytes(T)
    ds, dx = ctx.alloc(n), ctx.upload(x)
    dout, dids = filled(ctx, T * H), filled(ctx, T * K, np.uint32, 5)
    e = status_of(lambda: ctx.moe_execute(cfg, kq_hip.moe_weights(bufs), dx, T, dout, dids, ds, n))
    assert e.name == "NUMERIC_DOMAIN"
    assert unchanged(ctx, dout, T * H) and unchanged(ctx, dids, T * K, np.uint32, 5)
    for b in list(bufs.values()) + [ds, dx, dout, dids]:
        b.close()
    cfg.close()


def test_failed_in_place_write_keeps_branches(ctx):
    B, H, T = 4, 256, 2
    x = S.normal_f32(S.stream_key(S.W_MOE + 412, 0), T * B * H)
    o = S.normal_f32(S.stream_key(S.W_MOE + 412, 1), T * H).copy()
    o[H + 3] = np.nan
    g = S.normal_f32(S.stream_key(S.W_MOE + 412, 2), T * B)
    dims = kq_hip.gr_dims(B, H, 1, 1e-6)
    dx, do, dg = ctx.upload(x), ctx.upload(o), ctx.upload(g)
    e = status_of(lambda: ctx.gr_write(dims, dx, do, dg, T, dx))
    assert e.name == "NUMERIC_DOMAIN"
    assert np.array_equal(ctx.download(dx, np.float32, x.size).view(np.uint32), x.view(np.uint32))
    for b in (dx, do, dg):
        b.close()
