"""Device parity for the gated residual (hyper-connection read / write,
src/kq_layer_qwen38.c:40-208) and the MoE block around it
(src/kq_layer.c:779-813), through the C ABI, against the oracle and the
reference's layer fixtures.

Bars: the read's outputs (mixed state, write gates) per element within 1e-4
absolute or 1e-3 relative of the oracle, or of the binary64 value where the
oracle's own fp32 sums are off by more (conftest.assert_close,
tests/exact.py); the write bit-exact given the same inputs; the MoE block's
expert ids exact against the oracle routed from the device's own mixed state
(routing is bit-exact given its input), its output within the same bar."""
import numpy as np
import pytest

from conftest import assert_close, load_golden, oracle_threads

import exact

import kq_hip
import kq_oracle
import kq_synth as S

pytestmark = pytest.mark.gpu

LAYER = load_golden("layer_tier_a.json")
DIMS = LAYER["reduced"]
EPS = 1.0e-6  # src/kq_layer.c:146
F32, Q8_0 = kq_oracle.F32, kq_oracle.Q8_0


@pytest.fixture(scope="module")
def ctx():
    c = kq_hip.Context(0)
    yield c
    c.close()


def say(*a):
    print(*a, flush=True)


def arr(rec):
    return np.frombuffer(bytes.fromhex(rec["le_hex"]), np.float32).reshape(rec["shape"])


class Gr:
    """Gated residual weights on the device plus their host copies."""

    def __init__(self, ctx, B, H, R, norm, down, up, inject):
        self.B, self.H, self.R = B, H, R
        self.host = {"norm": norm, "down": down, "up": up, "inject": inject}
        self.bufs = {"norm": ctx.upload(norm), "down": ctx.upload(down[1]),
                     "up": ctx.upload(up[1]), "inject": ctx.upload(inject)}
        self.dims = kq_hip.gr_dims(B, H, R, EPS)
        self.w = kq_hip.gr_weights(self.bufs, down[0], up[0])

    def read(self, ctx, x):
        T = x.shape[0]
        n = kq_hip.gr_scratch_bytes(self.dims, T)
        bufs = [ctx.upload(x), ctx.alloc(T * self.H * 4), ctx.alloc(T * self.B * 4), ctx.alloc(n)]
        dx, dm, dg, ds = bufs
        ctx.gr_read(self.dims, self.w, dx, T, dm, dg, ds, n)
        out = (ctx.download(dm, np.float32, T * self.H).reshape(T, self.H),
               ctx.download(dg, np.float32, T * self.B).reshape(T, self.B))
        for b in bufs:
            b.close()
        return out

    def oracle(self, xt):
        h = self.host
        return kq_oracle.gr_read(xt, self.H, self.R, EPS, h["norm"], h["down"], h["up"],
                                 h["inject"])

    def exact(self, xt):
        h = self.host
        return exact.gr_read(xt, self.H, self.R, EPS, h["norm"], h["down"], h["up"],
                             h["inject"])

    def close(self):
        for b in self.bufs.values():
            b.close()


def device_write(ctx, B, H, x, o, g, in_place=False):
    T = x.shape[0]
    dims = kq_hip.gr_dims(B, H, 1, EPS)
    dx, do, dg = ctx.upload(x), ctx.upload(o), ctx.upload(g)
    dout = dx if in_place else ctx.alloc(x.nbytes)
    ctx.gr_write(dims, dx, do, dg, T, dout)
    y = ctx.download(dout, np.float32, x.size).reshape(x.shape)
    for b in {id(v): v for v in (dx, do, dg, dout)}.values():
        b.close()
    return y


def fixture_gr(ctx, w, prefix):
    return Gr(ctx, DIMS["branches"], DIMS["hidden"], DIMS["rank"],
              arr(w[prefix + ".hc_norm.weight"]),
              (F32, arr(w[prefix + ".input_mix_weight_down.weight"])),
              (F32, arr(w[prefix + ".input_mix_weight_up.weight"])),
              arr(w[prefix + ".block_inject_weight.weight"]))


CASES = [(corpus, c) for corpus in ("calibration", "holdout") for c in LAYER[corpus]]


@pytest.mark.parametrize("corpus,case", CASES, ids=[f"{k}-{c['id']}" for k, c in CASES])
def test_gated_residual_fixture_chain(ctx, corpus, case):
    # The reference's Tier A layer fixtures (4 branches x hidden 8, rank 4,
    # F32 projections): attention read, write of the mixer output, MoE read
    # and the final write, each on the device, against the fixture's
    # checkpoints and the oracle.
    H = DIMS["hidden"]
    w = case["weights"]
    x = arr(case["input"])[0]
    cp = {k: arr(v)[0] for k, v in case["checkpoints"].items()}
    if "ple_output" in cp:
        x = (x + cp["ple_output"]).astype(np.float32)  # src/kq_layer.c:721
    attn, mlp = fixture_gr(ctx, w, "attn_hyper_connection"), fixture_gr(ctx, w, "mlp_hyper_connection")
    B = attn.B
    assert x.shape[1] == B * H
    mixed, wg = attn.read(ctx, x)
    assert_close(mixed, cp["attn_gr"])
    for t in range(x.shape[0]):
        ref = attn.oracle(x[t])
        assert_close(mixed[t], ref["mixed"])
        assert_close(wg[t], ref["write_gate"])
    after = device_write(ctx, B, H, x, cp["mixer_output"], wg)
    want = np.stack([kq_oracle.gr_write(x[t], H, cp["mixer_output"][t], wg[t])
                     for t in range(x.shape[0])])
    assert np.array_equal(after.view(np.uint32), want.view(np.uint32))
    mixed, wg = mlp.read(ctx, after)
    assert_close(mixed, cp["moe_gr"])
    y = device_write(ctx, B, H, after, cp["moe_output"], wg, in_place=True)
    assert_close(y, arr(case["output"])[0])
    attn.close()
    mlp.close()


def model_gr(ctx, seed, B=4, H=2560, R=320):
    # The reference model's MoE hyper-connection: hc_ffn_down Q8_0 [320 x
    # 10240], hc_ffn_up Q8_0 [10240 x 320], norm and inject F32.
    W = B * H
    norm = S.normal_f32(S.stream_key(S.W_MOE + 90, 1, seed), W, 0.1)
    down = S.quant_matrix("Q8_0", S.stream_key(S.W_MOE + 90, 2, seed), R, W)
    up = S.quant_matrix("Q8_0", S.stream_key(S.W_MOE + 90, 3, seed), W, R)
    inject = S.normal_f32(S.stream_key(S.W_MOE + 90, 4, seed), B * W, 0.01)
    return Gr(ctx, B, H, R, norm, (Q8_0, down), (Q8_0, up), inject)


@pytest.fixture(scope="module")
def gr_model(ctx):
    say("uploading 4 x 2560 rank-320 gated residual")
    g = model_gr(ctx, 0)
    yield g
    g.close()


@pytest.mark.parametrize("tokens", [1, 3, 5, 37, 130])
def test_gated_residual_read_model_dims(ctx, gr_model, tokens):
    # up to 4 tokens the rank projections run on the row engine; from 5 on
    # MFMA in 16-token chunks (37 and 130: partial last chunks)
    g = gr_model
    x = S.normal_f32(S.stream_key(S.W_MOE + 91, tokens), tokens * g.B * g.H).reshape(tokens, -1)
    mixed, wg = g.read(ctx, x)
    for t in range(tokens):
        ref, ex = g.oracle(x[t]), g.exact(x[t])
        assert_close(mixed[t], ref["mixed"], exact=lambda i: ex["mixed"][i])
        assert_close(wg[t], ref["write_gate"], exact=lambda i: ex["write_gate"][i])


@pytest.mark.parametrize("in_place", [False, True])
def test_gated_residual_write_bit_exact(ctx, in_place):
    B, H, T = 4, 2560, 5
    rng = np.random.default_rng(11)
    x = rng.standard_normal((T, B * H)).astype(np.float32)
    o = rng.standard_normal((T, H)).astype(np.float32)
    g = (2.0 * rng.random((T, B))).astype(np.float32)
    y = device_write(ctx, B, H, x, o, g, in_place)
    want = np.stack([kq_oracle.gr_write(x[t], H, o[t], g[t]) for t in range(T)])
    assert np.array_equal(y.view(np.uint32), want.view(np.uint32))


MOE_ROLES = ("router", "gate", "up", "down", "shared_gate", "shared_up", "shared_down",
             "shared_gate_weight")


@pytest.mark.parametrize("E,K,T", [(64, 8, 1), (64, 8, 3), (512, 10, 1), (64, 8, 40)])
def test_moe_block_model_layer(ctx, gr_model, E, K, T):
    # The reference model's MoE block: hyper-connection read, MoE (hidden
    # 2560, intermediate 640, Q4_K gate/up, Q5_1 routed down, Q8_0 shared
    # expert), hyper-connection write, in one call.
    g, H, I = gr_model, 2560, 640
    seed = S.W_MOE + 5000 + E + T
    say(f"MoE block E={E} K={K} T={T}")
    w = S.moe_weights(seed, H, E, I, I, gate_fmt="Q4_K", down_fmt="Q5_1",
                      shared_gate_fmt="Q8_0", shared_down_fmt="Q8_0")
    t = kq_hip.TYPE_IDS
    bufs = {k: ctx.upload(v) for k, v in w.items()}
    mw = kq_hip.moe_weights(bufs, t["Q4_K"], t["Q5_1"], t["Q8_0"], t["Q8_0"])
    cfg = kq_hip.MoeConfig(H, E, K, I, I)
    x = S.normal_f32(S.stream_key(seed, S.R_HIDDEN), T * g.B * H).reshape(T, -1)
    n = kq_hip.moe_block_scratch_bytes(g.dims, cfg, T)
    dx, dout, dids, ds = ctx.upload(x), ctx.alloc(x.nbytes), ctx.alloc(T * K * 4), ctx.alloc(n)
    ctx.moe_block(g.dims, g.w, cfg, mw, dx, T, dout, dids, ds, n)
    y = ctx.download(dout, np.float32, x.size).reshape(x.shape)
    ids = ctx.download(dids, np.uint32, T * K).reshape(T, K)
    # the same read alone (same kernels, same result) gives the MoE's input
    mixed, wg = g.read(ctx, x)
    roles = {"router": F32, "gate": t["Q4_K"], "up": t["Q4_K"], "down": t["Q5_1"],
             "shared_gate": t["Q8_0"], "shared_up": t["Q8_0"], "shared_down": t["Q8_0"],
             "shared_gate_weight": F32}
    dims = dict(hidden=H, experts=E, top_k=K, inter=I, shared_inter=I)
    moe_ref, tr = kq_oracle.moe_execute(dims, {k: (roles[k], w[k]) for k in MOE_ROLES}, mixed,
                                        trace=True, threads=oracle_threads())
    assert np.array_equal(ids, tr["selected_ids"])
    want = np.stack([kq_oracle.gr_write(x[i], H, moe_ref[i], wg[i]) for i in range(T)])
    moe_ex = exact.moe(dims, roles, w, mixed, ids)
    W = g.B * H

    def y_parts(idx):
        t, j = idx // W, idx % W
        return t, j, t * H + j % H, wg[t, j // H].astype(np.float64)

    def y_value(idx):
        # branches + (binary64 MoE of the device's mixed state) * write gate
        t, j, m, g = y_parts(idx)
        return x[t, j].astype(np.float64) + moe_ex(m) * g

    def y_scale(idx):
        t, j, m, g = y_parts(idx)
        return np.abs(x[t, j].astype(np.float64)) + moe_ex.scale(m) * np.abs(g)
    assert_close(y, want, exact=exact.Exact(y_value, y_scale))
    # and the whole chain from the oracle's own read
    for i in range(T):
        r, ex = g.oracle(x[i]), g.exact(x[i])
        assert_close(mixed[i], r["mixed"], exact=lambda j: ex["mixed"][j])
    for b in list(bufs.values()) + [dx, dout, dids, ds]:
        b.close()
    cfg.close()


def test_gated_residual_fails_closed(ctx, gr_model):
    g = gr_model
    T = 2
    x = S.normal_f32(S.stream_key(S.W_MOE + 92, 0), T * g.B * g.H).reshape(T, -1).copy()
    x[1, 7] = np.nan
    with pytest.raises(kq_hip.KqError) as e:
        g.read(ctx, x)
    assert e.value.name == "NUMERIC_DOMAIN"
    n = kq_hip.gr_scratch_bytes(g.dims, T)
    dx, dm, dg, ds = ctx.upload(x), ctx.alloc(T * g.H * 4), ctx.alloc(T * g.B * 4), ctx.alloc(n)
    with pytest.raises(kq_hip.KqError) as e:
        ctx.gr_read(g.dims, g.w, dx, T, dm, dg, ds, n - 256)
    assert e.value.name == "BUFFER_TOO_SMALL"
    with pytest.raises(kq_hip.KqError) as e:
        ctx.gr_read(g.dims, g.w, dx, T, dx, dg, ds, n)
    assert e.value.name == "ALIASING_VIOLATION"
    with pytest.raises(kq_hip.KqError) as e:  # the grid's token axis; rejected before launch
        ctx.gr_read(g.dims, g.w, dx, 65536, dm, dg, ds, n)
    assert e.value.name == "LIMIT_EXCEEDED"
    # tokens x rank above 2^30 (the rank step's element count) is refused
    # before any launch
    big = kq_hip.gr_dims(1, 4, 65536, EPS)
    with pytest.raises(kq_hip.KqError) as e:
        ctx.gr_read(big, g.w, dx, 16385, dm, dg, ds, n)
    assert e.value.name == "LIMIT_EXCEEDED"
    bad = kq_hip.gr_dims(0, g.H, g.R, EPS)
    with pytest.raises(kq_hip.KqError) as e:
        ctx.gr_read(bad, g.w, dx, T, dm, dg, ds, n)
    assert e.value.name == "INVALID_ARGUMENT"
    with pytest.raises(kq_hip.KqError) as e:
        ctx.gr_write(g.dims, dx, dm, dg, T, dm)
    assert e.value.name == "ALIASING_VIOLATION"
    for b in (dx, dm, dg, ds):
        b.close()
    # and the read still runs correctly afterwards
    test_gated_residual_read_model_dims(ctx, gr_model, 1)
