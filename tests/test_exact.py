"""The binary64 restatements in tests/exact.py against the oracle.

exact.py is the second stage of the tolerance check: an element where the
device and the oracle differ by more than 1e-4 absolute and 1e-3 relative
passes only if the device is within that bar of exact.py's value. So
exact.py must compute the same equations as the oracle: a transposed
operand, a missing 1/B or a wrong gate would put it far from the oracle's
fp32 result, which these tests bound by a few binary32 roundings per term."""
import numpy as np
import pytest

import exact
import kq_oracle
import kq_synth as S

FMTS = {"Q4_K": kq_oracle.Q4_K, "Q8_0": kq_oracle.Q8_0, "Q6_K": kq_oracle.Q6_K,
        "Q5_K": kq_oracle.Q5_K, "Q5_1": kq_oracle.Q5_1, "IQ4_NL": kq_oracle.IQ4_NL}


def close_to_oracle(ex, ref, scale, tol=2e-5):
    """|exact - oracle| within tol of the size of the terms (`scale`)."""
    err = np.abs(np.asarray(ex, np.float64) - np.asarray(ref, np.float64))
    assert (err <= tol * scale).all(), float((err / scale).max())


@pytest.mark.parametrize("fmt", sorted(FMTS))
def test_matvec_matches_oracle(fmt):
    rows, cols, batch = 48, 512, 2
    key = S.stream_key(S.W_MATVEC_Q8_0, 200, FMTS[fmt])
    w = S.quant_matrix(fmt, key, rows, cols)
    x = S.normal_f32(key ^ 0x55, batch * cols).reshape(batch, cols)
    ref = kq_oracle.matvec(FMTS[fmt], w, rows, cols, x)
    f = exact.matvec(FMTS[fmt], w, rows, cols, x)
    got = f(np.arange(batch * rows)).reshape(batch, rows)
    dense = kq_oracle.dequantize(FMTS[fmt], w).reshape(rows, cols).astype(np.float64)
    scale = np.abs(dense) @ np.abs(x.astype(np.float64)).T  # [rows, batch]
    close_to_oracle(got, ref, scale.T)
    # rows and batch columns are not swapped: a permuted index gives
    # another value
    assert not np.allclose(f(np.array([1])), ref[0, 2])


def test_moe_matches_oracle():
    H, E, K, I, T = 512, 16, 4, 256, 2
    w = S.moe_weights(S.W_MOE + 401, H, E, I, I)
    roles = {"router": kq_oracle.F32, "gate": kq_oracle.Q4_K, "up": kq_oracle.Q4_K,
             "down": kq_oracle.Q6_K, "shared_gate": kq_oracle.Q4_K,
             "shared_up": kq_oracle.Q4_K, "shared_down": kq_oracle.Q6_K,
             "shared_gate_weight": kq_oracle.F32}
    dims = dict(hidden=H, experts=E, top_k=K, inter=I, shared_inter=I)
    x = S.normal_f32(S.stream_key(S.W_MOE + 401, S.R_HIDDEN), T * H).reshape(T, H)
    ref, tr = kq_oracle.moe_execute(dims, {k: (t, w[k]) for k, t in roles.items()}, x,
                                    trace=True)
    f = exact.moe(dims, roles, w, x, tr["selected_ids"])
    got = f(np.arange(T * H)).reshape(T, H)
    # the output's terms are each expert's weighted rows; their RMS bounds
    # the size of any one element's sum
    scale = np.sqrt(np.mean(ref.astype(np.float64) ** 2))
    close_to_oracle(got, ref, scale, tol=1e-5)
    # the shared expert and the routed weights both matter: dropping the
    # gate of the shared expert moves the result far beyond that
    tr2 = dict(w)
    tr2["shared_gate_weight"] = np.full(H, 0.0, np.float32)
    g2 = exact.moe(dims, roles, tr2, x, tr["selected_ids"])(np.arange(H))
    assert np.abs(g2 - got[0]).max() > 1e-3 * scale


@pytest.mark.parametrize("proj", ["F32", "Q8_0"])
def test_gr_read_matches_oracle(proj):
    B, H, R = 4, 256, 32
    W = B * H
    key = lambda i: S.stream_key(S.W_MOE + 402, 90, i)
    norm = S.normal_f32(key(1), W, 0.1)
    if proj == "F32":
        down = (kq_oracle.F32, S.normal_f32(key(2), R * W, 0.05))
        up = (kq_oracle.F32, S.normal_f32(key(3), W * R, 0.05))
    else:
        down = (kq_oracle.Q8_0, S.quant_matrix("Q8_0", key(2), R, W))
        up = (kq_oracle.Q8_0, S.quant_matrix("Q8_0", key(3), W, R))
    inject = S.normal_f32(key(4), B * W, 0.01)
    x = S.normal_f32(key(5), W)
    ref = kq_oracle.gr_read(x, H, R, 1e-6, norm, down, up, inject)
    got = exact.gr_read(x, H, R, 1e-6, norm, down, up, inject)
    close_to_oracle(got["mixed"], ref["mixed"], 1.0, tol=1e-5)
    close_to_oracle(got["write_gate"], ref["write_gate"], 1.0, tol=1e-5)


def test_assert_close_rule():
    from conftest import assert_close
    ref = np.array([0.0, 1.0, 1000.0, -0.05])
    assert_close(ref + np.array([9e-5, 9e-5, 0.9, -9e-5]), ref)          # abs or rel
    with pytest.raises(AssertionError):
        assert_close(ref + np.array([2e-4, 0, 0, 0]), ref)               # near zero: abs only
    with pytest.raises(AssertionError):
        assert_close(ref + np.array([0, 0, 1.1, 0]), ref)                # beyond 1e-3 rel
    # an element beyond the bar passes only when it is within the bar of
    # the exact value there
    got = ref + np.array([2e-4, 0, 0, 0])
    rec = assert_close(got, ref, exact=lambda i: got[i] - 5e-5)
    assert rec["beyond_bar_vs_ref"] == 1
    with pytest.raises(AssertionError):
        assert_close(got, ref, exact=lambda i: ref[i])


def _moe_f32_blas(dims, roles, w, x, ids):
    """The MoE equations in binary32 with numpy's (BLAS) summation order: a
    second valid binary32 evaluation, to be accepted by assert_close."""
    H, E, I = dims["hidden"], dims["experts"], dims["inter"]
    f32 = np.float32
    rt = np.asarray(w["router"], f32).reshape(E, H)

    def expert(role_w, e, n_exp):
        g = kq_oracle.dequantize(roles["gate"] if n_exp else roles["shared_gate"],
                                 np.asarray(role_w[0]).reshape(n_exp or 1, -1)[e]).reshape(I, H)
        u = kq_oracle.dequantize(roles["up"] if n_exp else roles["shared_up"],
                                 np.asarray(role_w[1]).reshape(n_exp or 1, -1)[e]).reshape(I, H)
        d = kq_oracle.dequantize(roles["down"] if n_exp else roles["shared_down"],
                                 np.asarray(role_w[2]).reshape(n_exp or 1, -1)[e]).reshape(H, I)
        return g, u, d

    out = np.zeros((x.shape[0], H), f32)
    for t in range(x.shape[0]):
        xt = x[t].astype(f32)
        lg = rt @ xt
        p = np.exp(lg - lg.max()).astype(f32)
        p /= p.sum()
        sel = [int(e) for e in ids[t]]
        wk = p[sel] / p[sel].sum()
        for k, e in enumerate(sel):
            g, u, d = expert((w["gate"], w["up"], w["down"]), e, E)
            gv, uv = g @ xt, u @ xt
            a = (gv / (f32(1) + np.exp(-gv))) * uv
            out[t] += wk[k] * (d @ a)
        g, u, d = expert((w["shared_gate"], w["shared_up"], w["shared_down"]), 0, 0)
        gv, uv = g @ xt, u @ xt
        a = (gv / (f32(1) + np.exp(-gv))) * uv
        gam = f32(1) / (f32(1) + np.exp(-(np.asarray(w["shared_gate_weight"], f32) @ xt)))
        out[t] += gam * (d @ a)
    return out


def test_moe_stages_accept_binary32_and_catch_planted_mistakes():
    # Another binary32 evaluation of the same layer (numpy's summation
    # order) passes assert_close against the oracle; the oracle's output with
    # one expert's weighted output removed, or the shared expert ungated,
    # fails it: near-cancelling elements do not hide a missing term.
    H, E, K, I, T = 2048, 40, 10, 512, 3
    w = S.moe_weights(S.W_MOE + 403, H, E, I, I)
    roles = {"router": kq_oracle.F32, "gate": kq_oracle.Q4_K, "up": kq_oracle.Q4_K,
             "down": kq_oracle.Q6_K, "shared_gate": kq_oracle.Q4_K,
             "shared_up": kq_oracle.Q4_K, "shared_down": kq_oracle.Q6_K,
             "shared_gate_weight": kq_oracle.F32}
    dims = dict(hidden=H, experts=E, top_k=K, inter=I, shared_inter=I)
    x = S.normal_f32(S.stream_key(S.W_MOE + 403, S.R_HIDDEN), T * H).reshape(T, H)
    ref, tr = kq_oracle.moe_execute(dims, {k: (t, w[k]) for k, t in roles.items()}, x,
                                    trace=True)
    ids = tr["selected_ids"]
    ex = exact.moe(dims, roles, w, x, ids)
    from conftest import assert_close
    with np.errstate(over="ignore"):
        other = _moe_f32_blas(dims, roles, w, x, ids)
    assert_close(other, ref, exact=ex)
    for k in (0, K - 1):
        with pytest.raises(AssertionError):
            assert_close(ref - tr["expert_weighted"][:, k, :], ref, exact=ex)
    with pytest.raises(AssertionError):
        assert_close(ref - tr["gated_shared"] + tr["shared_output"], ref, exact=ex)
