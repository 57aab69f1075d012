"""Binary64 restatements of the fp32-accumulated outputs, for the tolerance
check's second stage.

The reference sums in binary32 left to right (src/kq_numeric.c:474-496,
src/kq_moe_qwen38.c:722-826). At the benchmark shapes that sum itself is
off the mathematically exact value by more than 1e-4 at a few elements (a
2048-term row whose partial sums reach ~100 rounds each step by ~1e-6), so a
device result that is closer to the exact value can still differ from the
CPU's by more than the bar there. These functions give the exact value (to
binary64 rounding) of the same equations on the same decoded weights, so
that such elements are judged against it instead.

Only the equations are restated here; the weights are decoded by the oracle
(bit-exact with the reference's decode)."""
from __future__ import annotations

import numpy as np

import kq_oracle


def _rows(type_id: int, packed: np.ndarray, rows: int, cols: int, which) -> np.ndarray:
    """Decoded rows `which` of a packed [rows, cols] matrix, binary64."""
    be, bb = kq_oracle.geometry(type_id)
    rb = cols // be * bb
    m = np.ascontiguousarray(packed).view(np.uint8).reshape(rows, rb)
    sel = np.ascontiguousarray(m[np.asarray(which)])
    return kq_oracle.dequantize(type_id, sel.reshape(-1)).reshape(len(which), cols).astype(
        np.float64)


class Exact:
    """Binary64 values of selected output elements and, optionally, the
    magnitude S of the terms each is formed from (the sum of the absolute
    values of every product, first-order through intermediate results). A
    binary32 evaluation in any order errs by a small multiple of u * S at
    an element (u = 2^-24), however much its terms cancel; an error in the
    equations (a dropped or wrong term, a transposed operand) moves it by
    about one term, which is S / sqrt(n) or more."""

    def __init__(self, values, scale=None):
        self.values = values
        self.scale = scale

    def __call__(self, idx):
        return self.values(idx)


def matvec(type_id: int, packed: np.ndarray, rows: int, cols: int, x: np.ndarray) -> Exact:
    """y = W x in binary64 for output [batch, rows]; S = |W| |x|."""
    x64 = np.atleast_2d(np.asarray(x, np.float64)).reshape(-1, cols)

    def rows_of(idx):
        idx = np.asarray(idx)
        b, r = idx // rows, idx % rows
        return _rows(type_id, packed, rows, cols, r), x64[b]

    def f(idx):
        w, xb = rows_of(idx)
        return np.einsum("ij,ij->i", w, xb)

    def sc(idx):
        w, xb = rows_of(idx)
        return np.einsum("ij,ij->i", np.abs(w), np.abs(xb))
    return Exact(f, sc)


def _sig(v):
    with np.errstate(over="ignore"):
        return 1.0 / (1.0 + np.exp(-v))


def _expert(roles, w, e, x64, H, I, E):
    """One expert's output o = Wd (silu(Wg x) * (Wu x)) in binary64, and its
    term magnitude |Wd| A, where A bounds the activation and, to first
    order, its sensitivity to the rounding of the gate and up sums:
    A = |a| + |u silu'(g)| |Wg| |x| + |silu(g)| |Wu| |x|."""
    ge = np.asarray(w["gate"]).reshape(E, -1)[e]
    ue = np.asarray(w["up"]).reshape(E, -1)[e]
    de = np.asarray(w["down"]).reshape(E, -1)[e]
    Wg = _rows(roles["gate"], ge, I, H, range(I))
    Wu = _rows(roles["up"], ue, I, H, range(I))
    Wd = _rows(roles["down"], de, H, I, range(H))
    ax = np.abs(x64)
    g, u = Wg @ x64, Wu @ x64
    sg = _sig(g)
    silu = g * sg
    a = silu * u
    dsilu = sg * (1.0 + g * (1.0 - sg))
    A = np.abs(a) + np.abs(u * dsilu) * (np.abs(Wg) @ ax) + np.abs(silu) * (np.abs(Wu) @ ax)
    return Wd @ a, np.abs(Wd) @ A


def moe(dims: dict, roles: dict, w: dict, x: np.ndarray, ids: np.ndarray) -> Exact:
    """MoE output of each token in binary64 with the given (exact) expert
    ids: softmax weights renormalised over the selection, routed experts
    summed, plus the sigmoid-gated shared expert
    (src/kq_moe_qwen38.c:604-867). S sums each expert's term magnitude
    times its weight, plus the shared gate's sensitivity
    gamma (1 - gamma) |g_s| |x| |s|. Over [tokens, hidden]; a token is
    formed once, on first use."""
    H, E, I, Sh = dims["hidden"], dims["experts"], dims["inter"], dims["shared_inter"]
    x = np.atleast_2d(np.asarray(x, np.float32))
    ids = np.atleast_2d(np.asarray(ids))
    rt = np.asarray(w["router"], np.float32).reshape(E, H).astype(np.float64)
    cache = {}

    def token(t):
        if t not in cache:
            x64 = x[t].astype(np.float64)
            logits = rt @ x64
            p = np.exp(logits - logits.max())
            p /= p.sum()
            sel = [int(e) for e in ids[t]]
            wk = p[sel] / p[sel].sum()
            out, mag = np.zeros(H), np.zeros(H)
            for k, e in enumerate(sel):
                o, so = _expert(roles, w, e, x64, H, I, E)
                out += wk[k] * o
                mag += wk[k] * so
            sroles = {"gate": roles["shared_gate"], "up": roles["shared_up"],
                      "down": roles["shared_down"]}
            sw = {"gate": w["shared_gate"], "up": w["shared_up"], "down": w["shared_down"]}
            s, ss = _expert(sroles, sw, 0, x64, H, Sh, 1)
            gw = np.asarray(w["shared_gate_weight"], np.float64)
            gam = _sig(float(gw @ x64))
            out += gam * s
            mag += gam * ss + gam * (1.0 - gam) * float(np.abs(gw) @ np.abs(x64)) * np.abs(s)
            cache[t] = (out, mag)
        return cache[t]

    def pick(idx, part):
        idx = np.asarray(idx)
        return np.array([token(int(i) // H)[part][int(i) % H] for i in idx])
    return Exact(lambda idx: pick(idx, 0), lambda idx: pick(idx, 1))


def gr_read(branches: np.ndarray, hidden: int, rank: int, eps: float, norm: np.ndarray,
            down: tuple, up: tuple, inject: np.ndarray) -> dict:
    """Gated-residual read of one token in binary64 (the equations of
    src/kq_layer_qwen38.c:40-172): per-branch RMS norm scaled by (1 + w),
    rank = silu(down . normalized / B), read gates sigmoid(up . rank), the
    gated branch mean, and write gates 2 sigmoid(inject[b] . normalized / B).
    down / up are (type, packed rows) as for the device. Returns mixed
    [hidden] and write_gate [B]."""
    x = np.asarray(branches, np.float64).reshape(-1)
    B = x.size // hidden
    W = B * hidden
    xb = x.reshape(B, hidden)
    inv = 1.0 / np.sqrt((xb * xb).mean(axis=1, keepdims=True) + float(np.float32(eps)))
    nrm = (xb * inv * (1.0 + np.asarray(norm, np.float64).reshape(B, hidden))).reshape(-1)
    r = _rows(down[0], down[1], rank, W, range(rank)) @ nrm / B
    r = r * _sig(r)
    gate = _sig(_rows(up[0], up[1], W, rank, range(W)) @ r)
    mixed = (gate * nrm).reshape(B, hidden).sum(axis=0) / B
    wg = 2.0 * _sig(np.asarray(inject, np.float64).reshape(B, W) @ nrm / B)
    return {"mixed": mixed, "write_gate": wg}
