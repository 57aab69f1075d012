"""The MoE operator on F32 expert weights on the device
(kq_hip_moe_execute_f32), with the reference's route and checkpoint
observers, through the C ABI.

Bars: every checkpoint and the output bit-identical to the oracle (the
device runs the reference's left-to-right binary32 sums, one thread per
output); on the reference's Tier A operator fixtures
(moe-calibration/holdout.json) the ids exact and every checkpoint within
its calibrated contract of moe-native-validation.json (abs OR rel OR ulp,
tools/validate-native-moe.py:186-189); observers called in the reference's
order (src/kq_moe_qwen38.c:697-863)."""
import numpy as np
import pytest

from conftest import hex_le_f32, load_golden, ulp_distance

import kq_hip
import kq_oracle
import kq_synth as S

pytestmark = pytest.mark.gpu

TIER_A = load_golden("moe_tier_a.json")
F32 = kq_oracle.F32
ROLES = ("router", "gate", "up", "down", "shared_gate", "shared_up", "shared_down",
         "shared_gate_weight")
DEV_ROLE = {"router": "router", "gate": "routed_gate", "up": "routed_up", "down": "routed_down",
            "shared_gate": "shared_gate", "shared_up": "shared_up",
            "shared_down": "shared_down", "shared_gate_weight": "shared_gate_weight"}
# per-token checkpoint order of the reference (src/kq_moe_qwen38.c:709-863)
HEAD = ["router_logits", "router_probabilities", "selected_weights"]
PER_EXPERT = ["routed_gate", "routed_up", "routed_activated", "routed_expert_output",
              "routed_weighted_output"]
TAIL = ["routed_weighted_sum", "shared_gate_projection", "shared_up_projection",
        "shared_activated", "shared_output", "shared_scale_logit", "shared_scale",
        "gated_shared_output", "operator_output"]
# checkpoint kind -> oracle trace field (None: the operator output)
TRACE = {"router_logits": "router_logits", "router_probabilities": "router_probs",
         "selected_weights": "selected_weights", "routed_weighted_sum": "routed_sum",
         "shared_gate_projection": "shared_gate_proj", "shared_up_projection": "shared_up_proj",
         "shared_activated": "shared_activated", "shared_output": "shared_output",
         "shared_scale_logit": "shared_scale_logit", "shared_scale": "shared_scale",
         "gated_shared_output": "gated_shared", "operator_output": None,
         "routed_gate": "expert_gate", "routed_up": "expert_up",
         "routed_activated": "expert_activated", "routed_expert_output": "expert_output",
         "routed_weighted_output": "expert_weighted"}


@pytest.fixture(scope="module")
def ctx():
    c = kq_hip.Context(0)
    yield c
    c.close()


def run_f32(ctx, dims, w, x, observe=True):
    """w: role -> float32 array. Returns (out, observed calls)."""
    H, E, K, I, Sh = (dims["hidden"], dims["experts"], dims["top_k"], dims["inter"],
                      dims["shared_inter"])
    T = x.shape[0]
    cfg = kq_hip.MoeConfig(H, E, K, I, Sh)
    bufs = {DEV_ROLE[r]: ctx.upload(np.ascontiguousarray(w[r], np.float32)) for r in ROLES}
    counts = {DEV_ROLE[r]: int(np.asarray(w[r]).size) for r in ROLES}
    n = cfg.f32_scratch_bytes(T)
    scratch, dx, dout = ctx.alloc(n), ctx.upload(x), ctx.alloc(T * H * 4)
    seen = ctx.moe_execute_f32(cfg, kq_hip.moe_weights_f32(bufs, counts), dx, T, dout,
                               scratch, n, observe=observe)
    out = ctx.download(dout, np.float32, T * H).reshape(T, H)
    for b in list(bufs.values()) + [scratch, dx, dout]:
        b.close()
    cfg.close()
    return out, seen


def check_order(seen, T, K):
    """The reference's observer sequence: per token the route, then its
    checkpoints, experts in ascending id."""
    i = 0
    for t in range(T):
        kind, rec = seen[i]
        assert kind == "route" and rec["token"] == t
        ids = rec["ids"]
        i += 1
        expect = HEAD + PER_EXPERT * K + TAIL
        got = [seen[i + j][1]["kind"] for j in range(len(expect))]
        assert got == expect, (t, got)
        experts = [seen[i + 3 + 5 * j][1]["expert"] for j in range(K)]
        assert experts == sorted(int(e) for e in ids)
        for j in range(len(expect)):
            rec = seen[i + j][1]
            assert rec["token"] == t and rec["rank"] == 1
            assert rec["dims"] == (rec["values"].size, 0)
            if rec["kind"].startswith("routed_") and rec["kind"] != "routed_weighted_sum":
                assert ids[rec["position"]] == rec["expert"]
            else:
                assert rec["expert"] == 0xFFFFFFFF and rec["position"] == 0xFFFFFFFF
        i += len(expect)
    assert i == len(seen)


def by_token(seen):
    """token -> {"route": rec, kind: values, (kind, position): values}"""
    out = {}
    for kind, rec in seen:
        d = out.setdefault(rec["token"], {})
        if kind == "route":
            d["route"] = rec
        elif rec["kind"].startswith("routed_") and rec["kind"] != "routed_weighted_sum":
            d[(rec["kind"], rec["position"])] = rec["values"]
        else:
            d[rec["kind"]] = rec["values"]
    return out


def assert_bit_exact_vs_oracle(seen, out, ref, tr, T, K):
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))
    tok = by_token(seen)
    for t in range(T):
        d = tok[t]
        assert np.array_equal(d["route"]["ids"], tr["selected_ids"][t])
        for kind, field in TRACE.items():
            if kind.startswith("routed_") and kind != "routed_weighted_sum":
                for k in range(K):
                    want = tr[field][t, k]
                    assert np.array_equal(d[(kind, k)].view(np.uint32),
                                          np.asarray(want, np.float32).view(np.uint32)), (t, kind, k)
            else:
                want = ref[t] if field is None else np.atleast_1d(tr[field][t])
                assert np.array_equal(d[kind].view(np.uint32),
                                      np.asarray(want, np.float32).view(np.uint32)), (t, kind)


def within(contract, got, want):
    got = np.asarray(got, np.float32).ravel()
    want = np.asarray(want, np.float32).ravel()
    assert got.shape == want.shape
    if contract["class"] == "EXACT_BITS":
        return np.array_equal(got.view(np.uint32), want.view(np.uint32))
    a = np.abs(got.astype(np.float64) - want.astype(np.float64))
    denom = np.abs(want.astype(np.float64))
    with np.errstate(divide="ignore", invalid="ignore"):
        rel = np.where(denom != 0, a / np.where(denom != 0, denom, 1.0),
                       np.where(a == 0, 0.0, np.inf))
    ok = (a <= contract["abs_limit"]) | (rel <= contract["rel_limit"]) | \
        (ulp_distance(got, want) <= contract["ulp_limit"])
    return bool(ok.all())


def tier_a():
    cfg = TIER_A["tier_a_config"]
    w = {k: hex_le_f32(v["le_hex"]).reshape(v["shape"]) for k, v in TIER_A["weights"].items()}
    E, I, H = cfg["expert_count"], cfg["routed_intermediate_size"], cfg["hidden_size"]
    gate_up = w["experts.gate_up_proj"]  # [E, 2I, H]: gate rows, then up rows
    weights = {"router": w["gate.weight"], "gate": gate_up[:, :I, :], "up": gate_up[:, I:, :],
               "down": w["experts.down_proj"], "shared_gate": w["shared_expert.gate_proj.weight"],
               "shared_up": w["shared_expert.up_proj.weight"],
               "shared_down": w["shared_expert.down_proj.weight"],
               "shared_gate_weight": w["shared_expert_gate.weight"]}
    dims = dict(hidden=H, experts=E, top_k=cfg["top_k"], inter=I,
                shared_inter=cfg["shared_intermediate_size"])
    return dims, {k: np.ascontiguousarray(v, np.float32) for k, v in weights.items()}


# fixture key -> checkpoint kind
AGG = {"router_logits": "router_logits", "router_probabilities": "router_probabilities",
       "selected_weights": "selected_weights", "routed_weighted_sum": "routed_weighted_sum",
       "shared_gate_projection": "shared_gate_projection",
       "shared_up_projection": "shared_up_projection", "shared_activated": "shared_activated",
       "shared_output": "shared_output", "shared_gate_logit": "shared_scale_logit",
       "shared_gate": "shared_scale", "gated_shared_output": "gated_shared_output",
       "final_output": "operator_output"}
EXPERT = {"gate": "routed_gate", "up": "routed_up", "activated": "routed_activated",
          "output": "routed_expert_output", "weighted_output": "routed_weighted_output"}


@pytest.mark.parametrize("case", TIER_A["calibration"] + TIER_A["holdout"], ids=lambda c: c["id"])
def test_tier_a_fixture_checkpoints(ctx, case):
    # The reference's own operator fixtures (hidden 6, 4 experts, top-2,
    # intermediate 4, 1..5 tokens): ids exact, every checkpoint within its
    # calibrated contract, and bit-identical to the oracle.
    dims, w = tier_a()
    H, K = dims["hidden"], dims["top_k"]
    x = hex_le_f32(case["input"]["le_hex"]).reshape(-1, H)
    T = x.shape[0]
    out, seen = run_f32(ctx, dims, w, x)
    check_order(seen, T, K)
    tok = by_token(seen)
    exp = case["expected"]
    assert [list(map(int, tok[t]["route"]["ids"])) for t in range(T)] == \
        exp["selected_expert_ids"]
    for key, kind in AGG.items():
        want = hex_le_f32(exp[key]["le_hex"]).reshape(T, -1)
        got = np.stack([np.atleast_1d(tok[t][kind]) for t in range(T)])
        assert within(TIER_A["contracts"][key], got, want), key
    for sel in exp["selected_experts"]:
        t, pos = sel["token"], sel["top_k_position"]
        assert int(tok[t]["route"]["ids"][pos]) == sel["expert_id"]
        for key, kind in EXPERT.items():
            want = hex_le_f32(sel[key]["le_hex"])
            assert within(TIER_A["contracts"]["routed_" + key], tok[t][(kind, pos)], want), key
    ref, tr = kq_oracle.moe_execute(dims, {r: (F32, w[r]) for r in ROLES}, x, trace=True)
    assert_bit_exact_vs_oracle(seen, out, ref, tr, T, K)


@pytest.mark.parametrize("H,E,K,I,Sh,T", [(512, 32, 4, 256, 256, 3), (2048, 64, 10, 512, 512, 2),
                                          (6, 4, 2, 4, 4, 7), (1000, 20, 3, 300, 200, 2)])
def test_f32_moe_bit_exact_vs_oracle(ctx, H, E, K, I, Sh, T):
    # Random F32 layers, including sizes that are no multiple of 4 and a
    # shared intermediate of its own: output and every checkpoint bit for bit
    key = lambda r: S.stream_key(S.W_MOE + 700 + H, r)
    w = {"router": S.normal_f32(key(S.R_ROUTER), E * H, 0.05).reshape(E, H),
         "gate": S.normal_f32(key(S.R_GATE), E * I * H, 0.05),
         "up": S.normal_f32(key(S.R_UP), E * I * H, 0.05),
         "down": S.normal_f32(key(S.R_DOWN), E * H * I, 0.05),
         "shared_gate": S.normal_f32(key(S.R_SHARED_GATE), Sh * H, 0.05),
         "shared_up": S.normal_f32(key(S.R_SHARED_UP), Sh * H, 0.05),
         "shared_down": S.normal_f32(key(S.R_SHARED_DOWN), H * Sh, 0.05),
         "shared_gate_weight": S.normal_f32(key(S.R_SHARED_GATE_W), H, 0.05)}
    dims = dict(hidden=H, experts=E, top_k=K, inter=I, shared_inter=Sh)
    x = S.normal_f32(key(S.R_HIDDEN), T * H).reshape(T, H)
    out, seen = run_f32(ctx, dims, w, x)
    check_order(seen, T, K)
    ref, tr = kq_oracle.moe_execute(dims, {r: (F32, w[r]) for r in ROLES}, x, trace=True)
    assert_bit_exact_vs_oracle(seen, out, ref, tr, T, K)
    # without observers the output is the same
    out2, seen2 = run_f32(ctx, dims, w, x, observe=False)
    assert seen2 == [] and np.array_equal(out2.view(np.uint32), out.view(np.uint32))


def test_f32_moe_fails_closed(ctx):
    # the reference's statuses (src/kq_moe_qwen38.c:604-665); no observer
    # runs on a failed call
    dims, w = tier_a()
    H = dims["hidden"]
    x = hex_le_f32(TIER_A["calibration"][0]["input"]["le_hex"]).reshape(-1, H)
    cfg = kq_hip.MoeConfig(H, dims["experts"], dims["top_k"], dims["inter"], dims["shared_inter"])

    def call(wd, xin, counts=None, scratch_cut=0, out_is_x=False):
        bufs = {DEV_ROLE[r]: ctx.upload(np.ascontiguousarray(wd[r], np.float32)) for r in ROLES}
        cnt = {DEV_ROLE[r]: int(np.asarray(wd[r]).size) for r in ROLES}
        cnt.update(counts or {})
        n = cfg.f32_scratch_bytes(xin.shape[0])
        scratch, dx, dout = ctx.alloc(n), ctx.upload(xin), ctx.alloc(xin.size * 4)
        try:
            return ctx.moe_execute_f32(cfg, kq_hip.moe_weights_f32(bufs, cnt), dx, xin.shape[0],
                                       dx if out_is_x else dout, scratch, n - scratch_cut,
                                       observe=True)
        finally:
            for b in list(bufs.values()) + [scratch, dx, dout]:
                b.close()

    with pytest.raises(kq_hip.KqError) as e:
        call(w, x, counts={"routed_down": w["down"].size - 1})
    assert e.value.name == "DIMENSION_MISMATCH"
    bad = dict(w)
    bad["down"] = w["down"].copy()
    bad["down"][3].flat[5] = np.nan  # the last expert's down stack, selected or not
    with pytest.raises(kq_hip.KqError) as e:
        call(bad, x)
    assert e.value.name == "NUMERIC_DOMAIN"
    xb = x.copy()
    xb[0, 2] = np.inf
    with pytest.raises(kq_hip.KqError) as e:
        call(w, xb)
    assert e.value.name == "NUMERIC_DOMAIN"
    with pytest.raises(kq_hip.KqError) as e:
        call(w, x, scratch_cut=256)
    assert e.value.name == "BUFFER_TOO_SMALL"
    with pytest.raises(kq_hip.KqError) as e:
        call(w, x, out_is_x=True)
    assert e.value.name == "ALIASING_VIOLATION"
    # and the context still runs the layer correctly
    out, seen = run_f32(ctx, dims, w, x)
    ref = kq_oracle.moe_execute(dims, {r: (F32, w[r]) for r in ROLES}, x)
    assert np.array_equal(out.view(np.uint32), ref.view(np.uint32))
    cfg.close()
