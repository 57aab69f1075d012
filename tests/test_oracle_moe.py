"""Pins the CPU oracle's MoE routing and execution against the reference's
golden evidence (research/operators/.../moe-*.json). CPU only."""
import numpy as np
import pytest

from conftest import hex_le_f32, load_golden, ulp_distance

TIER_A = load_golden("moe_tier_a.json")
ROUTING = load_golden("moe_routing_vectors.json")


def tier_a_weights():
    cfg = TIER_A["tier_a_config"]
    w = {k: hex_le_f32(v["le_hex"]).reshape(v["shape"]) for k, v in TIER_A["weights"].items()}
    E, I, H = cfg["expert_count"], cfg["routed_intermediate_size"], cfg["hidden_size"]
    gate_up = w["experts.gate_up_proj"]  # [E, 2I, H]: gate rows then up rows
    F32 = 0
    weights = {
        "router": (F32, np.ascontiguousarray(w["gate.weight"])),
        "gate": (F32, np.ascontiguousarray(gate_up[:, :I, :])),
        "up": (F32, np.ascontiguousarray(gate_up[:, I:, :])),
        "down": (F32, np.ascontiguousarray(w["experts.down_proj"])),
        "shared_gate": (F32, np.ascontiguousarray(w["shared_expert.gate_proj.weight"])),
        "shared_up": (F32, np.ascontiguousarray(w["shared_expert.up_proj.weight"])),
        "shared_down": (F32, np.ascontiguousarray(w["shared_expert.down_proj.weight"])),
        "shared_gate_weight": (F32, np.ascontiguousarray(w["shared_expert_gate.weight"])),
    }
    dims = dict(hidden=H, experts=E, top_k=cfg["top_k"], inter=I,
                shared_inter=cfg["shared_intermediate_size"])
    return dims, weights


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
    ulp = ulp_distance(got, want)
    ok = (a <= contract["abs_limit"]) | (rel <= contract["rel_limit"]) | (ulp <= contract["ulp_limit"])
    return bool(ok.all())


AGG = {"router_logits": "router_logits", "router_probabilities": "router_probs",
       "selected_weights": "selected_weights", "routed_weighted_sum": "routed_sum",
       "shared_gate_projection": "shared_gate_proj", "shared_up_projection": "shared_up_proj",
       "shared_activated": "shared_activated", "shared_output": "shared_output",
       "shared_gate_logit": "shared_scale_logit", "shared_gate": "shared_scale",
       "gated_shared_output": "gated_shared", "final_output": None}
EXPERT = {"gate": "expert_gate", "up": "expert_up", "activated": "expert_activated",
          "output": "expert_output", "weighted_output": "expert_weighted"}


@pytest.mark.parametrize("case", TIER_A["calibration"] + TIER_A["holdout"],
                         ids=lambda c: c["id"])
def test_tier_a_checkpoints(oracle, case):
    # tools/validate-native-moe.py:222-268 comparison, contracts from
    # moe-native-validation.json (abs OR rel OR ulp within limit).
    dims, weights = tier_a_weights()
    H = dims["hidden"]
    x = hex_le_f32(case["input"]["le_hex"]).reshape(-1, H)
    out, tr = oracle.moe_execute(dims, weights, x, trace=True)
    exp = case["expected"]
    assert [list(map(int, r)) for r in tr["selected_ids"]] == exp["selected_expert_ids"]
    for key, field in AGG.items():
        want = hex_le_f32(exp[key]["le_hex"])
        got = out if field is None else tr[field]
        assert within(TIER_A["contracts"][key], got, want), key
    for sel in exp["selected_experts"]:
        t, pos = sel["token"], sel["top_k_position"]
        assert tr["selected_ids"][t][pos] == sel["expert_id"]
        for key, field in EXPERT.items():
            want = hex_le_f32(sel[key]["le_hex"])
            assert within(TIER_A["contracts"]["routed_" + key], tr[field][t, pos], want), key


@pytest.mark.parametrize("case", ROUTING["cases"], ids=lambda c: c["id"])
def test_tier_b_routing_exact(oracle, case):
    # 512 experts, top-10, hidden 4: EXACT_DISCRETE ids.
    cfg = ROUTING["config"]
    H, E, K = cfg["hidden_size"], cfg["expert_count"], cfg["top_k"]
    router = hex_le_f32(case["router_weight"]["le_hex"]).reshape(E, H)
    x = hex_le_f32(case["input"]["le_hex"]).reshape(-1, H)
    dims = dict(hidden=H, experts=E, top_k=K, inter=1, shared_inter=1)
    for t in range(x.shape[0]):
        logits, probs, ids, w = oracle.moe_route(dims, (0, router), x[t])
        assert list(map(int, ids)) == case["expected"]["selected_expert_ids"][t]
        want_l = hex_le_f32(case["expected"]["router_logits"]["le_hex"]).reshape(-1, E)[t]
        assert np.array_equal(logits, want_l)
        # The fixture's floats come from PyTorch's vectorised softmax, whose
        # sum order differs from the scalar left-to-right sum; the reference
        # validator compares only ids here (tools/validate-native-moe.py
        # run_routing_case). Floats are held to n*2^-24 relative, the error
        # bound of an n-term sequential sum of positive terms.
        want_p = hex_le_f32(case["expected"]["router_probabilities"]["le_hex"]).reshape(-1, E)[t]
        np.testing.assert_allclose(probs, want_p, rtol=E * 2.0 ** -24, atol=0)
        want_w = hex_le_f32(case["expected"]["selected_weights"]["le_hex"]).reshape(-1, K)[t]
        np.testing.assert_allclose(w, want_w, rtol=E * 2.0 ** -24, atol=0)


def test_reference_unit_routing(oracle):
    # tests/moe_test.c:157-191: equal logits -> ids 0,1 with weights 0.5/0.5.
    dims = dict(hidden=6, experts=4, top_k=2, inter=4, shared_inter=4)
    router = np.zeros((4, 6), np.float32)
    _, _, ids, w = oracle.moe_route(dims, (0, router), np.ones(6, np.float32))
    assert list(ids) == [0, 1] and list(w) == [0.5, 0.5]
    # tests/moe_test.c:253-268: 64 experts, one dominant late expert.
    dims = dict(hidden=1, experts=64, top_k=10, inter=1, shared_inter=1)
    router = np.zeros((64, 1), np.float32)
    router[63] = 1.0
    _, _, ids, _ = oracle.moe_route(dims, (0, router), np.ones(1, np.float32))
    assert list(ids) == [63] + list(range(1, 10))


def _select_brute(p, k):
    """Direct restatement of the documented selection rule
    (docs/MOE-OPERATOR-CONTRACT.md:81-92) as a set computation, used to
    cross-check the partial-selection loop on random tie-heavy inputs."""
    n = len(p)
    vals = np.sort(p)[::-1]
    vstar = vals[k - 1]
    G = [i for i in range(n) if p[i] > vstar]
    E = [i for i in range(n) if p[i] == vstar]
    count = 0
    t0 = None
    for t in range(n):
        if p[t] >= vstar:
            count += 1
        if count == k and t >= k - 1:
            t0 = t
            break
    e_in = [e for e in E if e <= t0]
    g_after = len([g for g in G if g > t0])
    keep = set(G) | set(e_in[g_after:])
    return sorted(keep, key=lambda i: (-p[i], i))


def test_select_top_k_matches_set_characterisation(oracle):
    rng = np.random.default_rng(21)
    for trial in range(400):
        n = int(rng.integers(10, 80))
        k = int(rng.integers(1, min(n, 12) + 1))
        p = rng.integers(0, 4 if trial % 2 else 40, n).astype(np.float32)
        ids = oracle.moe_select_top_k(p, k)
        assert list(map(int, ids)) == _select_brute(p, k)


def test_permutation_is_stable_counting_sort(oracle):
    rng = np.random.default_rng(4)
    T, K, E = 37, 5, 16
    ids = np.stack([rng.choice(E, K, replace=False) for _ in range(T)]).astype(np.uint32)
    off, tok, slot = oracle.moe_permutation(ids, E)
    pairs = sorted(((int(ids[t, s]), t, s) for t in range(T) for s in range(K)))
    assert [p[1] for p in pairs] == list(tok)
    assert [p[2] for p in pairs] == list(slot)
    counts = np.bincount(ids.ravel(), minlength=E)
    assert np.array_equal(np.diff(off), counts)


def test_quantized_moe_matches_dequantized_f32(oracle):
    # The packed-weight execution equals the F32 execution over the
    # dequantized matrices bit for bit: the provider path only replaces
    # where weights come from (src/kq_moe_qwen38.c:378-434).
    import kq_synth
    dims = dict(hidden=256, experts=8, top_k=3, inter=256, shared_inter=256)
    w = kq_synth.moe_weights(kq_synth.W_MOE + 40, 256, 8, 256, 256)
    Q4, Q6, F32 = oracle.Q4_K, oracle.Q6_K, oracle.F32
    packed = {"router": (F32, w["router"]), "gate": (Q4, w["gate"]), "up": (Q4, w["up"]),
              "down": (Q6, w["down"]), "shared_gate": (Q4, w["shared_gate"]),
              "shared_up": (Q4, w["shared_up"]), "shared_down": (Q6, w["shared_down"]),
              "shared_gate_weight": (F32, w["shared_gate_weight"])}
    deq = {k: (F32, oracle.dequantize(t, v) if t != F32 else v) for k, (t, v) in packed.items()}
    x = kq_synth.normal_f32(kq_synth.stream_key(kq_synth.W_MOE + 40, kq_synth.R_HIDDEN), 2 * 256)
    a = oracle.moe_execute(dims, packed, x.reshape(2, 256))
    b = oracle.moe_execute(dims, deq, x.reshape(2, 256))
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
