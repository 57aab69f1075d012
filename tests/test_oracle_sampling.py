"""The oracle's sampler (oracle/kq_sample.c) against the reference's sampling
evidence: the PCG32 RNG vectors (EXACT_BITS), the calibration and holdout
cases of research/sampling (membership, selection and RNG exact; processed
logits exact; probabilities within the calibrated contract) and, where
oracle/_ref is built, the reference's own kq_sampling_select_f32 on seeded
random logits, bit for bit. CPU only."""
import numpy as np
import pytest

from conftest import load_golden, ulp_distance

import kq_oracle
import kq_ref as R

SV = load_golden("sampling_vectors.json")
VOCAB, CANONICAL = 248320, 248077
STATUS = {"OK": 0, "INVALID_TOKEN_ID": 31, "NUMERIC_DOMAIN": 39}


def logits_of(case):
    lg = np.full(VOCAB, case["base_logit"], np.float32)
    for k, v in case["overrides"].items():
        lg[int(k)] = v
    return lg


def test_rng_vectors():
    for c in SV["rng"]["cases"]:
        st = kq_oracle.rng_seed(c["seed"], c["stream"])
        assert st.increment == int(c["increment_hex"], 16)
        assert st.state == int(c["seeded_state_hex"], 16)
        for w in c["words"]:
            word = kq_oracle.rng_next(st)
            assert word == int(w["word_hex"], 16) and st.draws == w["draw"]
            assert st.state == int(w["state_after_hex"], 16)
            assert float.fromhex(w["uniform_hex"]) == word / 4294967296.0
    for b in SV["rng"]["explicit_word_boundaries"]:
        assert int(b["word_hex"], 16) / 4294967296.0 == float.fromhex(b["uniform_hex"])


def f32(hexle):
    return np.frombuffer(bytes.fromhex(hexle), "<f4")[0]


@pytest.mark.parametrize("case", SV["calibration"] + SV["holdout"], ids=lambda c: c["id"])
def test_fixture_cases(case):
    o = case["oracle"]
    st = kq_oracle.rng_seed(case["seed"], case["stream"])
    assert st.state == int(o["rng_state_before"], 16)
    word = kq_oracle.rng_next(st)
    assert word == int(o["rng_word"], 16) and st.state == int(o["rng_state_after"], 16)
    status, r, scores, probs = kq_oracle.sample(case["policy"], logits_of(case), word, CANONICAL)
    assert status == STATUS[o["expected_status"]]
    assert r.selected_token_id == o["selected_token_id"]
    assert r.top_k_retained_count == o["top_k_retained_count"]
    assert r.retained_count == o["retained_count"]
    kept = np.flatnonzero(probs > 0)
    assert list(kept) == o["retained_ids"]
    lim = SV["floating_contract"]["probability"]
    for rec in o["retained"]:
        t = rec["token_id"]
        assert scores[t].view(np.uint32) == f32(rec["processed_logit_f32_le_hex"]).view(np.uint32)
        want = f32(rec["probability_f32_le_hex"])
        assert abs(float(probs[t]) - float(want)) <= lim["maximum_absolute"] or \
            ulp_distance(probs[t], want) <= lim["maximum_ulp"]


def test_categorical_boundary_words():
    # two kept tokens of equal probability: word 0 takes the first, 2^31 and
    # 2^32 - 1 the second (sampling-native-validation.json)
    lg = np.full(VOCAB, -80.0, np.float32)
    lg[0] = lg[1] = 5.0
    pol = {"temperature": 1.0, "top_k": 0, "top_p": 1.0}
    for b in SV["categorical_boundaries"]:
        st, r, _, _ = kq_oracle.sample(pol, lg, int(b["word_hex"], 16), CANONICAL)
        assert st == 0 and r.selected_token_id == b["selected_index"]


POLICIES = [{"temperature": 1.0, "top_k": 20, "top_p": 0.95},
            {"temperature": 0.7, "top_k": 0, "top_p": 0.9},
            {"temperature": 1.3, "top_k": 50, "top_p": 1.0},
            {"temperature": 1.0, "top_k": 0, "top_p": 1.0},
            {"temperature": 0.25, "top_k": 2000, "top_p": 0.5}]


@pytest.mark.skipif(not R.available(), reason="oracle/_ref not built (needs the reference sources)")
@pytest.mark.parametrize("pi", range(len(POLICIES)))
def test_against_reference_select(pi):
    pol = POLICIES[pi]
    rng = np.random.default_rng(pi)
    for trial in range(3):
        lg = (rng.standard_normal(VOCAB) * (1 + 3 * trial)).astype(np.float32)
        if trial == 2:
            lg[rng.integers(0, VOCAB, 50)] = lg.max()  # ties at the top
        seed, stream = 1000 + trial, 77 + pi
        status, res, after = R.sample(pol, seed, stream, lg)
        st = kq_oracle.rng_seed(seed, stream)
        word = kq_oracle.rng_next(st)
        ost, r, _, _ = kq_oracle.sample(pol, lg, word, CANONICAL)
        assert ost == status
        if status == 0:
            assert (after.state, after.draws, after.integrity) == (st.state, st.draws, st.integrity)
            for f in ("selected_token_id", "top_k_retained_count", "retained_count", "rng_word"):
                assert getattr(r, f) == getattr(res, f), f
            for f in ("selected_probability", "maximum_probability", "normalized_sum_f32",
                      "uniform_value"):
                assert np.array(getattr(r, f)).tobytes() == np.array(getattr(res, f)).tobytes(), f
