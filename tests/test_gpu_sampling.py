"""The device sampler (kq_hip_sampling_select_f32, kq_hip_lm_head_sample_f32)
through the C ABI against the reference's sampling evidence and the oracle.

Bars: the selected id, the retained counts, the RNG word, the RNG state
after the call and the result's float fields bit for bit equal to the
oracle's restatement of kq_sampling_select_f32 (src/kq_sampling.c:576-772)
on the same logits and word; the processed logits and the final
probabilities of every id bit for bit equal to the oracle's work arrays; on
the reference's calibration and holdout cases, membership, selection and
RNG exact and probabilities within the calibrated contract; statuses in the
reference's order, and the RNG state untouched by any failing call."""
import ctypes as C

import numpy as np
import pytest

from conftest import load_golden, ulp_distance

import kq_hip
import kq_oracle
import kq_synth as S

pytestmark = pytest.mark.gpu

SV = load_golden("sampling_vectors.json")
VOCAB, CANON = kq_hip.QWEN38_VOCAB, kq_hip.QWEN38_CANONICAL
STATUS = {0: "OK", 31: "INVALID_TOKEN_ID", 39: "NUMERIC_DOMAIN"}


@pytest.fixture(scope="module")
def ctx():
    c = kq_hip.Context(0)
    yield c
    c.close()


class Sampler:
    """One config, its scratch and a logits buffer on the device."""

    def __init__(self, ctx, pol: dict, vocab=None, canonical=None):
        self.ctx, self.pol = ctx, pol
        self.cfg = kq_hip.SamplingConfig(kq_hip.sampling_policy(**pol), vocab, canonical)
        self.n = self.cfg.vocabulary
        self.canonical = CANON if vocab is None else canonical
        self.scratch = ctx.alloc(self.cfg.scratch_bytes)
        self.logits = ctx.alloc(self.n * 4)

    def run(self, logits, state):
        d = kq_hip.Diagnostic()
        lg = np.ascontiguousarray(logits, np.float32)
        assert lg.size == self.n
        kq_hip.check(kq_hip.lib().kq_hip_upload(self.ctx._h, C.c_void_p(self.logits.ptr),
                                                lg.ctypes.data, lg.nbytes, C.byref(d)), d)
        try:
            return "OK", self.ctx.sample(self.cfg, state, self.logits, self.scratch)
        except kq_hip.KqError as e:
            return e.name, None

    def close(self):
        self.scratch.close()
        self.logits.close()
        self.cfg.close()


def f32bits(v) -> int:
    return int(np.array(v, np.float32).view(np.uint32))


def check_against_oracle(s: Sampler, logits, seed, stream, work=True):
    """Run the device and the oracle on the same logits and RNG state; every
    field and (optionally) both work arrays bit for bit."""
    st = kq_hip.rng_seed(seed, stream)
    before = bytes(st)
    name, r = s.run(logits, st)
    ost = kq_oracle.rng_seed(seed, stream)
    word = kq_oracle.rng_next(ost)
    ostatus, o, osc, opr = kq_oracle.sample(s.pol, logits, word, s.canonical)
    assert name == STATUS[ostatus], (name, ostatus)
    if name != "OK":
        assert bytes(st) == before  # no state advance on failure
        return name, None
    assert (st.state, st.draws, st.integrity) == (ost.state, ost.draws, ost.integrity)
    assert (r.rng_draws_before, r.rng_draws_after) == (0, 1)
    for f in ("selected_token_id", "top_k_retained_count", "retained_count", "rng_word"):
        assert getattr(r, f) == getattr(o, f), f
    for f in ("selected_probability", "maximum_probability", "normalized_sum_f32"):
        assert f32bits(getattr(r, f)) == f32bits(getattr(o, f)), f
    assert np.float64(r.uniform_value).tobytes() == np.float64(o.uniform_value).tobytes()
    if work:
        sc, pr = s.ctx.sampling_work(s.cfg, s.scratch)
        assert np.array_equal(sc.view(np.uint32), osc.view(np.uint32))
        assert np.array_equal(pr.view(np.uint32), opr.view(np.uint32))
    return name, r


def logits_of(case):
    lg = np.full(VOCAB, case["base_logit"], np.float32)
    for k, v in case["overrides"].items():
        lg[int(k)] = v
    return lg


def f32(hexle):
    return np.frombuffer(bytes.fromhex(hexle), "<f4")[0]


@pytest.mark.parametrize("case", SV["calibration"] + SV["holdout"], ids=lambda c: c["id"])
def test_reference_cases(ctx, case):
    o = case["oracle"]
    s = Sampler(ctx, {k: case["policy"][k] for k in ("temperature", "top_p", "top_k")})
    st = kq_hip.rng_seed(case["seed"], case["stream"])
    assert st.state == int(o["rng_state_before"], 16)
    before = bytes(st)
    name, r = s.run(logits_of(case), st)
    assert name == o["expected_status"]
    if name == "OK":
        assert r.selected_token_id == o["selected_token_id"]
        assert r.top_k_retained_count == o["top_k_retained_count"]
        assert r.retained_count == o["retained_count"]
        assert r.rng_word == int(o["rng_word"], 16)
        assert st.state == int(o["rng_state_after"], 16)
        sc, pr = ctx.sampling_work(s.cfg, s.scratch)
        assert list(np.flatnonzero(pr > 0)) == o["retained_ids"]
        lim = SV["floating_contract"]["probability"]
        for rec in o["retained"]:
            t = rec["token_id"]
            assert f32bits(sc[t]) == f32bits(f32(rec["processed_logit_f32_le_hex"]))
            want = f32(rec["probability_f32_le_hex"])
            assert abs(float(pr[t]) - float(want)) <= lim["maximum_absolute"] or \
                ulp_distance(pr[t], want) <= lim["maximum_ulp"]
    else:
        assert bytes(st) == before
    # and bit for bit with the oracle on the same case
    check_against_oracle(s, logits_of(case), case["seed"], case["stream"])
    s.close()


POLICIES = [{"temperature": 1.0, "top_k": 20, "top_p": 0.95},
            {"temperature": 0.7, "top_k": 0, "top_p": 0.9},
            {"temperature": 1.3, "top_k": 50, "top_p": 1.0},
            {"temperature": 1.0, "top_k": 0, "top_p": 1.0},
            {"temperature": 0.25, "top_k": 2000, "top_p": 0.5},
            {"temperature": 1.0, "top_k": 1, "top_p": 0.95},
            {"temperature": 1.0, "top_k": 5000, "top_p": 0.999},
            {"temperature": 2.0, "top_k": 0, "top_p": 0.0}]


@pytest.mark.parametrize("pi", range(len(POLICIES)))
def test_seeded_logits_full_vocabulary(ctx, pi):
    pol = POLICIES[pi]
    s = Sampler(ctx, pol)
    rng = np.random.default_rng(100 + pi)
    for trial in range(3):
        lg = (rng.standard_normal(VOCAB) * (1 + 3 * trial)).astype(np.float32)
        if trial == 2:
            lg[rng.integers(0, VOCAB, 50)] = lg.max()  # ties at the top
        check_against_oracle(s, lg, 1000 + trial, 77 + pi)
    s.close()


@pytest.mark.parametrize("sequential", [False, True], ids=["certified", "sequential"])
def test_many_kept_draw_paths(ctx, monkeypatch, sequential):
    # Over more kept ids than the LDS sort holds, the draw's binary64 walk
    # is replaced by parallel prefix sums when they are exact or when the
    # threshold clears the summation error bound; KQ_HIP_SAMPLE_SEQUENTIAL=1
    # forces the sequential walk. Both must give the oracle's draw, on
    # spreads where the prefix sums are exact (all probabilities multiples
    # of 2^-52: equal logits) and where they are not (N(0, s) logits, and
    # weights down to underflow).
    if sequential:
        monkeypatch.setenv("KQ_HIP_SAMPLE_SEQUENTIAL", "1")
    rng = np.random.default_rng(4242)
    cases = [np.full(VOCAB, 0.25, np.float32)]
    cases += [(rng.standard_normal(VOCAB) * sd).astype(np.float32) for sd in (0.5, 1.0, 3.0)]
    under = -np.linspace(0.0, 120.0, VOCAB, dtype=np.float32)
    rng.shuffle(under)
    cases.append(under)
    for pol in ({"temperature": 1.0, "top_k": 0, "top_p": 1.0},
                {"temperature": 0.8, "top_k": 0, "top_p": 0.7}):
        s = Sampler(ctx, pol)
        for ci, lg in enumerate(cases):
            for seed in range(4):
                check_against_oracle(s, lg, 31 * ci + seed, 9, work=seed == 0)
        s.close()


# vocabularies around the wave (64), the prep block (256), the in-LDS
# kept-id sort's capacity (4096) and the draw's 2048 LDS checkpoints of 512
# ids each (past 1,048,576 ids a checkpoint covers several runs)
SMALL = [(1, 1), (2, 1), (63, 60), (64, 64), (65, 65), (1000, 997), (4096, 4096),
         (4097, 4000), (8191, 8191), (70001, 69000), (1200007, 1200000)]
SMALL_POL = [{"temperature": 1.0, "top_k": 0, "top_p": 1.0},
             {"temperature": 0.5, "top_k": 0, "top_p": 0.8},
             {"temperature": 1.0, "top_k": 3, "top_p": 0.95},
             {"temperature": 0.9, "top_k": 1 << 30, "top_p": 1.0}]  # top-k = vocabulary


@pytest.mark.parametrize("vocab,canonical", SMALL, ids=[f"{v}-{c}" for v, c in SMALL])
def test_ragged_vocabularies(ctx, vocab, canonical):
    rng = np.random.default_rng(vocab)
    for pj, pol in enumerate(SMALL_POL):
        pol = dict(pol, top_k=min(pol["top_k"], vocab))
        s = Sampler(ctx, pol, vocab, canonical)
        for trial in range(3):
            lg = (rng.standard_normal(vocab) * 2).astype(np.float32)
            check_against_oracle(s, lg, 7 * trial + pj, 5)
        s.close()


def test_ties_everywhere(ctx):
    # all logits equal: top-k keeps every tie (all 248,320 ids, past the LDS
    # sort's capacity), the draw is uniform over ids
    lg = np.full(VOCAB, 0.5, np.float32)
    for pol in ({"temperature": 1.0, "top_k": 5, "top_p": 1.0},
                {"temperature": 1.0, "top_k": 0, "top_p": 0.5},
                {"temperature": 1.0, "top_k": 20, "top_p": 0.95}):
        s = Sampler(ctx, pol)
        for seed in range(3):
            check_against_oracle(s, lg, seed, 11)
        s.close()


def test_signed_zero_and_underflow(ctx):
    rng = np.random.default_rng(3)
    s = Sampler(ctx, {"temperature": 1.0, "top_k": 0, "top_p": 1.0})
    lg = np.zeros(VOCAB, np.float32)
    lg[rng.integers(0, VOCAB, 1000)] = -0.0  # -0 and +0 compare equal: id order decides
    check_against_oracle(s, lg, 1, 2)
    # weights that underflow to 0 are retained but carry no mass
    lg = -np.linspace(0.0, 200.0, VOCAB, dtype=np.float32)
    rng.shuffle(lg)
    name, r = check_against_oracle(s, lg, 2, 2)
    assert r.retained_count == VOCAB
    s.close()


def test_numeric_failures_leave_state(ctx):
    s = Sampler(ctx, {"temperature": 0.25, "top_k": 20, "top_p": 0.95})
    base = np.random.default_rng(9).standard_normal(VOCAB).astype(np.float32)
    for bad in (np.nan, np.inf, -np.inf, 3.0e38):  # 3e38 / 0.25 overflows
        lg = base.copy()
        lg[123457] = bad
        name, _ = check_against_oracle(s, lg, 4, 4, work=False)
        assert name == "NUMERIC_DOMAIN"
    s.close()


def integrity(st) -> int:
    h = 1469598103934665603
    for f in (st.version, st.reserved, st.seed, st.stream, st.state, st.increment, st.draws):
        h = ((h ^ f) * 1099511628211) % 2 ** 64
    return h


def test_statuses_in_reference_order(ctx):
    L = kq_hip.lib()
    s = Sampler(ctx, {"temperature": 1.0, "top_k": 20, "top_p": 0.95})
    lg = np.random.default_rng(1).standard_normal(VOCAB).astype(np.float32)
    name, _ = s.run(lg, kq_hip.rng_seed(1, 2))
    assert name == "OK"

    def call(cfg=s.cfg.handle, state=None, logits=s.logits.ptr, count=VOCAB,
             scratch=s.scratch.ptr, nbytes=s.cfg.scratch_bytes, result=True):
        st = state if state is not None else kq_hip.rng_seed(1, 2)
        before = bytes(st)
        r, d = kq_hip.SamplingResult(), kq_hip.Diagnostic()
        code = L.kq_hip_sampling_select_f32(ctx._h, C.c_void_p(cfg), C.byref(st),
                                            C.c_void_p(logits), count, C.c_void_p(scratch),
                                            nbytes, C.byref(r) if result else None, C.byref(d))
        if code != 0:
            assert bytes(st) == before
        return kq_hip.STATUS[code]

    assert call(cfg=None) == "INCOMPATIBLE_SAMPLING"
    assert call(count=VOCAB - 1) == "INVALID_ARGUMENT"
    assert call(logits=None) == "INVALID_ARGUMENT"
    assert call(result=False) == "INVALID_ARGUMENT"
    bad = kq_hip.rng_seed(1, 2)
    bad.integrity ^= 1
    assert call(state=bad) == "INVALID_RNG_STATE"
    assert call(nbytes=s.cfg.scratch_bytes - 1) == "BUFFER_TOO_SMALL"
    assert call(scratch=None) == "BUFFER_TOO_SMALL"
    assert call(logits=s.scratch.ptr + 4096) == "ALIASING_VIOLATION"
    # the draw counter at its maximum: a numeric failure is reported first,
    # then the counter overflow (src/kq_sampling.c:742-748)
    top = kq_hip.rng_seed(1, 2)
    top.draws = 2 ** 64 - 1
    top.integrity = integrity(top)
    assert call(state=top) == "ARITHMETIC_OVERFLOW"
    s.run(np.where(np.arange(VOCAB) == 5, np.float32(np.nan), lg), kq_hip.rng_seed(1, 2))
    assert call(state=top) == "NUMERIC_DOMAIN"
    s.close()


def test_decode_sequence_200_draws(ctx):
    # one RNG stream across 200 steps of changing logits, as a decode loop
    # draws: ids, words and states exact at every step
    s = Sampler(ctx, {"temperature": 1.0, "top_k": 20, "top_p": 0.95})
    rng = np.random.default_rng(42)
    st = kq_hip.rng_seed(2024, kq_hip.SAMPLING_DEFAULT_STREAM)
    ost = kq_oracle.rng_seed(2024, kq_hip.SAMPLING_DEFAULT_STREAM)
    lg = (rng.standard_normal(VOCAB) * 3).astype(np.float32)
    for step in range(200):
        lg[rng.integers(0, VOCAB, 64)] += rng.standard_normal(64).astype(np.float32) * 4
        lg[CANON:] = -30.0  # padding ids out of reach: every step succeeds
        name, r = s.run(lg, st)
        word = kq_oracle.rng_next(ost)
        ostatus, o, _, _ = kq_oracle.sample(s.pol, lg, word, CANON)
        assert name == STATUS[ostatus], step
        if name == "OK":
            assert r.selected_token_id == o.selected_token_id, step
            assert r.rng_word == word and (r.rng_draws_before, r.rng_draws_after) == (step, step + 1)
        assert (st.state, st.draws) == (ost.state, ost.draws), step
    s.close()


@pytest.mark.parametrize("vocab,cols", [(8192, 2048), (VOCAB, 2048)])
def test_lm_head_sample_fused(ctx, vocab, cols):
    # the Q6_K LM head of the reference model (248,320 x 2048) and a small one
    t = kq_hip.TYPE_Q6_K
    key = S.stream_key(S.W_MATVEC_Q8_0, 95, vocab, cols)
    w = S.quant_matrix("Q6_K", key, vocab, cols)
    h = S.normal_f32(key ^ 0x55, cols)
    dw, dh = ctx.upload(w), ctx.upload(h)
    canon = CANON if vocab == VOCAB else vocab - 5
    pol = {"temperature": 0.8, "top_k": 40, "top_p": 0.9}
    s = Sampler(ctx, pol, None if vocab == VOCAB else vocab, None if vocab == VOCAB else canon)
    logits = ctx.alloc(vocab * 4)
    ref_logits = ctx.alloc(vocab * 4)
    for seed in range(5):
        st = kq_hip.rng_seed(seed, 3)
        r = ctx.lm_head_sample(s.cfg, st, t, dw, vocab, cols, dh, logits, s.scratch)
        # the fused logits are the matvec's, bit for bit
        ctx.matvec(t, dw, vocab, cols, dh, 1, ref_logits)
        got = ctx.download(logits, np.float32, vocab)
        assert np.array_equal(got.view(np.uint32),
                              ctx.download(ref_logits, np.float32, vocab).view(np.uint32))
        # and the draw is the oracle's on those logits
        ost = kq_oracle.rng_seed(seed, 3)
        word = kq_oracle.rng_next(ost)
        ostatus, o, _, _ = kq_oracle.sample(pol, got, word, canon)
        assert ostatus == 0 and r.selected_token_id == o.selected_token_id
        assert f32bits(r.selected_probability) == f32bits(o.selected_probability)
        assert (st.state, st.draws) == (ost.state, ost.draws)
    for b in (dw, dh, logits, ref_logits):
        b.close()
    s.close()
