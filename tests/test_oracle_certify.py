"""Soundness of the device's certified one-token routing, on the CPU.

The one-token MoE execute skips the reference's binary32 router chains
(src/kq_numeric.c:474-496 through src/kq_moe_qwen38.c:276-376) when a
proven bound separates the selection (kestrel-q_amd/csrc/kq_moe.hip:
router_bounds, route_certify). oracle/kq_certify.c restates that decision
step by step; here it runs against the oracle's exact route on over a
million generated router/activation pairs, and on near ties planted at
gaps around the bound, inside the selection and far below the bound (where
the chains' rounding decides the order). A certified selection must always
be the exact route's ids in the exact route's order. The same campaign with
the bounds and margin scaled down (a planted unsound certification) must
find mismatches, so the campaign can see one."""
import pytest

import kq_oracle

THREADS = 8

# (experts, hidden, top_k, trials): 1,005,000 random cases in all
RANDOM = [(64, 128, 4, 500_000), (128, 256, 8, 200_000), (40, 64, 3, 150_000),
          (96, 512, 6, 100_000), (130, 256, 10, 50_000), (512, 2048, 10, 5_000)]


@pytest.mark.parametrize("E,H,K,n", RANDOM, ids=[f"{e}x{h}k{k}" for e, h, k, _ in RANDOM])
def test_certified_selection_is_exact_route_random(E, H, K, n):
    r = kq_oracle.certify_campaign(0x5EED + E + H, n, E, H, K, "random", threads=THREADS)
    assert r["route_failures"] == 0
    assert r["certified_mismatch"] == 0, r
    # logits ~N(0, 0.02 sqrt(H)): nearly every token certifies
    assert r["certified"] >= 0.9 * n, r


NEAR = [(64, 128, 4, 100_000), (128, 256, 8, 50_000), (512, 2048, 10, 3_000)]


@pytest.mark.parametrize("mode", ["tie-at-boundary", "tie-inside", "tie-below-bound"])
@pytest.mark.parametrize("E,H,K,n", NEAR, ids=[f"{e}x{h}k{k}" for e, h, k, _ in NEAR])
def test_certified_selection_is_exact_route_near_ties(E, H, K, n, mode):
    r = kq_oracle.certify_campaign(0xA11 + E + H, n, E, H, K, mode, threads=THREADS)
    assert r["route_failures"] == 0
    assert r["certified_mismatch"] == 0, r
    if mode == "tie-below-bound":
        # gaps of 2^-16 .. 2^-2 bounds: certification refuses them all, and
        # the chains' rounding flips some selections against the binary64
        # order (at 2048 columns the bound is loose enough that it rarely
        # does)
        assert r["certified"] == 0, r
        if H <= 256:
            assert r["rounding_decided"] > 0, r
    else:
        # gaps of 2^-6 .. 2^6 bounds straddle the certification threshold
        assert 0 < r["certified"] < n, r


@pytest.mark.parametrize("slack", [0.0, 0.01])
def test_campaign_catches_unsound_certification(slack):
    # bounds and margin scaled down: the campaign must report certified
    # selections that are not the exact route's
    r = kq_oracle.certify_campaign(99, 20_000, 64, 128, 4, "tie-below-bound",
                                   threads=THREADS, slack=slack)
    assert r["certified_mismatch"] > 0, r
    assert r["first_mismatch_plus_1"] > 0


def test_certified_selection_large_activations():
    # activations scaled by up to 2^28: the lower selected probabilities
    # underflow to zero and tie, and the CPU orders ties by id. The rule
    # that a pair's higher probability be a normal binary32 number keeps
    # certification sound there; without it the campaign finds certified
    # selections that are not the exact route's.
    n = 20_000
    r = kq_oracle.certify_campaign(0x5CA1E, n, 64, 128, 4, "large-activations", threads=THREADS)
    assert r["route_failures"] == 0
    assert r["certified_mismatch"] == 0, r
    assert 0 < r["certified"] < n, r
    r = kq_oracle.certify_campaign(0x5CA1E, n, 64, 128, 4, "large-activations", threads=THREADS,
                                   slack=-1.0)
    assert r["certified_mismatch"] > 0, r


def test_restatement_entry_matches_campaign_rule():
    # kqo_route_certify on one planted-free case: certified, ids equal to
    # the exact route's
    import numpy as np
    import kq_synth as S
    E, H, K = 512, 2048, 10
    router = S.normal_f32(S.stream_key(S.W_MOE, S.R_ROUTER, 77), E * H, 0.02).reshape(E, H)
    x = S.normal_f32(S.stream_key(S.W_MOE, S.R_HIDDEN, 77), H)
    cert, ids = kq_oracle.route_certify(router, x, K)
    dims = dict(hidden=H, experts=E, top_k=K, inter=1, shared_inter=1)
    _, _, exact_ids, _ = kq_oracle.moe_route(dims, (kq_oracle.F32, router), x)
    assert cert and np.array_equal(ids, exact_ids)
    # a duplicated selected row is an exact tie: never certified
    order = np.argsort(-(router.astype(np.float64) @ x.astype(np.float64)))
    router[order[K]] = router[order[K - 1]]
    cert, _ = kq_oracle.route_certify(router, x, K)
    assert not cert
