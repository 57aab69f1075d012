"""Oracle gated residual (hyper-connection read / write around a layer block)
against the reference's layer fixtures (Tier A: 4 branches x hidden 8, rank
4, 4 experts, top-2; Transformers Class-C expected values).

Per token the chain is (src/kq_layer.c:697-813):
  per-layer embedding (PLE layers): input += ple_output
  attention read:  mixed_attn = gr_read(input)             == attn_gr
  after the mixer: after = gr_write(input, mixer_output, write_gate_attn)
  MoE read:        mixed_moe = gr_read(after)              == moe_gr
  MoE:             moe_execute(mixed_moe)                   == moe_output
  output:          gr_write(after, moe_output, write_gate_moe) == output
with mixer_output taken from the fixture (the GDN / QSA mixers are not on
this path). The bound is the contract's calibrated absolute limit (2e-6,
layer-native-validation.json), which the reference's own C code meets.
"""
import numpy as np
import pytest

from conftest import load_golden

import kq_oracle

LAYER = load_golden("layer_tier_a.json")
EPS = 1.0e-6  # src/kq_layer.c:146
LIMIT = LAYER["limit_abs"]
DIMS = LAYER["reduced"]


def arr(rec):
    return np.frombuffer(bytes.fromhex(rec["le_hex"]), np.float32).reshape(rec["shape"])


def gr_weights(w, prefix):
    return {"norm": arr(w[prefix + ".hc_norm.weight"]),
            "down": (kq_oracle.F32, arr(w[prefix + ".input_mix_weight_down.weight"])),
            "up": (kq_oracle.F32, arr(w[prefix + ".input_mix_weight_up.weight"])),
            "inject": arr(w[prefix + ".block_inject_weight.weight"])}


def moe_weights(w):
    I = DIMS["intermediate"]
    gate_up = arr(w["mlp.experts.gate_up_proj"])  # [E, 2I, H]: gate rows then up rows
    F32 = kq_oracle.F32
    return {"router": (F32, arr(w["mlp.gate.weight"])),
            "gate": (F32, np.ascontiguousarray(gate_up[:, :I, :])),
            "up": (F32, np.ascontiguousarray(gate_up[:, I:, :])),
            "down": (F32, np.ascontiguousarray(arr(w["mlp.experts.down_proj"]))),
            "shared_gate": (F32, arr(w["mlp.shared_expert.gate_proj.weight"])),
            "shared_up": (F32, arr(w["mlp.shared_expert.up_proj.weight"])),
            "shared_down": (F32, arr(w["mlp.shared_expert.down_proj.weight"])),
            "shared_gate_weight": (F32, arr(w["mlp.shared_expert_gate.weight"]))}


def read(branches, g):
    return kq_oracle.gr_read(branches, DIMS["hidden"], DIMS["rank"], EPS, g["norm"],
                             g["down"], g["up"], g["inject"])


CASES = [(corpus, c) for corpus in ("calibration", "holdout") for c in LAYER[corpus]]


@pytest.mark.parametrize("corpus,case", CASES, ids=[f"{k}-{c['id']}" for k, c in CASES])
def test_gated_residual_chain(corpus, case):
    H = DIMS["hidden"]
    w = case["weights"]
    attn, mlp = gr_weights(w, "attn_hyper_connection"), gr_weights(w, "mlp_hyper_connection")
    x = arr(case["input"])[0]
    out = arr(case["output"])[0]
    cp = {k: arr(v)[0] for k, v in case["checkpoints"].items()}
    dims = dict(hidden=H, experts=DIMS["experts"], top_k=DIMS["top_k"],
                inter=DIMS["intermediate"], shared_inter=DIMS["intermediate"])
    mw = moe_weights(w)
    if "ple_output" in cp:
        # the per-layer embedding is added before the attention read
        # (src/kq_layer.c:721): current = input + ple_output
        x = (x + cp["ple_output"]).astype(np.float32)
    for t in range(x.shape[0]):
        ra = read(x[t], attn)
        assert np.abs(ra["mixed"] - cp["attn_gr"][t]).max() <= LIMIT
        after = kq_oracle.gr_write(x[t], H, cp["mixer_output"][t], ra["write_gate"])
        rm = read(after, mlp)
        assert np.abs(rm["mixed"] - cp["moe_gr"][t]).max() <= LIMIT
        moe = kq_oracle.moe_execute(dims, mw, rm["mixed"][None, :])[0]
        assert np.abs(moe - cp["moe_output"][t]).max() <= LIMIT
        y = kq_oracle.gr_write(after, H, cp["moe_output"][t], rm["write_gate"])
        assert np.abs(y - out[t]).max() <= LIMIT


def test_gr_write_closed_form():
    rng = np.random.default_rng(5)
    b = rng.standard_normal(4 * 8).astype(np.float32)
    o = rng.standard_normal(8).astype(np.float32)
    g = rng.standard_normal(4).astype(np.float32)
    want = (b.reshape(4, 8) + (o[None, :] * g[:, None]).astype(np.float32)).reshape(-1)
    assert np.array_equal(kq_oracle.gr_write(b, 8, o, g), want.astype(np.float32))


def test_gr_read_quantized_rows_equal_dequantized_f32():
    # The provider path reads packed rows through row dots: a Q8_0 down/up
    # must give what the same weights dequantized to F32 give.
    import kq_synth as S
    H, NB, R = 64, 4, 32
    W = NB * H
    x = S.normal_f32(S.stream_key(S.W_MOE + 70, 1), W)
    norm = (S.normal_f32(S.stream_key(S.W_MOE + 70, 2), W) * np.float32(0.1))
    down_q = S.quant_matrix("Q8_0", S.stream_key(S.W_MOE + 70, 3), R, W)
    up_q = S.quant_matrix("Q8_0", S.stream_key(S.W_MOE + 70, 4), W, R)
    inject = S.normal_f32(S.stream_key(S.W_MOE + 70, 5), NB * W) * np.float32(0.02)
    down_f = kq_oracle.dequantize(kq_oracle.Q8_0, down_q.reshape(-1)).reshape(R, W)
    up_f = kq_oracle.dequantize(kq_oracle.Q8_0, up_q.reshape(-1)).reshape(W, R)
    a = kq_oracle.gr_read(x, H, R, EPS, norm, (kq_oracle.Q8_0, down_q), (kq_oracle.Q8_0, up_q),
                          inject)
    b = kq_oracle.gr_read(x, H, R, EPS, norm, (kq_oracle.F32, down_f), (kq_oracle.F32, up_f),
                          inject)
    for k in a:
        assert np.array_equal(a[k].view(np.uint32), b[k].view(np.uint32)), k
