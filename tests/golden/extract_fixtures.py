"""Extract the reference's committed golden vectors into compact data fixtures.

Run in a container where the reference checkout exists:
    python tests/golden/extract_fixtures.py [/root/reference]

Only inputs, expected outputs and stated tolerance contracts are copied (as
hex strings); the fixtures are data, not source. Provenance of each file:

  numeric_vectors.json    research/numerics/.../dequant-vectors.json
                          (EXACT_BITS, oracle llama.cpp 90c26fcd to_float)
  primitive_vectors.json  research/numerics/.../primitive-{calibration,holdout}.json
                          (NumPy explicit F32 order; per-op ULP contracts)
  moe_tier_a.json         research/operators/.../moe-contract.json (weights,
                          Tier A dims), moe-{calibration,holdout}.json
                          (Transformers Class-C expected checkpoints) and the
                          calibrated contracts of moe-native-validation.json
  moe_routing_vectors.json research/operators/.../moe-routing-vectors.json
                          (512 experts, top-10, EXACT_DISCRETE)
  layer_tier_a.json       research/operators/.../layer-{calibration,holdout}.json
                          (Transformers Class-C layer input, output and the
                          ple_output / attn_gr / mixer_output / moe_gr /
                          moe_output checkpoints; the hyper-connection and MoE
                          weights only) and the layer-native-validation.json
                          contract
  sampling_vectors.json   research/sampling/.../sampling-{calibration,holdout}.json
                          (policy, seed, stream, logits as base + overrides,
                          expected retained ids / processed logits /
                          probabilities, selected id, RNG word and states),
                          sampling-rng-vectors.json (PCG32 words, EXACT_BITS)
                          and the float contract and categorical boundary
                          words of sampling-native-validation.json
"""
from __future__ import annotations

import json
import sys
from pathlib import Path

REV = "de4b8e4d43b917e7706784d8bb445c9af86a3540"
OUT = Path(__file__).resolve().parent


def _join(hexes: list[str]) -> str:
    return "".join(hexes)


def _f32_array(rec: dict) -> dict:
    return {"shape": rec["shape"], "le_hex": _join(rec["f32_le_hex"])}


def numeric(ref: Path) -> None:
    src = json.loads((ref / "research/numerics/Qwen3.8-Flash-Next" / REV /
                      "dequant-vectors.json").read_text())
    cases = [{"id": c["id"], "type": c["type"], "packed_hex": c["packed_hex"],
              "expected_f32_bits": c["expected_f32_bits"]} for c in src["cases"]]
    rows = [{"id": c["id"], "type": c["type"], "source_case_id": c["source_case_id"],
             "activation_f32_bits": c["activation_f32_bits"],
             "expected_f32_bits": c["expected_f32_bits"]} for c in src["row_dot_cases"]]
    doc = {"source": f"research/numerics/Qwen3.8-Flash-Next/{REV}/dequant-vectors.json",
           "oracle": src["oracle"], "type_geometry": src["type_geometry"],
           "cases": cases, "row_dot_cases": rows}
    (OUT / "numeric_vectors.json").write_text(json.dumps(doc, indent=0, sort_keys=True))


def primitives(ref: Path) -> None:
    base = ref / "research/numerics/Qwen3.8-Flash-Next" / REV
    doc = {"source": [f"research/numerics/Qwen3.8-Flash-Next/{REV}/primitive-calibration.json",
                      f"research/numerics/Qwen3.8-Flash-Next/{REV}/primitive-holdout.json"]}
    for corpus in ("calibration", "holdout"):
        src = json.loads((base / f"primitive-{corpus}.json").read_text())
        keep = ("id", "operation", "input_left_f32_bits", "input_right_f32_bits",
                "epsilon_f32_bits", "k", "expected_f32_bits", "expected_indices")
        doc[corpus] = [{k: c[k] for k in keep if k in c} for c in src["cases"]]
        doc.setdefault("contracts", {})
        for op, con in src["contracts"].items():
            doc["contracts"][op] = {"classification": con["classification"],
                                    "ulp_limit": con["acceptance"]["ulp_limit"]}
    (OUT / "primitive_vectors.json").write_text(json.dumps(doc, indent=0, sort_keys=True))


def moe(ref: Path) -> None:
    base = ref / "research/operators/Qwen3.8-Flash-Next" / REV
    contract = json.loads((base / "moe-contract.json").read_text())
    val = json.loads((base / "moe-native-validation.json").read_text())
    doc = {"source": [f"research/operators/Qwen3.8-Flash-Next/{REV}/moe-contract.json",
                      f"research/operators/Qwen3.8-Flash-Next/{REV}/moe-calibration.json",
                      f"research/operators/Qwen3.8-Flash-Next/{REV}/moe-holdout.json",
                      f"research/operators/Qwen3.8-Flash-Next/{REV}/moe-native-validation.json"],
           "tier_a_config": contract["tier_a_config"],
           "routing_contract": contract["routing_contract"],
           "weights": {k: _f32_array(v) for k, v in contract["weights"].items()},
           "contracts": {k: {"class": v["class"], "abs_limit": v["abs_limit"],
                             "rel_limit": v["rel_limit"], "ulp_limit": v["ulp_limit"]}
                         for k, v in val["contracts"].items()}}
    for corpus in ("calibration", "holdout"):
        src = json.loads((base / f"moe-{corpus}.json").read_text())
        cases = []
        for c in src["cases"]:
            exp = c["expected"]
            e2 = {}
            for k, v in exp.items():
                if k == "selected_expert_ids":
                    e2[k] = v
                elif k == "selected_experts":
                    e2[k] = [{kk: (_f32_array(vv) if isinstance(vv, dict) else vv)
                              for kk, vv in s.items()} for s in v]
                else:
                    e2[k] = _f32_array(v)
            cases.append({"id": c["id"], "input": _f32_array(c["input"]), "expected": e2})
        doc[corpus] = cases
    (OUT / "moe_tier_a.json").write_text(json.dumps(doc, indent=0, sort_keys=True))


def layer(ref: Path) -> None:
    base = ref / "research/operators/Qwen3.8-Flash-Next" / REV
    contract = json.loads((base / "layer-contract.json").read_text())
    val = json.loads((base / "layer-native-validation.json").read_text())
    doc = {"source": [f"research/operators/Qwen3.8-Flash-Next/{REV}/layer-{c}.json"
                      for c in ("contract", "calibration", "holdout", "native-validation")],
           "reduced": contract["reduced"],
           "limit_abs": max(r["limit_abs"] for r in val["records"])}
    for corpus in ("calibration", "holdout"):
        src = json.loads((base / f"layer-{corpus}.json").read_text())
        cases = []
        for c in src["cases"]:
            w = {k: _f32_array(v) for k, v in c["weights"].items()
                 if "hyper_connection" in k or k.startswith("mlp.")}
            cases.append({"id": c["id"], "family": c["family"], "input": _f32_array(c["input"]),
                          "output": _f32_array(c["output"]),
                          "checkpoints": {k: _f32_array(v) for k, v in c["checkpoints"].items()
                                          if k in ("ple_output", "attn_gr", "mixer_output",
                                                   "moe_gr", "moe_output")},
                          "weights": w})
        doc[corpus] = cases
    (OUT / "layer_tier_a.json").write_text(json.dumps(doc, indent=0, sort_keys=True))


def routing(ref: Path) -> None:
    base = ref / "research/operators/Qwen3.8-Flash-Next" / REV
    src = json.loads((base / "moe-routing-vectors.json").read_text())
    cases = []
    for c in src["cases"]:
        exp = {k: (_f32_array(v) if isinstance(v, dict) else v)
               for k, v in c["expected"].items()}
        cases.append({"id": c["id"], "input": _f32_array(c["input"]),
                      "router_weight": _f32_array(c["router_weight"]), "expected": exp})
    doc = {"source": f"research/operators/Qwen3.8-Flash-Next/{REV}/moe-routing-vectors.json",
           "config": src["config"], "comparison_class": src["comparison_class"],
           "cases": cases}
    (OUT / "moe_routing_vectors.json").write_text(json.dumps(doc, indent=0, sort_keys=True))


def sampling(ref: Path) -> None:
    base = ref / "research/sampling/Qwen3.8-Flash-Next" / REV
    cal = json.loads((base / "sampling-calibration.json").read_text())
    hold = json.loads((base / "sampling-holdout.json").read_text())
    rng = json.loads((base / "sampling-rng-vectors.json").read_text())
    val = json.loads((base / "sampling-native-validation.json").read_text())
    doc = {"source": [f"research/sampling/Qwen3.8-Flash-Next/{REV}/{n}" for n in (
               "sampling-calibration.json", "sampling-holdout.json",
               "sampling-rng-vectors.json", "sampling-native-validation.json")],
           "calibration": cal["cases"], "holdout": hold["cases"],
           "comparison": cal["comparison"],
           "rng": {k: rng[k] for k in ("algorithm", "cases", "explicit_word_boundaries",
                                       "uniform_mapping", "comparison_class")},
           "floating_contract": val["floating_contract"],
           "categorical_boundaries": val["categorical_boundaries"]}
    (OUT / "sampling_vectors.json").write_text(json.dumps(doc, indent=0, sort_keys=True))


def main() -> None:
    ref = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
    numeric(ref)
    primitives(ref)
    moe(ref)
    routing(ref)
    layer(ref)
    sampling(ref)
    for p in sorted(OUT.glob("*.json")):
        print(p.name, p.stat().st_size)


if __name__ == "__main__":
    main()
