"""CPU pins of the checkpoint trace layer (row A23).

The reference's golden traces (tests/goldens/native-det-{full,terminal}.json,
copied to tests/golden/traces/) hold one SHA-256 per checkpoint payload. Here
the payloads are rebuilt in Python from the oracle's commitments, following
the reference's payload builders, and each digest is compared with the
golden entry. This pins the prompt ids, the JSON conventions (compact, keys
ordered, f32 formatting) and the position/count semantics that the GPU
trace driver (det_trace_run) must reproduce byte for byte.
"""
import hashlib
import json
import pathlib

import pytest

import fixtures
import oracle_lib

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"
PROMPT = json.loads((GOLDEN / "tiny_gemma_dev" / "trace_prompt.json").read_text())


def compact(v) -> str:
    # serde_json::to_vec of a json! map: no whitespace, keys in byte order
    return json.dumps(v, separators=(",", ":"), sort_keys=True, ensure_ascii=False)


def digest(v) -> str:
    return hashlib.sha256(compact(v).encode()).hexdigest()


def golden(name: str) -> list[tuple[str, str]]:
    return [next(iter(e.items())) for e in json.loads((GOLDEN / "traces" / f"{name}.json").read_text())]


def test_token_id_commitments_match_reference_known_answers():
    # build_prompt_commitment / build_output_decode_commitment tests
    # (prompt_prepare/native/tests.rs:47-54, output_finalize/native/tests.rs:13-19)
    assert digest([1, 2, 3]) == "a615eeaee21de5179de080de8c3052c8da901138406ba71c38c032845f7d54f4"
    assert digest([4, 5]) == "d4c7a98da55490b0a5a65cc5057db99aa708a436609b177748505342d569457b"


def test_prompt_fixture_matches_tokenizer():
    tokenizers = pytest.importorskip("tokenizers")
    tok = tokenizers.Tokenizer.from_file(str(GOLDEN / "tiny_gemma_dev" / "tokenizer.json"))
    assert tok.encode(PROMPT["prompt_text"], add_special_tokens=True).ids == PROMPT["prompt_token_ids"]


def test_prompt_prepare_entry():
    ids = PROMPT["prompt_token_ids"]
    payload = {"prompt_text": PROMPT["prompt_text"], "prompt_token_ids": ids, "prompt_token_ids_sha256": digest(ids),
               "sampling": {"max_new_tokens": 2, "temperature": 1.0, "top_k": None, "top_p": None}}
    assert golden("native-det-full")[0] == ("prompt.prepare", digest(payload))
    assert golden("native-det-terminal")[0] == ("prompt.prepare", digest(payload))


def test_oracle_commitments_reproduce_golden_entries():
    cfg, blob = fixtures.tiny_gemma_dev()
    om = oracle_lib.OracleModel(cfg).load_detwgt(blob).finalize()
    ids = PROMPT["prompt_token_ids"]
    n = len(ids)
    cap = om.capture(ids, 2)
    pre, steps = cap["prefill"], cap["decode_steps"]
    g = dict()
    for i, (name, h) in enumerate(golden("native-det-full")):
        g.setdefault(name, []).append((i, h))
    emb = {"det_embedded_prompt_activations_sha256": pre["embedding"], "prompt_token_ids": ids,
           "prompt_token_ids_sha256": digest(ids)}
    assert digest(dict(emb, raster=None)) == g["input.embedding"][0][1]
    assert digest(emb) == g["prefill.prepare_aux"][0][1]
    assert digest({"det_final_hidden_states_sha256": pre["final_hidden"], "det_prefill_logits_sha256": pre["logits"],
                   "decode_position": n, "decode_token_count": n,
                   "det_layer_caches_sha256": pre["kv"]}) == g["prefill.finalize"][0][1]
    # the first decode step: select at (n, n), layer range over all layers at
    # (n, n), transition to (n + 1, n + 1)
    t1 = steps[0]["token"]
    full, gen = ids + [t1], [t1]
    tok_fields = {"full_token_ids": full, "full_token_ids_sha256": digest(full), "generated_token_ids": gen,
                  "generated_token_ids_sha256": digest(gen)}
    assert digest(dict(tok_fields, det_current_logits_sha256=pre["logits"], selected_next_token=t1,
                       decode_position=n, decode_token_count=n, max_new_tokens=2)) == g["decode.select_token"][0][1]
    assert digest({"next_token": t1, "decode_position": n, "decode_token_count": n, "layer_start": 0, "layer_end": 4,
                   "layer_count": 4, "det_current_activation_sha256": steps[0]["activation"],
                   "det_layer_caches_sha256": steps[0]["kv"], "execution_mode": "deterministic",
                   "completed_layer_output_det_sha256s": [e["layer_output"] for e in cap["first_step_layers"]]}) \
        == g["decode.layer_range"][0][1]
    assert digest(dict(tok_fields, det_current_logits_sha256=steps[0]["logits"], decode_position=n + 1,
                       decode_token_count=n + 1)) == g["decode.transition_finalize"][0][1]
    # output.finalize: both generated ids are <bos>, decoded with special
    # tokens skipped to the empty string
    t2 = steps[1]["token"]
    full2, gen2 = full + [t2], [t1, t2]
    assert (t1, t2) == (1, 1)
    assert digest({"full_token_ids": full2, "full_token_ids_sha256": digest(full2), "generated_token_ids": gen2,
                   "generated_token_ids_sha256": digest(gen2), "generated_text": "", "generated_token_count": 2,
                   "stop_reason": "max_new_tokens"}) == g["output.finalize"][0][1]


def test_trace_builder_over_oracle_reproduces_both_golden_traces():
    # every entry of native-det-full.json (and its terminal prefix) from the
    # restated payload builders over the oracle's checkpoint commitments
    import trace_builder

    cfg, blob = fixtures.tiny_gemma_dev()
    om = oracle_lib.OracleModel(cfg).load_detwgt(blob).finalize()
    ids = PROMPT["prompt_token_ids"]
    cap = om.trace_capture(ids, 2)
    # both generated ids are <bos>, which decodes (special tokens skipped) to ""
    exp = trace_builder.expected_trace(cap, PROMPT["prompt_text"], ids, 2, "")
    assert exp == golden("native-det-full")
    assert exp[:12] == golden("native-det-terminal")


def test_trace_capture_range_widths_agree_with_the_single_range():
    import trace_builder

    cfg, blob = fixtures.tiny_gemma_dev()
    om = oracle_lib.OracleModel(cfg).load_detwgt(blob).finalize()
    ids = PROMPT["prompt_token_ids"]
    whole = om.trace_capture(ids, 2)
    split = om.trace_capture(ids, 2, prefill_width=5, decode_width=3)
    assert [len(l["ranges"]) for l in split["prefill"]["layers"]] == [4] * 4
    for a, b in zip(whole["prefill"]["layers"], split["prefill"]["layers"]):
        assert (a["output"], a["kv"]) == (b["output"], b["kv"])
    # the effective caches after the last layer are the fully updated caches
    assert whole["steps"][0]["layers"][-1]["kv"] == split["steps"][0]["layers"][-1]["kv"]
    assert "kv" in split["steps"][0]["layers"][2] and "kv" not in split["steps"][0]["layers"][1]
    names = [n for n, _ in trace_builder.expected_trace(split, PROMPT["prompt_text"], ids, 2, "", 5, 3)]
    assert names.count("prefill.range") == 16 and names.count("decode.layer_range") == 4
