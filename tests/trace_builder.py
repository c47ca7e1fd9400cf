"""Expected checkpoint traces built from the oracle's commitments (test
infrastructure).

The native deterministic sequence (src/runtime/sequence.rs,
src/runtime/executors/native.rs:60-450) commits one SHA-256 per checkpoint
over the compact serde_json of its payload, keys in byte order
(src/runtime/trace.rs:262-288, 425-430). The payload builders restated here
are those of:

* prompt.prepare            routines/prompt_prepare (executors/native.rs:68-90)
* input.embedding           routines/input_embedding/mod.rs:88-130
* prefill.prepare_aux       routines/prefill_prepare_aux/mod.rs:175-210
* prefill.range             routines/prefill_range/mod.rs:25-88
* prefill.range_finalize    routines/prefill_range_finalize/mod.rs:17-73
* prefill.finalize          routines/prefill_finalize/native/tiles.rs:68-94
* decode.select_token       routines/decode_select_token/mod.rs:19-47, 362-390
* decode.layer_range        routines/decode_layer_range/mod.rs:553-664
* decode.transition_finalize routines/decode_transition_finalize/mod.rs:67-99
* output.finalize           routines/output_finalize/mod.rs:18-52

The commitments come from oracle_lib.OracleModel.trace_capture.
"""
from __future__ import annotations

import hashlib
import json


def compact(v) -> str:
    # serde_json::to_vec of a json! map: no whitespace, keys in byte order
    return json.dumps(v, separators=(",", ":"), sort_keys=True, ensure_ascii=False)


def digest(v) -> str:
    return hashlib.sha256(compact(v).encode()).hexdigest()


def ranges(n: int, width: int):
    w = min(max(width or n, 1), max(n, 1))
    return [(a, min(n, a + w)) for a in range(0, n, w)]


def expected_trace(cap: dict, prompt_text: str, ids: list[int], max_new_tokens, generated_text: str,
                   prefill_width: int = 0, decode_width: int = 0, prompt_checkpoint: bool = True):
    """[(checkpoint, sha256 of its payload)] of a full greedy run."""
    out = []
    n = len(ids)
    max_new = max_new_tokens or 0
    ids_sha = digest(ids)
    if prompt_checkpoint:
        out.append(("prompt.prepare", digest({"prompt_text": prompt_text, "prompt_token_ids": ids,
                                              "prompt_token_ids_sha256": ids_sha,
                                              "sampling": {"max_new_tokens": max_new_tokens, "temperature": 1.0,
                                                           "top_k": None, "top_p": None}})))
    pre = cap["prefill"]
    emb = {"det_embedded_prompt_activations_sha256": pre["embedding"], "prompt_token_ids": ids,
           "prompt_token_ids_sha256": ids_sha}
    out.append(("input.embedding", digest(dict(emb, raster=None))))
    out.append(("prefill.prepare_aux", digest(emb)))
    outputs = []
    for l, layer in enumerate(pre["layers"]):
        outputs.append(layer["output"])
        for (a, b), rc in zip(ranges(n, prefill_width), layer["ranges"]):
            out.append(("prefill.range", digest({"det_range_activations_sha256": rc, "execution_mode": "deterministic",
                                                 "layer_idx": l, "range_end": b, "range_start": a,
                                                 "token_count": n})))
        out.append(("prefill.range_finalize", digest({
            "completed_layer_output_det_sha256s": list(outputs), "det_current_activations_sha256": layer["output"],
            "det_layer_caches_sha256": layer["kv"], "execution_mode": "deterministic", "next_layer_idx": l + 1})))
    out.append(("prefill.finalize", digest({"decode_position": n, "decode_token_count": n,
                                            "det_final_hidden_states_sha256": pre["final_hidden"],
                                            "det_layer_caches_sha256": pre["kv"],
                                            "det_prefill_logits_sha256": pre["logits"]})))
    full, gen = list(ids), []
    logits = pre["logits"]
    layer_count = len(pre["layers"])
    for i, step in enumerate(cap["steps"][:max_new]):
        pos, t = n + i, step["token"]
        full, gen = full + [t], gen + [t]
        tok = {"full_token_ids": full, "full_token_ids_sha256": digest(full), "generated_token_ids": gen,
               "generated_token_ids_sha256": digest(gen)}
        out.append(("decode.select_token", digest(dict(tok, decode_position=pos, decode_token_count=pos,
                                                       det_current_logits_sha256=logits, max_new_tokens=max_new,
                                                       selected_next_token=t))))
        outs = [e["output"] for e in step["layers"]]
        for a, b in ranges(layer_count, decode_width):
            out.append(("decode.layer_range", digest({
                "completed_layer_output_det_sha256s": outs[:b], "decode_position": pos, "decode_token_count": pos,
                "det_current_activation_sha256": outs[b - 1], "det_layer_caches_sha256": step["layers"][b - 1]["kv"],
                "execution_mode": "deterministic", "layer_count": layer_count, "layer_end": b, "layer_start": a,
                "next_token": t})))
        logits = step["logits"]
        out.append(("decode.transition_finalize", digest(dict(tok, decode_position=pos + 1,
                                                              decode_token_count=pos + 1,
                                                              det_current_logits_sha256=logits))))
    out.append(("output.finalize", digest({"full_token_ids": full, "full_token_ids_sha256": digest(full),
                                           "generated_text": generated_text, "generated_token_count": len(gen),
                                           "generated_token_ids": gen, "generated_token_ids_sha256": digest(gen),
                                           "stop_reason": "max_new_tokens"})))
    return out
