"""Claimer/challenger trace comparison on the CPU, through the C ABI
(det_trace_locate_divergence, host code only).

The cases follow the reference's role tests (tests/challenger_audit.rs):
an honest trace has no divergence; a commitment tampered at
checkpoint:occurrence is located exactly, with the --raster-at spec of that
routine occurrence as the detour (challenger_audit.rs:208-248); prompt.prepare
has no detour (:352-372); a truncated trace is a structural divergence at its
first missing entry with no detour (:376-403). The traces are the reference's
golden artifacts (tests/goldens/native-det-full.json).
"""
import json
import pathlib

import pytest

rd = pytest.importorskip("rasterdet")

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden" / "traces"
FULL = (GOLDEN / "native-det-full.json").read_bytes()
ENTRIES = [next(iter(e.items())) for e in json.loads(FULL)]


def pretty(entries) -> bytes:
    # serde_json::to_vec_pretty of the array of single-entry maps
    return json.dumps([{k: v} for k, v in entries], indent=2).encode()


def tamper(entries, checkpoint_id: str, occurrence: int):
    # tamper_commitment (challenger_audit.rs:181-206)
    out, seen = list(entries), 0
    for i, (k, _) in enumerate(out):
        if k == checkpoint_id:
            seen += 1
            if seen == occurrence:
                out[i] = (k, "0" * 64)
                return out
    raise AssertionError(f"no occurrence {occurrence} of {checkpoint_id}")


def test_pretty_rewrite_of_the_golden_is_byte_identical():
    # the test's writer is the artifact writer, so tampered traces differ
    # from honest ones only in the tampered commitment
    assert pretty(ENTRIES) == FULL


def test_honest_trace_has_no_divergence():
    out = rd.locate_divergence(FULL, FULL)
    assert out == rd.AuditOutcome() and not out.diverged
    # whitespace does not matter, only the parsed entries
    compact = json.dumps([{k: v} for k, v in ENTRIES], separators=(",", ":")).encode()
    assert not rd.locate_divergence(compact, FULL).diverged


@pytest.mark.parametrize("checkpoint,occurrence,detour", [
    ("input.embedding", 1, "input.embedding"),
    ("prefill.prepare_aux", 1, "prefill.prepare_aux"),
    ("prefill.range", 1, "prefill.range"),
    ("prefill.range", 2, "prefill.range:2"),
    ("prefill.range", 4, "prefill.range:4"),
    ("prefill.finalize", 1, "prefill.finalize"),
    ("decode.select_token", 1, "decode.select_token"),
    ("decode.select_token", 2, "decode.select_token:2"),
    ("decode.layer_range", 2, "decode.layer_range:2"),
    ("decode.transition_finalize", 1, "decode.transition_finalize"),
    ("output.finalize", 1, "output.finalize"),
    # routines without a raster detour (DETOURABLE_ROUTINES, challenger.rs:28-37)
    ("prompt.prepare", 1, None),
    ("prefill.range_finalize", 3, None),
])
def test_tampered_commitment_is_located_exactly(checkpoint, occurrence, detour):
    claimed = tamper(ENTRIES, checkpoint, occurrence)
    out = rd.locate_divergence(pretty(claimed), FULL)
    d = out.divergence
    idx = next(i for i, (a, b) in enumerate(zip(claimed, ENTRIES)) if a != b)
    assert (d.checkpoint_id, d.occurrence, d.entry_index) == (checkpoint, occurrence, idx)
    assert d.claimed_checkpoint_id is None
    assert d.claimed_commitment == "0" * 64 and d.replayed_commitment == ENTRIES[idx][1]
    assert out.detour == detour


def test_truncated_trace_is_a_structural_divergence():
    claimed = ENTRIES[:-1]
    d = rd.locate_divergence(pretty(claimed), FULL)
    assert d.divergence == rd.CheckpointDivergence(len(claimed), ENTRIES[-1][0], 1, None, None, ENTRIES[-1][1])
    assert d.detour is None
    # an empty claim diverges at its first entry
    e = rd.locate_divergence(b"[]", FULL).divergence
    assert (e.entry_index, e.checkpoint_id, e.claimed_commitment) == (0, "prompt.prepare", None)


def test_extra_claimed_entry_is_a_structural_divergence():
    extra = ("decode.select_token", "ab" * 32)
    d = rd.locate_divergence(pretty(ENTRIES + [extra]), FULL)
    # the claimed trace's 3rd decode.select_token
    assert d.divergence == rd.CheckpointDivergence(len(ENTRIES), extra[0], 3, None, extra[1], None)
    assert d.detour is None


def test_checkpoint_id_sequence_divergence_has_no_detour():
    swapped = list(ENTRIES)
    swapped[1], swapped[2] = swapped[2], swapped[1]
    d = rd.locate_divergence(pretty(swapped), FULL)
    assert d.divergence == rd.CheckpointDivergence(1, ENTRIES[1][0], 1, ENTRIES[2][0], ENTRIES[2][1],
                                                   ENTRIES[1][1])
    assert d.detour is None


def test_occurrence_counts_per_checkpoint_id():
    # the 2nd decode.layer_range entry is the 17th entry of the golden trace
    idx = [i for i, (k, _) in enumerate(ENTRIES) if k == "decode.layer_range"][1]
    d = rd.locate_divergence(pretty(tamper(ENTRIES, "decode.layer_range", 2)), FULL).divergence
    assert d.entry_index == idx == 16


def test_escaped_and_repeated_keys_follow_json_semantics():
    # "\u0070" is "p"; of repeated keys the last one counts (as in a JSON map)
    body = FULL.decode().replace('"prompt.prepare"', '"\\u0070rompt.prepare"', 1)
    assert not rd.locate_divergence(body.encode(), FULL).diverged
    first_key, first_val = ENTRIES[0]
    dup = FULL.decode().replace(f'"{first_key}": "{first_val}"',
                                f'"{first_key}": "{"1" * 64}", "{first_key}": "{first_val}"', 1)
    assert json.loads(dup) == json.loads(FULL)
    assert not rd.locate_divergence(dup.encode(), FULL).diverged


@pytest.mark.parametrize("claimed,needle", [
    (b"", "not valid JSON"),
    (b"[", "not valid JSON"),
    (b"[] x", "trailing characters"),
    (b"[{\"a\": \"b\",}]", "not valid JSON"),
    (b"[01]", "not valid JSON"),
    (b"[\"\\ud800\"]", "lone leading surrogate"),
    (b"[\"\\udc00\"]", "lone trailing surrogate"),
    (b"[\"\xc3\x28\"]", "invalid UTF-8"),
    (b"[\"\xed\xa0\x80\"]", "invalid UTF-8"),
    (b"[\"a\nb\"]", "control character"),
    (b"[" * 200 + b"]" * 200, "recursion limit"),
    (b"{\"prompt.prepare\": \"x\"}", "should be a JSON array"),
    (b"[[\"prompt.prepare\"]]", "entry 0 should be an object"),
    (b"[{}]", "entry 0 should contain exactly one commitment"),
    (b"[{\"a\": \"x\", \"b\": \"y\"}]", "entry 0 should contain exactly one commitment"),
    (b"[{\"a\": \"x\"}, {\"a\": 5}]", "entry 1 commitment should be a string"),
])
def test_malformed_claimed_traces_are_refused(claimed, needle):
    with pytest.raises(rd.DetError) as e:
        rd.locate_divergence(claimed, FULL)
    assert needle in str(e.value)


def test_json_value_forms_parse_before_the_shape_check():
    # every JSON value form is read; the shape check then refuses it
    for v in (b"true", b"false", b"null", b"-1.5e+3", b"0", b"[1, {}]", b"{\"k\": []}"):
        with pytest.raises(rd.DetError) as e:
            rd.locate_divergence(b"[{\"a\": \"x\"}, {\"a\": " + v + b"}]", FULL)
        assert "entry 1 commitment should be a string" in str(e.value)
    # nesting below the limit is fine
    ok = b"[{\"a\": \"x\", \"b\": " + b"[" * 120 + b"]" * 120 + b"}]"
    with pytest.raises(rd.DetError) as e:
        rd.locate_divergence(ok, FULL)
    assert "exactly one commitment" in str(e.value)


def test_string_escapes_decode_as_json_does():
    # the claimed strings come back in the outcome as decoded text
    raw = b"\"s\\/\\b\\f\\n\\r\\t\\\\\\\"\\u00e9\\ud83d\\ude00\xc3\xa9\""
    d = rd.locate_divergence(b"[{" + raw + b": " + raw + b"}]", FULL).divergence
    assert d.claimed_checkpoint_id == d.claimed_commitment == json.loads(raw)
    assert (d.entry_index, d.checkpoint_id) == (0, "prompt.prepare")
