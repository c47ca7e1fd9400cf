"""Claimer/challenger roles on the GPU executor (runtime/roles/{claimer,
challenger}.rs), after the reference's tests/challenger_audit.rs: the claimer
trace is the native golden byte for byte (:252-270), an audit of an honest
claim finds no divergence (:272-280), a commitment tampered at
checkpoint:occurrence is located exactly with that routine occurrence as the
raster detour spec (:208-248, 282-350), prompt.prepare has no detour
(:352-372) and a truncated claim is a structural divergence (:376-403).
The replay runs det_trace_run's sequence on the GPU; the raster detour run
itself is not part of this executor, so the detour is checked as its spec.
"""
import json
import pathlib

import pytest

import fixtures

pytestmark = pytest.mark.gpu
rd = pytest.importorskip("rasterdet")

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"
PROMPT = json.loads((GOLDEN / "tiny_gemma_dev" / "trace_prompt.json").read_text())
FULL = (GOLDEN / "traces" / "native-det-full.json").read_bytes()


@pytest.fixture(scope="module")
def model():
    c = rd.Context(0)
    cfg, blob = fixtures.tiny_gemma_dev()
    m = rd.Model(c, cfg).load_detwgt(blob).finalize()
    yield m
    c.close()


@pytest.fixture(scope="module")
def detokenize():
    tokenizers = pytest.importorskip("tokenizers")
    tok = tokenizers.Tokenizer.from_file(str(GOLDEN / "tiny_gemma_dev" / "tokenizer.json"))
    return lambda ids: tok.decode(ids, skip_special_tokens=True)


def audit(model, detokenize, claimed: bytes, **kw):
    args = dict(max_new_tokens=2, temperature=1.0, detokenize=detokenize)
    args.update(kw)
    return model.audit(PROMPT["prompt_text"], PROMPT["prompt_token_ids"], claimed, **args)


def entries(artifact: bytes):
    return [next(iter(e.items())) for e in json.loads(artifact)]


def pretty(es) -> bytes:
    return json.dumps([{k: v} for k, v in es], indent=2).encode()


def tamper(artifact: bytes, checkpoint_id: str, occurrence: int) -> bytes:
    es, seen = entries(artifact), 0
    for i, (k, _) in enumerate(es):
        if k == checkpoint_id:
            seen += 1
            if seen == occurrence:
                es[i] = (k, "0" * 64)
                return pretty(es)
    raise AssertionError(f"no occurrence {occurrence} of {checkpoint_id}")


def test_claimer_trace_matches_the_native_golden(model, detokenize):
    claim = model.claim(PROMPT["prompt_text"], PROMPT["prompt_token_ids"], max_new_tokens=2, detokenize=detokenize)
    assert claim == FULL


def test_audit_of_an_honest_claim_reports_no_divergence(model, detokenize):
    assert audit(model, detokenize, FULL) == rd.AuditOutcome()


@pytest.mark.parametrize("checkpoint,occurrence,spec", [
    ("prefill.range", 1, "prefill.range"),
    ("prefill.range", 2, "prefill.range:2"),
    ("input.embedding", 1, "input.embedding"),
    ("prefill.finalize", 1, "prefill.finalize"),
    ("decode.select_token", 1, "decode.select_token"),
    ("decode.transition_finalize", 1, "decode.transition_finalize"),
    ("output.finalize", 1, "output.finalize"),
])
def test_audit_locates_a_tampered_commitment(model, detokenize, checkpoint, occurrence, spec):
    out = audit(model, detokenize, tamper(FULL, checkpoint, occurrence))
    d = out.divergence
    assert (d.checkpoint_id, d.occurrence) == (checkpoint, occurrence)
    assert d.claimed_checkpoint_id is None
    assert d.replayed_commitment == entries(FULL)[d.entry_index][1]
    assert out.detour == spec


def test_audit_reports_a_tampered_prompt_prepare_without_detour(model, detokenize):
    out = audit(model, detokenize, tamper(FULL, "prompt.prepare", 1))
    assert (out.divergence.checkpoint_id, out.divergence.occurrence) == ("prompt.prepare", 1)
    assert out.detour is None


def test_audit_reports_a_truncated_claim_as_structural(model, detokenize):
    es = entries(FULL)
    out = audit(model, detokenize, pretty(es[:-1]))
    d = out.divergence
    assert (d.entry_index, d.checkpoint_id) == (len(es) - 1, es[-1][0])
    assert d.claimed_commitment is None and d.replayed_commitment == es[-1][1]
    assert out.detour is None


def test_a_claim_for_another_request_diverges_at_the_prompt(model, detokenize):
    # the claim of a 1-token run against a 2-token replay: prompt.prepare
    # commits the sampling config, so the first entry differs
    other = model.claim(PROMPT["prompt_text"], PROMPT["prompt_token_ids"], max_new_tokens=1, detokenize=detokenize)
    out = audit(model, detokenize, other)
    assert (out.divergence.entry_index, out.divergence.checkpoint_id, out.detour) == (0, "prompt.prepare", None)
    # and a claim of the GPU's own run of that request is honest
    assert not audit(model, detokenize, other, max_new_tokens=1).diverged


def test_audit_errors(model, detokenize):
    with pytest.raises(rd.DetError, match="not valid JSON"):
        audit(model, detokenize, b"[{")
    # the replay must complete: unsupported sampling fails after prefill
    with pytest.raises(rd.DetError, match="temperature"):
        audit(model, detokenize, FULL, temperature=0.7)
