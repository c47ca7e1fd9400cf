"""GPU parity of the checkpoint trace (row A23): det_trace_run on
tiny-gemma-dev must write the reference's golden trace artifacts
(tests/goldens/native-det-{full,terminal}.json, golden_traces.rs:224-264)
byte for byte, and stop, resume-free, at any terminal checkpoint with the
prefix of that trace.
"""
import json
import pathlib

import pytest

import fixtures

pytestmark = pytest.mark.gpu
rd = pytest.importorskip("rasterdet")

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"
PROMPT = json.loads((GOLDEN / "tiny_gemma_dev" / "trace_prompt.json").read_text())


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
    # detokenize_output_tokens (output_finalize/native/tiles.rs:5-13)
    return lambda ids: tok.decode(ids, skip_special_tokens=True)


def golden_bytes(name: str) -> bytes:
    return (GOLDEN / "traces" / f"{name}.json").read_bytes()


def entries(artifact: bytes) -> list[tuple[str, str]]:
    return [next(iter(e.items())) for e in json.loads(artifact)]


def run(model, detokenize, **kw):
    args = dict(max_new_tokens=2, temperature=1.0, detokenize=detokenize)
    args.update(kw)
    return model.trace(PROMPT["prompt_text"], PROMPT["prompt_token_ids"], **args)


def test_native_det_full_trace_is_byte_identical(model, detokenize):
    artifact, paused = run(model, detokenize)
    assert not paused
    assert artifact == golden_bytes("native-det-full")


def test_native_det_terminal_trace_is_byte_identical(model, detokenize):
    artifact, paused = run(model, detokenize, terminal_checkpoint="prefill.finalize")
    assert paused
    assert artifact == golden_bytes("native-det-terminal")


@pytest.mark.parametrize("terminal,count", [
    ("prompt.prepare", 1), ("input.embedding", 2), ("prefill.prepare_aux", 3), ("prefill.range", 4),
    ("prefill.range:3", 8), ("prefill.range_finalize:4", 11), ("decode.select_token", 13),
    ("decode.layer_range:2", 17), ("decode.transition_finalize:2", 18), ("output.finalize", 19),
    # layer_token checkpoints are never committed but still end the run
    ("prefill.layer_token.layer_1.token_4", 7), ("prefill.layer_token.layer_3.token_18", 11)])
def test_terminal_checkpoints_stop_at_the_golden_prefix(model, detokenize, terminal, count):
    full = entries(golden_bytes("native-det-full"))
    artifact, paused = run(model, detokenize, terminal_checkpoint=terminal)
    assert paused
    assert entries(artifact) == full[:count]


def test_range_widths_split_checkpoints(model, detokenize):
    # 19 prompt tokens in ranges of 5 (4 prefill.range per layer), 4 layers in
    # decode ranges of 3 (2 decode.layer_range per step); every checkpoint
    # whose payload does not depend on the widths is unchanged
    full = entries(golden_bytes("native-det-full"))
    got = entries(run(model, detokenize, prefill_token_range_width=5, decode_layer_range_width=3)[0])
    names = [n for n, _ in got]
    assert names.count("prefill.range") == 16 and names.count("decode.layer_range") == 4
    invariant = [e for e in full if e[0] not in ("prefill.range", "decode.layer_range")]
    assert [e for e in got if e[0] not in ("prefill.range", "decode.layer_range")] == invariant
    # a decode range ending at the last layer has the payload of the single
    # full range except layer_start
    assert [h for n, h in got if n == "decode.layer_range"][1] != [h for n, h in full if n == "decode.layer_range"][0]


def test_without_prompt_checkpoint_and_without_tokens(model, detokenize):
    full = entries(golden_bytes("native-det-full"))
    got = entries(run(model, detokenize, prompt_checkpoint=False)[0])
    assert got == full[1:]
    # max_new_tokens None (= 0): straight to output.finalize with no text
    got0 = entries(run(model, None, max_new_tokens=None, prompt_checkpoint=False)[0])
    assert [n for n, _ in got0] == [n for n, _ in full[1:12]] + ["output.finalize"]
    assert got0[:11] == full[1:12]


def test_unsupported_sampling_fails_after_prefill_with_partial_trace(model, detokenize):
    full = entries(golden_bytes("native-det-full"))
    with pytest.raises(rd.TraceError) as e:
        run(model, detokenize, temperature=0.7)
    assert "temperature" in str(e.value)
    got = entries(e.value.artifact)
    # prompt.prepare carries the sampling config, so only it differs
    assert [n for n, _ in got] == [n for n, _ in full[:12]]
    assert got[1:] == full[1:12] and got[0] != full[0]


# ---------------------------------------------------------------------------
# traces against the oracle's checkpoint commitments (tests/trace_builder.py
# restates the payload builders; it reproduces both golden traces on the CPU)
# ---------------------------------------------------------------------------
def id_text(ids):
    return ",".join(map(str, ids))


@pytest.mark.parametrize("pw,dw", [(5, 3), (1, 1), (7, 2)])
def test_per_op_trace_with_range_widths_matches_oracle(model, detokenize, pw, dw):
    import oracle_lib
    import trace_builder

    cfg, blob = fixtures.tiny_gemma_dev()
    om = oracle_lib.OracleModel(cfg).load_detwgt(blob).finalize()
    ids = PROMPT["prompt_token_ids"]
    cap = om.trace_capture(ids, 3, prefill_width=pw, decode_width=dw)
    gen = [s["token"] for s in cap["steps"]]
    exp = trace_builder.expected_trace(cap, PROMPT["prompt_text"], ids, 3, detokenize(gen), pw, dw)
    got, paused = run(model, detokenize, max_new_tokens=3, prefill_token_range_width=pw, decode_layer_range_width=dw)
    assert not paused
    assert entries(got) == exp


@pytest.fixture(scope="module")
def e4b_two_layer():
    import oracle_lib
    from rasterdet import synthetic

    c = rd.Context(0)
    cfg = synthetic.e4b_config(layers=2, vocab=4096, sliding_window=8)
    om, gm = fixtures.load_both(cfg, synthetic.synthetic_model_fast(cfg, seed=31, scale_max=256), c,
                                threads=oracle_lib.cpu_count())
    yield om, gm
    del om, gm
    c.close()


@pytest.mark.parametrize("pw,dw", [(0, 0), (4, 1), (7, 2)])
def test_fused_decode_trace_matches_oracle(e4b_two_layer, pw, dw):
    # the fused, graph-captured step with every layer's output row captured and
    # the KV commitments hashed on the host pool from the append-only mirror
    import trace_builder

    om, gm = e4b_two_layer
    ids = list(range(40, 61))  # 21 tokens: the sliding ring (window 8) wraps
    steps = 6
    cap = om.trace_capture(ids, steps, prefill_width=pw, decode_width=dw)
    gen = [s["token"] for s in cap["steps"]]
    exp = trace_builder.expected_trace(cap, "e4b two-layer prompt", ids, steps, id_text(gen), pw, dw)
    got, paused = gm.trace("e4b two-layer prompt", ids, max_new_tokens=steps, detokenize=id_text,
                           prefill_token_range_width=pw, decode_layer_range_width=dw)
    assert not paused
    assert entries(got) == exp
