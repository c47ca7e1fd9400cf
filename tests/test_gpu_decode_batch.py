"""GPU parity of batched decode over ragged sequences.

det_session_decode_batch runs one decode step for n independent sessions in
shared launches (projections over M = n activation rows, attention over each
session's own cache window). The requirement is that every session's per-step
results (next token, activation / logits / KV commitments) equal its solo
decode on an identical session, whose commitments are themselves pinned to
the oracle in test_gpu_decode_fused.py and test_gpu_parity.py.
"""
import numpy as np
import pytest

import fixtures

pytestmark = pytest.mark.gpu
rd = pytest.importorskip("rasterdet")
from rasterdet import synthetic  # noqa: E402


@pytest.fixture(scope="module")
def ctx():
    c = rd.Context(0)
    yield c
    c.close()


def build(ctx, cfg, tensors):
    gm = rd.Model(ctx, cfg)
    for name, v, s in tensors:
        gm.set_tensor(name, v, s)
    return gm.finalize()


def key(r):
    return (r.activation, r.logits, r.kv, r.next_token)


def ragged_prompts(n, lo, hi, vocab, seed):
    rng = np.random.default_rng(seed)
    lens = rng.integers(lo, hi + 1, size=n)
    return [rng.integers(0, vocab, size=int(k)).tolist() for k in lens]


def run_batch_vs_solo(gm, vocab, prompts, steps, max_tokens, flags=rd.DET_COMMIT_ALL, solo_flags=0, live=None):
    """Prefills each prompt twice, then decodes one copy per sequence in
    batches and the other alone; live(step) selects the batch members."""
    batch = [gm.session(max_tokens) for _ in prompts]
    solo = [gm.session(max_tokens) for _ in prompts]
    tok_b = [s.prefill(p).next_token for s, p in zip(batch, prompts)]
    tok_s = [s.prefill(p).next_token for s, p in zip(solo, prompts)]
    assert tok_b == tok_s
    for step in range(steps):
        members = live(step) if live else list(range(len(prompts)))
        res = rd.decode_batch([batch[i] for i in members], [tok_b[i] for i in members], flags)
        for i, r in zip(members, res):
            e = solo[i].decode(tok_s[i], flags | solo_flags)
            assert key(r) == key(e), (step, i)
            tok_b[i], tok_s[i] = r.next_token, e.next_token
    for b, s in zip(batch, solo):
        assert b.position() == s.position()
        assert np.array_equal(b.logits(vocab), s.logits(vocab))


def sharing_model(ctx):
    """KV-sharing donors, k_eq_v full layers, sliding rings, softcap, layer scalars."""
    cfg = {"text_config": {
        "enable_moe_block": False, "head_dim": 64, "hidden_activation": "gelu_pytorch_tanh", "hidden_size": 256,
        "intermediate_size": 512, "layer_types": ["sliding_attention", "full_attention", "sliding_attention",
                                                  "full_attention"],
        "num_attention_heads": 4, "num_hidden_layers": 4, "num_key_value_heads": 2, "num_global_key_value_heads": 1,
        "attention_k_eq_v": True, "num_kv_shared_layers": 2, "final_logit_softcapping": 30.0,
        "rope_parameters": {"full_attention": {"partial_rotary_factor": 0.5, "rope_theta": 5000.0},
                            "sliding_attention": {"rope_theta": 10000.0}},
        "rms_norm_eps": 1e-6, "sliding_window": 5, "tie_word_embeddings": False, "vocab_size": 1000,
    }}
    tc = cfg["text_config"]
    tensors = []
    for name, v, s in fixtures.custom_model(cfg, seed=3, layer_scalars=True):
        if (".self_attn.k_proj" in name or ".self_attn.v_proj" in name) and \
                tc["layer_types"][int(name.split(".layers.")[1].split(".")[0])] == "full_attention":
            v, s = v[:64], s[:64]
        tensors.append((name, v, s))
    return build(ctx, cfg, tensors)


def test_tiny_gemma_dev_batch_matches_solo(ctx):
    cfg, blob = fixtures.tiny_gemma_dev()
    gm = rd.Model(ctx, cfg).load_detwgt(blob).finalize()
    vocab = cfg["text_config"]["vocab_size"]
    prompts = ragged_prompts(6, 1, 12, vocab, seed=1)
    run_batch_vs_solo(gm, vocab, prompts, steps=5, max_tokens=32)


MODES = {"graph": 0, "eager": rd.DET_DECODE_EAGER, "per_op": rd.DET_DECODE_PER_OP}


@pytest.mark.parametrize("mode", list(MODES))
@pytest.mark.parametrize("n", [1, 3, 5, 8, 16, 19])
def test_sharing_model_batch_matches_solo(ctx, n, mode):
    # fused step: GEMVs with 1, 2 or 4 token groups (19 = one pass of 16 + one
    # of 3); per-op step: n >= 16 takes the slab GEMM, fewer rows the GEMV
    gm = sharing_model(ctx)
    prompts = ragged_prompts(n, 1, 14, 1000, seed=n)
    run_batch_vs_solo(gm, 1000, prompts, steps=4, max_tokens=24, flags=rd.DET_COMMIT_ALL | MODES[mode],
                      solo_flags=rd.DET_DECODE_PER_OP)


def test_batch_with_longer_session_joining_later(ctx):
    # a session with a larger cache joins: the batched attention grids grow and
    # the captured step is rebuilt; windows wrap the rings of sliding layers
    gm = sharing_model(ctx)
    caps = [24, 24, 300, 24]
    prompts = ragged_prompts(4, 3, 20, 1000, seed=21)
    prompts[2] = ragged_prompts(1, 260, 260, 1000, seed=22)[0]
    batch = [gm.session(c) for c in caps]
    solo = [gm.session(c) for c in caps]
    tb = [s.prefill(p).next_token for s, p in zip(batch, prompts)]
    ts = [s.prefill(p).next_token for s, p in zip(solo, prompts)]
    for step in range(5):
        members = [0, 1, 3] if step < 2 else [0, 1, 2, 3]
        res = rd.decode_batch([batch[i] for i in members], [tb[i] for i in members])
        for i, r in zip(members, res):
            e = solo[i].decode(ts[i])
            assert key(r) == key(e), (step, i)
            tb[i], ts[i] = r.next_token, e.next_token


def test_batch_matches_fused_solo_with_changing_membership(ctx):
    # sequences join and leave the batch; the solo side uses the fused graph step
    gm = sharing_model(ctx)
    prompts = ragged_prompts(7, 2, 16, 1000, seed=9)
    live = lambda step: [i for i in range(7) if (i + step) % 3 != 0]  # noqa: E731
    run_batch_vs_solo(gm, 1000, prompts, steps=6, max_tokens=32, live=live)


@pytest.mark.parametrize("mode", ["graph", "per_op"])
def test_e4b_shaped_layers_batch_of_16_matches_solo(ctx, mode):
    cfg = synthetic.e4b_config(layers=2, vocab=4096, sliding_window=8)
    gm = build(ctx, cfg, synthetic.synthetic_model_fast(cfg, seed=7))
    prompts = ragged_prompts(16, 1, 40, 4096, seed=5)
    run_batch_vs_solo(gm, 4096, prompts, steps=3, max_tokens=48, flags=rd.DET_COMMIT_ALL | MODES[mode])


@pytest.mark.parametrize("hidden,ff", [(1536, 6144), (2048, 8192)])
@pytest.mark.parametrize("n", [6, 16])
def test_other_widths_batch_matches_solo(ctx, hidden, ff, n):
    """Widths whose batched GEMVs take 3 and 4 half-steps per wave: K 1536 /
    2048 for q/k/v, gate/up and the vocabulary projection, 6144 / 8192 for
    down (12 and 16 K chunks)."""
    cfg = synthetic.e4b_config(layers=2, vocab=8192, sliding_window=8)
    cfg["text_config"].update({"hidden_size": hidden, "intermediate_size": ff})
    gm = build(ctx, cfg, synthetic.synthetic_model_fast(cfg, seed=hidden + n))
    prompts = ragged_prompts(n, 1, 40, 8192, seed=hidden // 64 + n)
    run_batch_vs_solo(gm, 8192, prompts, steps=3, max_tokens=48, flags=rd.DET_COMMIT_ALL)


@pytest.mark.parametrize("n", [5, 7, 13, 19, 21])
def test_e4b_shaped_layers_partial_batches_match_solo(ctx, n):
    """Batches of 5-8 tokens take the two-token-group GEMV instances and
    13 tokens a partly filled last group (E4B widths: K of 2048-10240); 19
    and 21 tokens run a second pass of 3 (single-group kernels on the limb
    planes) or 5 tokens (the operand-major copy at its second-pass offset)."""
    cfg = synthetic.e4b_config(layers=2, vocab=4096, sliding_window=8)
    gm = build(ctx, cfg, synthetic.synthetic_model_fast(cfg, seed=11))
    prompts = ragged_prompts(n, 1, 40, 4096, seed=n)
    run_batch_vs_solo(gm, 4096, prompts, steps=3, max_tokens=48, flags=rd.DET_COMMIT_ALL)


def test_batch_rejects_bad_inputs_without_touching_state(ctx):
    gm = sharing_model(ctx)
    a, b, full = gm.session(8), gm.session(8), gm.session(4)
    ta = a.prefill([1, 2, 3]).next_token
    tb = b.prefill([4, 5]).next_token
    tf = full.prefill([6, 7, 8, 9]).next_token
    with pytest.raises(rd.DetError):
        rd.decode_batch([a, a], [ta, ta])
    with pytest.raises(rd.DetError):
        rd.decode_batch([a, full], [ta, tf])  # full is at capacity
    with pytest.raises(rd.DetError):
        rd.decode_batch([a, b], [ta, 5000])  # token out of range
    fresh = gm.session(8)
    with pytest.raises(rd.DetError):
        rd.decode_batch([a, fresh], [ta, 1])  # not prefilled
    assert (a.position(), b.position(), full.position()) == (3, 2, 4)
    # the failed calls left both sessions as they were
    ref_a, ref_b = gm.session(8), gm.session(8)
    ref_a.prefill([1, 2, 3])
    ref_b.prefill([4, 5])
    got = rd.decode_batch([a, b], [ta, tb])
    assert key(got[0]) == key(ref_a.decode(ta))
    assert key(got[1]) == key(ref_b.decode(tb))


def test_batch_of_16_long_windows_split_softmax(ctx):
    # full-attention windows up to ~650 rows over 16 sequences: more than 256
    # weighted-sum workgroups, so the batched step runs the separate
    # statistics pass; sliding layers keep the single-kernel form
    gm = sharing_model(ctx)
    prompts = ragged_prompts(16, 300, 640, 1000, seed=33)
    run_batch_vs_solo(gm, 1000, prompts, steps=3, max_tokens=700, solo_flags=rd.DET_DECODE_PER_OP)


def ple_sharing_model(ctx):
    """Per-layer inputs (width 64) with KV-sharing donors, softcap and layer scalars."""
    cfg = {"text_config": {
        "enable_moe_block": False, "head_dim": 64, "hidden_activation": "gelu_pytorch_tanh", "hidden_size": 256,
        "intermediate_size": 512, "layer_types": ["sliding_attention", "full_attention", "sliding_attention",
                                                  "full_attention"],
        "num_attention_heads": 4, "num_hidden_layers": 4, "num_key_value_heads": 2, "num_kv_shared_layers": 2,
        "final_logit_softcapping": 30.0, "hidden_size_per_layer_input": 64, "vocab_size_per_layer_input": 1000,
        "rms_norm_eps": 1e-6, "sliding_window": 5, "tie_word_embeddings": False, "vocab_size": 1000,
    }}
    return build(ctx, cfg, fixtures.custom_model(cfg, seed=9, layer_scalars=True))


@pytest.mark.parametrize("mode", ["graph", "eager"])
@pytest.mark.parametrize("n", [3, 5, 16, 19])
def test_per_layer_input_model_batch_matches_solo(ctx, n, mode):
    # the fused batched step with the per-layer input stage (every layer's
    # inputs of each sequence's token, then per layer the gate GEMV over the
    # residual rows, GELU x input, the projection GEMV and the second residual
    # norm) against solo steps through the fused single-sequence step, whose
    # PLE block is pinned to the oracle in test_gpu_decode_fused.py
    gm = ple_sharing_model(ctx)
    assert gm.fused_decode
    prompts = ragged_prompts(n, 1, 14, 1000, seed=40 + n)
    run_batch_vs_solo(gm, 1000, prompts, steps=4, max_tokens=24, flags=rd.DET_COMMIT_ALL | MODES[mode])


def test_per_layer_input_model_fused_batch_matches_per_op_batch(ctx):
    gm = ple_sharing_model(ctx)
    prompts = ragged_prompts(6, 2, 12, 1000, seed=77)
    a = [gm.session(24) for _ in prompts]
    b = [gm.session(24) for _ in prompts]
    ta = [s.prefill(p).next_token for s, p in zip(a, prompts)]
    tb = [s.prefill(p).next_token for s, p in zip(b, prompts)]
    for step in range(5):
        ra = rd.decode_batch(a, ta, rd.DET_COMMIT_ALL)
        rb = rd.decode_batch(b, tb, rd.DET_COMMIT_ALL | rd.DET_DECODE_PER_OP)
        assert [key(r) for r in ra] == [key(r) for r in rb], step
        ta, tb = [r.next_token for r in ra], [r.next_token for r in rb]


def test_e4b_shaped_per_layer_input_batch_of_16_matches_solo(ctx):
    # hidden 2560, PLE width 256: the 16-token GEMVs over the model projection
    # (L*P x H), the per-layer gate (P x H) and projection (H x P)
    cfg = synthetic.e4b_config(layers=2, vocab=4096, sliding_window=8, ple=256)
    gm = build(ctx, cfg, synthetic.synthetic_model_fast(cfg, seed=21, scale_max=256))
    assert gm.fused_decode
    prompts = ragged_prompts(16, 1, 40, 4096, seed=6)
    run_batch_vs_solo(gm, 4096, prompts, steps=3, max_tokens=48)
