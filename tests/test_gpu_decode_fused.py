"""GPU parity of the fused, graph-captured decode step.

The fused step (one HIP graph per session: fused QKV GEMV, head-norm/RoPE/KV
append, split-context attention, O GEMV with requantize-on-load, gate/up
GEMV with the GELU epilogue, down GEMV, norm/residual kernels) must produce
exactly the reference's commitments: checked against the oracle and against
the per-op kernel schedule on the same session state.
"""
import numpy as np
import pytest

import fixtures
import oracle_lib

pytestmark = pytest.mark.gpu
rd = pytest.importorskip("rasterdet")
from rasterdet import synthetic  # noqa: E402


@pytest.fixture(scope="module")
def ctx():
    c = rd.Context(0)
    yield c
    c.close()


def e4b_two_layer_config(window=8, vocab=4096):
    cfg = synthetic.e4b_config(layers=2, vocab=vocab, sliding_window=window)
    return cfg


def test_e4b_shaped_layers_fused_decode_matches_oracle(ctx):
    cfg = e4b_two_layer_config()
    tensors = list(synthetic.synthetic_model_fast(cfg, seed=7))
    om, gm = fixtures.load_both(cfg, tensors, ctx, threads=oracle_lib.cpu_count())
    prompt = list(range(3, 3 + 21))  # 21 tokens > sliding window 8: ring wraps
    exp = om.capture(prompt, 6)
    got = gm.capture(prompt, 6)
    assert got["prefill"] == exp["prefill"]
    assert got["first_step_layers"] == exp["first_step_layers"]
    assert got["decode_steps"] == exp["decode_steps"]
    assert got["end_to_end"] == exp["end_to_end"]


def test_fused_and_per_op_decode_agree_over_many_steps(ctx):
    cfg = e4b_two_layer_config(window=5, vocab=2048)
    gm = rd.Model(ctx, cfg)
    for name, v, s in synthetic.synthetic_model_fast(cfg, seed=11):
        gm.set_tensor(name, v, s)
    gm.finalize()
    prompt = list(range(100, 112))
    a, b = gm.session(64), gm.session(64)
    ta = a.prefill(prompt).next_token
    tb = b.prefill(prompt).next_token
    assert ta == tb
    for step in range(40):
        ra = a.decode(ta, rd.DET_COMMIT_ALL)
        rb = b.decode(tb, rd.DET_COMMIT_ALL | (rd.DET_DECODE_PER_OP if step % 2 else rd.DET_DECODE_EAGER))
        assert (ra.activation, ra.logits, ra.kv, ra.next_token) == (rb.activation, rb.logits, rb.kv, rb.next_token), step
        ta, tb = ra.next_token, rb.next_token


def test_fused_decode_with_kv_sharing_k_eq_v_softcap_and_scalars(ctx):
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
    # full layers use num_global_key_value_heads under attention_k_eq_v (gemma/io.rs:1910-1918)
    tensors = []
    for name, v, s in fixtures.custom_model(cfg, seed=3, layer_scalars=True):
        if (".self_attn.k_proj" in name or ".self_attn.v_proj" in name) and \
                tc["layer_types"][int(name.split(".layers.")[1].split(".")[0])] == "full_attention":
            v, s = v[:64], s[:64]
        tensors.append((name, v, s))
    om, gm = fixtures.load_both(cfg, tensors, ctx)
    prompt = [5, 900, 17, 3, 250, 64, 64, 1, 999]
    exp = om.capture(prompt, 12)
    got = gm.capture(prompt, 12)
    assert got == exp


def test_fused_decode_long_context_split_softmax_matches_per_op(ctx):
    # a full-attention window of ~9000 rows: the fused step computes the
    # softmax statistics in their own pass (more than 256 weighted-sum
    # workgroups); the per-op schedule uses the prefill attention kernel
    cfg = e4b_two_layer_config(window=5, vocab=1024)
    tc = cfg["text_config"]
    tc.update({"hidden_size": 256, "intermediate_size": 512, "head_dim": 64, "num_attention_heads": 4,
               "num_key_value_heads": 1})
    gm = rd.Model(ctx, cfg)
    for name, v, s in fixtures.custom_model(cfg, seed=17):
        gm.set_tensor(name, v, s)
    gm.finalize()
    rng = np.random.default_rng(4)
    prompt = rng.integers(0, 1024, size=9000).tolist()
    a, b = gm.session(9024), gm.session(9024)
    ta = a.prefill(prompt, rd.DET_COMMIT_NONE).next_token
    tb = b.prefill(prompt, rd.DET_COMMIT_NONE).next_token
    assert ta == tb
    for step in range(6):
        ra = a.decode(ta, rd.DET_COMMIT_ALL | (rd.DET_DECODE_EAGER if step % 2 else 0))
        rb = b.decode(tb, rd.DET_COMMIT_ALL | rd.DET_DECODE_PER_OP)
        assert (ra.activation, ra.logits, ra.kv, ra.next_token) == (rb.activation, rb.logits, rb.kv, rb.next_token), step
        ta, tb = ra.next_token, rb.next_token


def test_fused_decode_with_per_layer_inputs_matches_oracle(ctx):
    # E4B-shaped layers with per-layer inputs (PLE width 256): the fused step
    # computes every layer's per-layer input once per step and runs the PLE
    # block (gate GEMV, GELU x input, projection GEMV, norm + residual)
    # between the MLP and the next layer
    cfg = synthetic.e4b_config(layers=2, vocab=4096, sliding_window=8, ple=256)
    om, gm = fixtures.load_both(cfg, synthetic.synthetic_model_fast(cfg, seed=21, scale_max=256), ctx,
                                threads=oracle_lib.cpu_count())
    assert gm.fused_decode
    prompt = list(range(40, 40 + 21))
    exp = om.capture(prompt, 6)
    got = gm.capture(prompt, 6)
    assert got["prefill"] == exp["prefill"]
    assert got["first_step_layers"] == exp["first_step_layers"]
    assert got["decode_steps"] == exp["decode_steps"]
    assert got["end_to_end"] == exp["end_to_end"]


def test_fused_decode_with_per_layer_inputs_kv_sharing_and_scalars(ctx):
    cfg = {"text_config": {
        "enable_moe_block": False, "head_dim": 64, "hidden_activation": "gelu_pytorch_tanh", "hidden_size": 256,
        "intermediate_size": 512, "layer_types": ["sliding_attention", "full_attention", "sliding_attention",
                                                  "full_attention"],
        "num_attention_heads": 4, "num_hidden_layers": 4, "num_key_value_heads": 2, "num_kv_shared_layers": 2,
        "final_logit_softcapping": 30.0, "hidden_size_per_layer_input": 64, "vocab_size_per_layer_input": 1000,
        "rms_norm_eps": 1e-6, "sliding_window": 5, "tie_word_embeddings": False, "vocab_size": 1000,
    }}
    om, gm = fixtures.load_both(cfg, fixtures.custom_model(cfg, seed=9, layer_scalars=True), ctx)
    assert gm.fused_decode
    prompt = [5, 900, 17, 3, 250, 64, 64, 1, 999, 12]
    assert gm.capture(prompt, 12) == om.capture(prompt, 12)
    # the same steps through the per-op schedule, step by step
    a, b = gm.session(32), gm.session(32)
    ta = a.prefill(prompt).next_token
    tb = b.prefill(prompt).next_token
    for step in range(10):
        ra = a.decode(ta, rd.DET_COMMIT_ALL | (rd.DET_DECODE_EAGER if step % 2 else 0))
        rb = b.decode(tb, rd.DET_COMMIT_ALL | rd.DET_DECODE_PER_OP)
        assert (ra.activation, ra.logits, ra.kv, ra.next_token) == (rb.activation, rb.logits, rb.kv, rb.next_token), step
        ta, tb = ra.next_token, rb.next_token


def test_e4b_shaped_layers_with_scalars_and_per_layer_inputs_match_oracle(ctx):
    # hidden 2560: between prefill layers the last residual norm, the layer
    # scalar and the next layer's input norm run as one row pass (two layer
    # boundaries here, one after a PLE block)
    cfg = synthetic.e4b_config(layers=3, vocab=4096, sliding_window=8, ple=256)
    om, gm = fixtures.load_both(cfg, fixtures.custom_model(cfg, seed=5, scale_max=256, layer_scalars=True), ctx,
                                threads=oracle_lib.cpu_count())
    prompt = list(range(300, 300 + 19))
    exp = om.capture(prompt, 3)
    got = gm.capture(prompt, 3)
    assert got["prefill"] == exp["prefill"]
    assert got["first_step_layers"] == exp["first_step_layers"]
    assert got["decode_steps"] == exp["decode_steps"]
