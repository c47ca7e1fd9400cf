"""GPU parity against the oracle at the configurations' own sizes.

* attention at E4B head shapes (hd 256, 8 query / 2 KV heads) for 129-1000
  queries, unbounded and 512-row windows: several score passes per query;
* the seven E4B projections (config 3) at M = 128, 512 and 2048 token rows;
* the 2-layer E4B-shaped decoder after prompts longer than the 512-row sliding
  window: decode attention over many 32-row chunks, the ring wrapped;
* 16 sequences of 300-700 tokens decoded in shared batched steps, each
  sequence's commitments equal to the oracle's capture of that sequence alone
  (multi-chunk workgroups and the separate softmax statistics pass);
* the full 42-layer E4B-shaped model (config 4): 512-token prompt, then all
  256 greedy decode steps, every capture entry equal to the oracle's;
* the longest prompt of the ragged 16-sequence set (config 5, 1643 tokens)
  through the 42 layers, equal to the oracle's capture (full-attention
  windows past 1600 rows), and all 16 sequences decoded in shared batched
  steps for the 128 steps of config 5, equal to their solo decodes.

The oracle runs on all host cores with the reference's parallel schedule
(token-parallel slab GEMV in groups of 16 token rows, item-parallel
attention); it is itself pinned by test_oracle_*.py.
"""
import time

import numpy as np
import pytest

import fixtures
import oracle_lib

pytestmark = pytest.mark.gpu
rd = pytest.importorskip("rasterdet")
from rasterdet import synthetic  # noqa: E402

THREADS = oracle_lib.cpu_count()


@pytest.fixture(scope="module", autouse=True)
def grouped_oracle_slabs():
    # the oracle's slab GEMVs take 16 token rows per work item here (the same
    # sums as the reference's one-row items, test_oracle_goldens.py), so the
    # long prompts' prefills read each weight row once per 16 tokens
    oracle_lib.set_slab_group(16)
    yield
    oracle_lib.set_slab_group(1)


@pytest.fixture(scope="module")
def ctx():
    c = rd.Context(0)
    yield c
    c.close()


def expand16(q, s):
    w = q.astype(np.int32) * s.astype(np.int32)[:, None]
    assert np.abs(w).max() < 32768
    return w.astype(np.int16)


@pytest.mark.parametrize("nq,window,mag", [(129, 0, 17), (300, 512, 17), (600, 0, 18), (600, 512, 17),
                                           (1000, 0, 16), (1000, 512, 20)])
def test_attention_causal_e4b_heads(ctx, nq, window, mag):
    nh, nkv, hd = 8, 2, 256
    rng = np.random.default_rng(nq * 7 + window + mag)
    lim = 1 << mag
    q = rng.integers(-lim, lim, size=(nq, nh * hd), dtype=np.int64).astype(np.int32)
    k = rng.integers(-lim, lim, size=(nq, nkv * hd), dtype=np.int64).astype(np.int32)
    v = rng.integers(-lim, lim, size=(nq, nkv * hd), dtype=np.int64).astype(np.int32)
    out = ctx.empty((nq, nh * hd))
    ctx.attention(ctx.to_device(q), ctx.to_device(k), ctx.to_device(v), nq, nq, nh, nkv, hd, window, out)
    exp = oracle_lib.attention_causal(q, k, v, nq, nq, nh, nkv, hd, window, threads=THREADS)
    assert np.array_equal(out.numpy(), exp)


E4B_PROJECTIONS = [("q", 2048, 2560), ("k", 512, 2560), ("v", 512, 2560), ("o", 2560, 2048),
                   ("gate", 10240, 2560), ("up", 10240, 2560), ("down", 2560, 10240)]


@pytest.fixture(scope="module")
def e4b_projections(ctx):
    mats = []
    for i, (name, n, k) in enumerate(E4B_PROJECTIONS):
        q, s = synthetic.fast_int8_matrix(977 + i, n, k, 256)
        mats.append((name, ctx.upload_matrix(q, s), expand16(q, s)))
    return mats


@pytest.mark.parametrize("m", [128, 512, 2048])
def test_prefill_projections_e4b_layer(ctx, e4b_projections, m):
    rng = np.random.default_rng(m)
    acts = {k: synthetic.f32_to_act(rng.standard_normal((m, k)).astype(np.float32)) for k in (2048, 2560, 10240)}
    for name, mat, w16 in e4b_projections:
        a = acts[w16.shape[1]]
        out = ctx.empty((m, mat.rows))
        ctx.det_linear_slab(mat, m, ctx.to_device(a), out)
        exp = oracle_lib.det_linear_slab(w16, a, threads=THREADS)
        assert np.array_equal(out.numpy(), exp), name


def e4b_two_layers(ctx, vocab=4096, window=512, seed=7):
    cfg = synthetic.e4b_config(layers=2, vocab=vocab, sliding_window=window)
    tensors = synthetic.synthetic_model_fast(cfg, seed=seed, scale_max=256)
    return fixtures.load_both(cfg, tensors, ctx, threads=THREADS)


@pytest.fixture(scope="module")
def two_layer_models(ctx):
    return e4b_two_layers(ctx)


# 65, 100 and 128 tokens: the layer prefill's gate/up GEMM with the GELU
# epilogue in one round of 64 x 160 blocks (65: one token in the last block),
# q/k/v in 32 x 48 blocks (100, 128), o in 16 x 80 blocks (128)
@pytest.mark.parametrize("prompt_len", [65, 100, 128, 600, 777])
def test_two_layer_e4b_long_prompt_capture(two_layer_models, prompt_len):
    om, gm = two_layer_models
    rng = np.random.default_rng(prompt_len)
    prompt = rng.integers(0, 4096, size=prompt_len).tolist()
    exp = om.capture(prompt, 6)
    got = gm.capture(prompt, 6)
    assert got["prefill"] == exp["prefill"]
    assert got["first_step_layers"] == exp["first_step_layers"]
    assert got["decode_steps"] == exp["decode_steps"]
    assert got["end_to_end"] == exp["end_to_end"]


def test_two_layer_e4b_batch_of_16_matches_oracle(two_layer_models):
    om, gm = two_layer_models
    rng = np.random.default_rng(2026)
    lens = rng.integers(300, 701, size=16)
    prompts = [rng.integers(0, 4096, size=int(k)).tolist() for k in lens]
    steps = 3
    t0 = time.time()
    exp = []
    for p in prompts:
        exp.append(om.capture(p, steps))
        print(f"[batch16] oracle capture of {len(p)} tokens done at {time.time() - t0:.1f}s", flush=True)
    sess = [gm.session(int(k) + steps + 1) for k in lens]
    toks = []
    for s, p, e in zip(sess, prompts, exp):
        r = s.prefill(p)
        assert (r.embedding.decode(), r.final_hidden.decode(), r.logits.decode()) == (
            e["prefill"]["embedding"], e["prefill"]["final_hidden"], e["prefill"]["logits"])
        toks.append(r.next_token)
    for step in range(steps):
        res = rd.decode_batch(sess, toks, rd.DET_COMMIT_ALL)
        for i, r in enumerate(res):
            e = exp[i]["decode_steps"][step]
            assert toks[i] == e["token"], (step, i)
            assert (r.activation.decode(), r.logits.decode(), r.kv.decode()) == (
                e["activation"], e["logits"], e["kv"]), (step, i)
        toks = [r.next_token for r in res]


def test_long_window_split_softmax_decode_matches_oracle(ctx):
    # ~9000-row full-attention window with one KV head: more than 256
    # weighted-sum workgroups, so the fused step runs the separate softmax
    # statistics pass
    cfg = synthetic.e4b_config(layers=2, vocab=1024, sliding_window=5)
    cfg["text_config"].update({"hidden_size": 256, "intermediate_size": 512, "head_dim": 64,
                               "num_attention_heads": 4, "num_key_value_heads": 1})
    om, gm = fixtures.load_both(cfg, fixtures.custom_model(cfg, seed=17), ctx, threads=THREADS)
    prompt = np.random.default_rng(4).integers(0, 1024, size=9000).tolist()
    exp = om.capture(prompt, 3)
    got = gm.capture(prompt, 3)
    assert got == exp


@pytest.fixture(scope="module")
def e4b_full(ctx):
    """Config 4: the 42-layer E4B-shaped model (vocab 262144, alternating
    sliding-512 / full attention) with q int8 and row scales in [1, 256]."""
    cfg = synthetic.e4b_config()
    t0 = time.time()
    om, gm = fixtures.load_both(cfg, synthetic.synthetic_model_fast(cfg, seed=2024, scale_max=256), ctx,
                                threads=THREADS)
    print(f"[e4b] 42-layer model on GPU and oracle in {time.time() - t0:.1f}s ({THREADS} oracle threads)", flush=True)
    yield om, gm
    del om, gm


E4B_DECODE_STEPS = 256  # config 4's greedy steps (contexts 512..767)


def test_e4b_42_layers_prompt_512_capture_matches_oracle(e4b_full):
    # every checkpoint of the det_goldens capture: prefill embedding / final
    # hidden / logits / KV, each first-step layer output and effective-cache
    # commitment, then each greedy step's token, activation, logits and KV
    om, gm = e4b_full
    prompt = np.random.default_rng(2024).integers(0, 262144, size=512).tolist()
    t0 = time.time()
    got = gm.capture(prompt, E4B_DECODE_STEPS)
    print(f"[e4b] GPU capture {time.time() - t0:.1f}s", flush=True)
    t0 = time.time()
    exp = om.capture(prompt, E4B_DECODE_STEPS)
    print(f"[e4b] oracle capture {time.time() - t0:.1f}s", flush=True)
    assert got["prefill"] == exp["prefill"]
    assert len(got["first_step_layers"]) == 42
    assert got["first_step_layers"] == exp["first_step_layers"]
    assert got["decode_steps"] == exp["decode_steps"]
    assert got["end_to_end"] == exp["end_to_end"]


def test_e4b_42_layers_checkpoint_trace_matches_oracle(e4b_full):
    # the claimer's trace (det_trace_run: fused decode with every layer's
    # output captured, KV commitments hashed on the host pool from the
    # append-only mirror) equals the payloads built from the oracle's
    # checkpoint commitments, entry for entry
    import trace_builder

    om, gm = e4b_full
    prompt = np.random.default_rng(77).integers(0, 262144, size=512).tolist()
    steps = 8
    text = lambda ids: ",".join(map(str, ids))  # noqa: E731
    t0 = time.time()
    got, paused = gm.trace("e4b prompt", prompt, max_new_tokens=steps, detokenize=text)
    print(f"[e4b] GPU trace {time.time() - t0:.1f}s", flush=True)
    t0 = time.time()
    cap = om.trace_capture(prompt, steps)
    print(f"[e4b] oracle trace capture {time.time() - t0:.1f}s", flush=True)
    gen = [s["token"] for s in cap["steps"]]
    exp = trace_builder.expected_trace(cap, "e4b prompt", prompt, steps, text(gen))
    import json
    assert not paused
    assert [next(iter(e.items())) for e in json.loads(got)] == exp


def ragged_prompts():
    # config 5: 16 prompts with seeded lengths uniform in [32, 2048] (the
    # ragged set bench.py decodes: seed 2029, lengths 91-1643)
    rng = np.random.default_rng(2029)
    lens = rng.integers(32, 2049, size=16)
    return lens, [rng.integers(0, 262144, size=int(k)).tolist() for k in lens]


def test_e4b_42_layers_longest_ragged_prompt_matches_oracle(e4b_full):
    # the solo decode that the batched steps are compared with below, anchored
    # to the oracle at config 5's longest prompt: full-attention windows of
    # 1643-1651 rows, sliding rings wrapped three times
    om, gm = e4b_full
    lens, prompts = ragged_prompts()
    prompt = prompts[int(np.argmax(lens))]
    assert len(prompt) == 1643
    steps = 8
    t0 = time.time()
    got = gm.capture(prompt, steps)
    print(f"[e4b-1643] GPU capture {time.time() - t0:.1f}s", flush=True)
    t0 = time.time()
    exp = om.capture(prompt, steps)
    print(f"[e4b-1643] oracle capture {time.time() - t0:.1f}s", flush=True)
    assert got["prefill"] == exp["prefill"]
    assert got["first_step_layers"] == exp["first_step_layers"]
    assert got["decode_steps"] == exp["decode_steps"]
    assert got["end_to_end"] == exp["end_to_end"]


RAGGED_STEPS = 128  # config 5's greedy steps


def test_e4b_42_layers_ragged_16_batch_matches_solo(e4b_full):
    # config 5: 16 sequences with seeded prompt lengths in [32, 2048] decoded
    # in shared batched steps for all 128 steps; each sequence's activation
    # and logits commitments every step, and its KV commitment every 16th
    # step and at the last, equal its solo decode (whose commitments are the
    # oracle's at 512 and 1643 tokens, above)
    _, gm = e4b_full
    lens, prompts = ragged_prompts()
    steps = RAGGED_STEPS
    t0 = time.time()
    batch = [gm.session(int(k) + steps + 1) for k in lens]
    toks = [s.prefill(p, rd.DET_COMMIT_NONE).next_token for s, p in zip(batch, prompts)]
    solo = [s.clone() for s in batch]
    tok_s = list(toks)
    print(f"[ragged16] prefilled {int(lens.sum())} tokens in {time.time() - t0:.1f}s", flush=True)
    for step in range(steps):
        kv = step % 16 == 0 or step == steps - 1
        flags = rd.DET_COMMIT_ALL if kv else rd.DET_COMMIT_ACTIVATIONS
        res = rd.decode_batch(batch, toks, flags)
        for i, r in enumerate(res):
            e = solo[i].decode(tok_s[i], flags)
            assert (r.activation, r.logits, r.kv, r.next_token) == (e.activation, e.logits, e.kv, e.next_token), \
                (step, i, int(lens[i]))
            toks[i], tok_s[i] = r.next_token, e.next_token
        if kv:
            print(f"[ragged16] step {step} checked (with KV) at {time.time() - t0:.1f}s", flush=True)
    print(f"[ragged16] {steps} batched steps checked against solo in {time.time() - t0:.1f}s", flush=True)
