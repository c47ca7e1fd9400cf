"""GPU parity of the reference's own i16 / i32 weights on the int8 MFMA path.

The reference stores Q16.16 weight bits as i16, or i32 when a value does not
fit (src/shared/numerics/det_num/artifact.rs:57-63), and streams them through
dot_act_i16 / dot_act_i32 (det_simd.rs:246-265). Bits that do not factor into
int8 x row scale are held here as int8 digit planes, W = s * sum_p 256^p d_p
with s = +1 or -1 per row: two planes for i16 rows, four for i32 rows or for
i16 rows with values near both ends of the range. Every GEMV and GEMM kernel
reads the planes as extra weight tiles and combines them with shifts. The
oracle computes the reference's wrapping i64 sums on the i16 / i32 bits
themselves.
"""
import numpy as np
import pytest

import fixtures
import oracle_lib

pytestmark = pytest.mark.gpu
rd = pytest.importorskip("rasterdet")
from rasterdet import synthetic  # noqa: E402

THREADS = oracle_lib.cpu_count()


@pytest.fixture(scope="module")
def ctx():
    c = rd.Context(0)
    yield c
    c.close()


def gpu_rows(ctx, mat, acts):
    acts = np.atleast_2d(acts)
    m = acts.shape[0]
    out = ctx.empty((m, mat.rows))
    a = ctx.to_device(np.ascontiguousarray(acts))
    if m == 1:
        ctx.det_linear_into(mat, a, out)
    else:
        ctx.det_linear_slab(mat, m, a, out)
    return out.numpy().reshape(m, mat.rows)


def wide_i32(rng, rows, cols):
    # i32 bits beyond int16 with row mass < 2^31; row 3 holds a value near
    # +2^31 (the negated four-digit form) and row 5 one near -2^31
    lim = (2**31 - 1) // (2 * cols)
    w = rng.integers(-lim, lim, size=(rows, cols)).astype(np.int32)
    w[:, 0] = 70001
    if rows > 5:
        w[3, :] = 0
        w[3, 1] = 2**31 - 1
        w[5, :] = 0
        w[5, 2] = -(2**31) + 1
    return w


# shapes of the decode GEMVs (one tile per workgroup, several load batches,
# the persistent kernel past 4096 tiles) and ragged tails
@pytest.mark.parametrize("rows,cols", [(2560, 2560), (10240, 2560), (2560, 10240), (385, 64), (37, 3),
                                       (33, 16384), (100, 12345), (65552, 128)])
def test_gemv_i16_digit_planes(ctx, rows, cols):
    w = synthetic.fast_i16_matrix(rows * 31 + cols, rows, cols)
    rng = np.random.default_rng(rows + cols)
    act = synthetic.f32_to_act(rng.standard_normal(cols).astype(np.float32))
    mat = ctx.upload_matrix(w)
    assert mat.storage == rd.DET_STORAGE_I16
    assert np.array_equal(gpu_rows(ctx, mat, act)[0], oracle_lib.det_linear(w, act, threads=THREADS))


def test_gemv_i16_full_range_and_extreme_activations(ctx):
    # i16 bits over the whole range, rows holding both 32767 and -32768 (the
    # matrix takes four planes), activations at the i32 edges
    rng = np.random.default_rng(11)
    rows, cols = 96, 700
    w = rng.integers(-32768, 32768, size=(rows, cols)).astype(np.int16)
    w[::5, 3] = 32767
    w[::5, 4] = -32768
    mat = ctx.upload_matrix(w)
    for act in (np.full(cols, 2**31 - 1, dtype=np.int32), np.full(cols, -(2**31), dtype=np.int32),
                rng.integers(-(2**31), 2**31, size=cols).astype(np.int32)):
        assert np.array_equal(gpu_rows(ctx, mat, act)[0], oracle_lib.det_linear(w, act))


@pytest.mark.parametrize("rows,cols", [(129, 333), (2048, 2560), (512, 10240)])
def test_gemv_i32_digit_planes(ctx, rows, cols):
    rng = np.random.default_rng(rows * 3 + cols)
    w = wide_i32(rng, rows, cols)
    act = rng.integers(-(2**31), 2**31, size=cols).astype(np.int32)
    mat = ctx.upload_matrix(w)
    assert mat.storage == rd.DET_STORAGE_I32
    assert np.array_equal(gpu_rows(ctx, mat, act)[0], oracle_lib.det_linear(w, act, threads=THREADS))


def test_raw_accumulators_i16(ctx):
    w = synthetic.fast_i16_matrix(5, 300, 777)
    act = np.random.default_rng(5).integers(-(2**31), 2**31, size=777).astype(np.int32)
    mat = ctx.upload_matrix(w)
    out = ctx.empty(300, np.int64)
    ctx.det_linear_acc_i64(mat, ctx.to_device(act), out)
    assert np.array_equal(out.numpy(), oracle_lib.det_linear_acc_i64(w.astype(np.int32), act))


# slabs: 2-15 rows on the GEMV kernels, 16+ on the MFMA GEMM (128- and
# 256-row blocks, K split into partial planes at 128 rows)
@pytest.mark.parametrize("m", [2, 3, 4, 5, 9, 16, 33, 128, 512])
@pytest.mark.parametrize("rows,cols", [(512, 2560), (2560, 2048)])
def test_slab_i16_digit_planes(ctx, m, rows, cols):
    w = synthetic.fast_i16_matrix(m * 101 + rows, rows, cols)
    rng = np.random.default_rng(m)
    acts = synthetic.f32_to_act(rng.standard_normal((m, cols)).astype(np.float32))
    mat = ctx.upload_matrix(w)
    assert np.array_equal(gpu_rows(ctx, mat, acts), oracle_lib.det_linear_slab(w, acts, threads=THREADS))


@pytest.mark.parametrize("m", [3, 20, 64, 300])
def test_slab_i32_digit_planes(ctx, m):
    rng = np.random.default_rng(m + 7)
    w = wide_i32(rng, 400, 1000)
    acts = rng.integers(-(2**31), 2**31, size=(m, 1000)).astype(np.int32)
    mat = ctx.upload_matrix(w)
    assert np.array_equal(gpu_rows(ctx, mat, acts), oracle_lib.det_linear_slab(w, acts, threads=THREADS))


def i16_model(ctx, layers=2, vocab=4096, window=64, seed=3, lim=4096):
    cfg = synthetic.e4b_config(layers=layers, vocab=vocab, sliding_window=window)
    tensors = list(synthetic.synthetic_model_i16(cfg, seed=seed, lim=lim))
    return cfg, fixtures.load_both(cfg, tensors, ctx, threads=THREADS)


@pytest.fixture(scope="module")
def i16_two_layers(ctx):
    return i16_model(ctx)


def test_i16_e4b_shaped_model_takes_the_fused_step(i16_two_layers):
    _, (om, gm) = i16_two_layers
    assert gm.fused_decode


@pytest.mark.parametrize("prompt_len", [9, 100])
def test_i16_e4b_shaped_capture_matches_oracle(i16_two_layers, prompt_len):
    # prefill (GEMV under 16 rows, MFMA GEMMs with the fused q/k/v and the
    # gate/up GELU epilogue above), then the fused decode step graph-replayed
    _, (om, gm) = i16_two_layers
    prompt = np.random.default_rng(prompt_len).integers(0, 4096, size=prompt_len).tolist()
    exp = om.capture(prompt, 12)
    got = gm.capture(prompt, 12)
    assert got["prefill"] == exp["prefill"]
    assert got["first_step_layers"] == exp["first_step_layers"]
    assert got["decode_steps"] == exp["decode_steps"]
    assert got["end_to_end"] == exp["end_to_end"]


@pytest.mark.parametrize("n", [3, 16])
def test_i16_e4b_shaped_batch_matches_solo(i16_two_layers, n):
    # batched fused steps (4-token and 16-token GEMVs over the digit planes)
    _, (om, gm) = i16_two_layers
    rng = np.random.default_rng(n)
    lens = rng.integers(20, 120, size=n)
    prompts = [rng.integers(0, 4096, size=int(k)).tolist() for k in lens]
    steps = 6
    batch = [gm.session(int(k) + steps + 1) for k in lens]
    toks = [s.prefill(p, rd.DET_COMMIT_NONE).next_token for s, p in zip(batch, prompts)]
    solo = [s.clone() for s in batch]
    tok_s = list(toks)
    for step in range(steps):
        res = rd.decode_batch(batch, toks, rd.DET_COMMIT_ALL)
        for i, r in enumerate(res):
            e = solo[i].decode(tok_s[i], rd.DET_COMMIT_ALL)
            assert (r.activation, r.logits, r.kv, r.next_token) == (e.activation, e.logits, e.kv, e.next_token), \
                (step, i)
            toks[i], tok_s[i] = r.next_token, e.next_token


@pytest.mark.parametrize("n", [6, 16])
def test_mixed_i16_int8_batch_matches_solo(ctx, n):
    # gate/up and the q/k/v projections in i16 digit planes (the four-token-group
    # batched GEMV and its GELU epilogue), down, O and the vocabulary projection
    # int8 (the register-activation GEMV on the activations the digit-plane
    # epilogue and the row kernels write)
    cfg = synthetic.e4b_config(layers=2, vocab=8192, sliding_window=64)
    wide = list(synthetic.synthetic_model_i16(cfg, seed=5))
    narrow = {name: (v, s) for name, v, s in synthetic.synthetic_model_fast(cfg, seed=5)}
    gm = rd.Model(ctx, cfg)
    for name, v, s in wide:
        if any(k in name for k in ("mlp.down_proj", "o_proj", "lm_head", "embed_tokens")):
            v, s = narrow[name]
        gm.set_tensor(name, v, s)
    gm = gm.finalize()
    assert gm.fused_decode
    rng = np.random.default_rng(n + 40)
    lens = rng.integers(10, 60, size=n)
    prompts = [rng.integers(0, 8192, size=int(k)).tolist() for k in lens]
    steps = 4
    batch = [gm.session(int(k) + steps + 1) for k in lens]
    toks = [s.prefill(p, rd.DET_COMMIT_NONE).next_token for s, p in zip(batch, prompts)]
    solo = [s.clone() for s in batch]
    tok_s = list(toks)
    for step in range(steps):
        res = rd.decode_batch(batch, toks, rd.DET_COMMIT_ALL)
        for i, r in enumerate(res):
            e = solo[i].decode(tok_s[i], rd.DET_COMMIT_ALL)
            assert (r.activation, r.logits, r.kv, r.next_token) == (e.activation, e.logits, e.kv, e.next_token), \
                (step, i)
            toks[i], tok_s[i] = r.next_token, e.next_token


def test_i32_model_matches_oracle(ctx):
    # every matrix in four digit planes (one wide value per matrix): the
    # GEMMs take the 256-row blocks, the decode step its per-op form where
    # the fused kernels' job counts do not fit
    cfg = synthetic.e4b_config(layers=2, vocab=1024, sliding_window=16)
    cfg["text_config"].update({"hidden_size": 256, "intermediate_size": 512, "head_dim": 64,
                               "num_attention_heads": 4, "num_key_value_heads": 2})
    tensors = []
    for name, v, s in synthetic.synthetic_model_i16(cfg, seed=9, lim=2000):
        if v.ndim == 2:
            v = v.astype(np.int32)
            v[1, 1] = 70000  # past int16: the matrix is i32
        tensors.append((name, v, s))
    om, gm = fixtures.load_both(cfg, tensors, ctx, threads=THREADS)
    prompt = list(range(5, 45))
    assert gm.capture(prompt, 8) == om.capture(prompt, 8)
