"""GPU parity of the int8 prefill GEMM (det_linear_slab with 16 or more rows).

Small and ragged shapes are compared with the oracle's det_linear_slab
(det_kernels.rs:180-203); shapes at E4B's projection sizes are compared row
by row with the GPU GEMV, whose results are themselves pinned to the oracle
in test_gpu_parity.py (every output element of the slab GEMM has the term set
of the single-row GEMV).
"""
import numpy as np
import pytest

import oracle_lib

pytestmark = pytest.mark.gpu

rd = pytest.importorskip("rasterdet")
from rasterdet import synthetic  # noqa: E402


@pytest.fixture(scope="module")
def ctx():
    c = rd.Context(0)
    yield c
    c.close()


def expand(q, s):
    w = q.astype(np.int64) * s.astype(np.int64)[:, None]
    return w.astype(np.int16) if np.abs(w).max(initial=0) < 32768 else w.astype(np.int32)


def gpu_slab(ctx, mat, acts):
    acts = np.ascontiguousarray(acts, dtype=np.int32)
    m = acts.shape[0]
    a = ctx.to_device(acts)
    out = ctx.empty((m, mat.rows))
    ctx.det_linear_slab(mat, m, a, out)
    return out.numpy().reshape(m, mat.rows)


def gpu_rows(ctx, mat, acts):
    """Each row through the single-row GEMV (oracle-pinned in test_gpu_parity.py)."""
    rows = []
    for r in acts:
        a = ctx.to_device(np.ascontiguousarray(r, dtype=np.int32))
        out = ctx.empty(mat.rows)
        ctx.det_linear_into(mat, a, out)
        rows.append(out.numpy().copy())
    return np.stack(rows)


def act_slab(m, k, seed):
    rng = np.random.default_rng(seed)
    return synthetic.f32_to_act(rng.standard_normal((m, k)).astype(np.float32))


@pytest.mark.parametrize("m,n,k", [(16, 16, 64), (17, 33, 100), (31, 129, 128), (32, 128, 256), (33, 200, 2600),
                                   (100, 1000, 777), (128, 520, 130), (257, 64, 2048)])
def test_gemm_matches_oracle(ctx, m, n, k):
    rng = np.random.default_rng(m * 1000 + n + k)
    q, s = synthetic.random_int8_matrix(rng, n, k, scale_max=256)
    acts = act_slab(m, k, seed=m + k)
    mat = ctx.upload_matrix(q, s)
    got = gpu_slab(ctx, mat, acts)
    exp = oracle_lib.det_linear_slab(expand(q, s), acts, threads=oracle_lib.cpu_count())
    assert np.array_equal(got, exp)


@pytest.mark.parametrize("m,n,k", [(40, 96, 16384), (40, 96, 17000), (24, 64, 33000)])
def test_gemm_longest_rows(ctx, m, n, k):
    # one value past 2^23 in the last column part of one token group: 16384
    # columns (64 parts), each part with its own limb count; 17000 and 33000
    # columns: more parts than the per-group flag mask holds, so every part
    # takes four limbs
    rng = np.random.default_rng(k)
    q, s = synthetic.random_int8_matrix(rng, n, k, scale_max=256)
    acts = act_slab(m, k, seed=k)
    acts[5, k - 3] = 2**23 + 5
    mat = ctx.upload_matrix(q, s)
    got = gpu_slab(ctx, mat, acts)
    exp = oracle_lib.det_linear_slab(expand(q, s), acts, threads=oracle_lib.cpu_count())
    assert np.array_equal(got, exp)


def test_gemm_adversarial_values(ctx):
    # activations at the i32 edges, weights at +-127, scales at the largest
    # value that keeps every row mass below 2^31 (wrapping accumulators)
    rng = np.random.default_rng(7)
    m, n, k = 40, 64, 1024
    q = rng.integers(-127, 128, size=(n, k), dtype=np.int8)
    q[0, :] = 127
    q[1, :] = -127
    q[2, ::2] = 127
    mass = np.abs(q.astype(np.int64)).sum(axis=1)
    s = ((2**31 - 1) // np.maximum(mass, 1)).astype(np.int32)
    edges = np.array([-(2**31), 2**31 - 1, 0, 1, -1, 65536, -65536], dtype=np.int32)
    acts = rng.choice(edges, size=(m, k))
    acts[0, :] = 2**31 - 1
    acts[1, :] = -(2**31)
    mat = ctx.upload_matrix(q, s)
    got = gpu_slab(ctx, mat, acts)
    exp = oracle_lib.det_linear_slab(expand(q, s), acts, threads=oracle_lib.cpu_count())
    assert np.array_equal(got, exp)


@pytest.mark.parametrize("m,n,k", [(100, 300, 2600), (200, 1000, 777), (64, 128, 4096)])
def test_gemm_limb_decompositions(ctx, m, n, k):
    # token groups of 16 whose activations lie in [-2^23, 2^23) over a
    # 256-column part take three limbs there, the others four: values at both
    # edges of the range, groups with a single value outside it, values at the
    # top of the int32 range, blocks mixing both kinds
    rng = np.random.default_rng(m + n + k)
    q, s = synthetic.random_int8_matrix(rng, n, k, scale_max=256)
    acts = act_slab(m, k, seed=k)
    acts[0, :4] = [2**23 - 1, -(2**23), 2**23 - 1, -(2**23)]     # group 0: three limbs, at the edges
    acts[17, k // 2] = 2**23                                       # group 1: four limbs (one value)
    acts[40, k - 1] = -(2**23) - 1                                  # group 2: four limbs (last column)
    acts[50, 3] = 2**31 - 2**23                                     # group 3: top of the int32 range
    acts[51, k // 3] = 2**31 - 2**23 - 1
    acts[52, 130] = 2**31 - 1
    if m > 64:
        acts[64:80, :] = rng.integers(-(2**31), 2**31, size=(16, k), dtype=np.int64).astype(np.int32)
    mat = ctx.upload_matrix(q, s)
    got = gpu_slab(ctx, mat, acts)
    exp = oracle_lib.det_linear_slab(expand(q, s), acts, threads=oracle_lib.cpu_count())
    assert np.array_equal(got, exp)


def test_gemm_unaligned_activation_rows(ctx):
    # rows whose stride is not a multiple of 16 bytes take the per-element loads
    m, n, k = 40, 96, 301
    rng = np.random.default_rng(5)
    q, s = synthetic.random_int8_matrix(rng, n, k, scale_max=256)
    acts = act_slab(m, k, seed=9)
    acts[3, 7] = 2**31 - 1
    acts[20, 300] = -(2**31)
    mat = ctx.upload_matrix(q, s)
    got = gpu_slab(ctx, mat, acts)
    exp = oracle_lib.det_linear_slab(expand(q, s), acts, threads=oracle_lib.cpu_count())
    assert np.array_equal(got, exp)


# (160, 16384, 2560): one round of 256 x 256 blocks filling at least five
# eighths of the CUs instead of more than one round of 128 x 128 blocks (a
# ragged last token block). One-round blocks whose copy halves per K step do
# not divide over the waves: (128 | 100 | 65, 20480, 2560) 64 x 160 blocks
# (the stacked gate/up slab; 65 rows: one token in the last block),
# (128 | 100 | 97, 3072, 2560) 32 x 48 blocks (q/k/v), (128 | 113, 2560, 2048)
# 16 x 80 blocks (o; 113 rows: one token in the last group).
@pytest.mark.parametrize("m,n,k", [(128, 3072, 2560), (100, 3072, 2560), (97, 3072, 2560), (64, 2560, 10240),
                                   (48, 2560, 2048), (128, 2560, 2048), (113, 2560, 2048), (256, 16384, 512),
                                   (300, 13100, 2600), (128, 20480, 2560), (100, 20480, 2560), (65, 20480, 2560),
                                   (160, 16384, 2560)])
def test_gemm_e4b_shapes_match_gemv_rows(ctx, m, n, k):
    q, s = synthetic.fast_int8_matrix(n * 31 + k, n, k, 256)
    acts = act_slab(m, k, seed=n + k)
    mat = ctx.upload_matrix(q, s)
    assert np.array_equal(gpu_slab(ctx, mat, acts), gpu_rows(ctx, mat, acts))


def test_captured_slab_calls_replay_exactly(ctx):
    # det_ctx_capture_begin/end: the calls are recorded, not run, and every
    # replay of the graph produces the direct calls' outputs (split-K GEMMs
    # included: 16 x 512 x 2560 takes the partial-plane path)
    shapes = [(512, 2560), (2560, 10240), (2048, 2560)]
    m = 128
    mats, acts, outs, want = [], [], [], []
    for i, (n, k) in enumerate(shapes):
        q, s = synthetic.fast_int8_matrix(900 + i, n, k, 256)
        mats.append(ctx.upload_matrix(q, s))
        acts.append(ctx.to_device(act_slab(m, k, seed=i)))
        outs.append(ctx.empty((m, n)))
    for mat, a, o in zip(mats, acts, outs):
        ctx.det_linear_slab(mat, m, a, o)
    want = [o.numpy().copy() for o in outs]

    def calls():
        for mat, a, o in zip(mats, acts, outs):
            ctx.det_linear_slab(mat, m, a, o)

    for o in outs:
        o.upload(np.zeros(o.shape, np.int32))
    graph = ctx.capture(calls)
    ctx.synchronize()
    assert all(not o.numpy().any() for o in outs)  # recorded, not run
    for _ in range(3):
        graph.launch()
        ctx.synchronize()
        assert all(np.array_equal(o.numpy(), w) for o, w in zip(outs, want))
        for o in outs:
            o.upload(np.zeros(o.shape, np.int32))


def test_capture_refuses_growing_scratch_and_ends():
    # a fresh context has no GEMM scratch yet: the recorded call would have to
    # allocate it, so it is refused, the capture ends and the stream runs again
    c = rd.Context(0)
    try:
        q, s = synthetic.fast_int8_matrix(5, 512, 2560, 256)
        mat = c.upload_matrix(q, s)
        a = c.to_device(act_slab(128, 2560, seed=3))
        o = c.empty((128, 512))
        with pytest.raises(rd.DetError, match="run the call once before capturing"):
            c.capture(lambda: c.det_linear_slab(mat, 128, a, o))
        c.det_linear_slab(mat, 128, a, o)
        want = o.numpy().copy()
        assert np.array_equal(want, gpu_rows(c, mat, act_slab(128, 2560, seed=3)))
        o.upload(np.zeros(o.shape, np.int32))
        graph = c.capture(lambda: c.det_linear_slab(mat, 128, a, o))
        for _ in range(2):
            graph.launch()
            c.synchronize()
            assert np.array_equal(o.numpy(), want)
    finally:
        c.close()
