"""GPU parity: the HIP det path against the CPU oracle, bit-exact.

Every case calls the product through its C ABI (libdetgpu.so via ctypes) and
compares with the oracle restatement of the reference on the same seeded
inputs. The oracle itself is pinned by test_oracle_*.py.
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


def expand(q, s):
    return q.astype(np.int64) * s.astype(np.int64)[:, None]


def oracle_gemv(w64, act):
    w = w64.astype(np.int16) if np.abs(w64).max(initial=0) < 32768 else w64.astype(np.int32)
    return oracle_lib.det_linear(w, act, threads=4)


def gpu_linear(ctx, mat, act_rows):
    act_rows = np.atleast_2d(act_rows).astype(np.int32)
    m = act_rows.shape[0]
    a = ctx.to_device(act_rows)
    out = ctx.empty((m, mat.rows))
    if m == 1:
        ctx.det_linear_into(mat, a, out)
    else:
        ctx.det_linear_slab(mat, m, a, out)
    return out.numpy()


@pytest.mark.parametrize("cols", list(range(1, 41)) + [63, 64, 65, 127, 128, 129, 200, 1000, 2560])
def test_gemv_int8_every_tail_length(ctx, cols):
    rng = np.random.default_rng(cols)
    rows = 37
    q, s = synthetic.random_int8_matrix(rng, rows, cols)
    act = rng.integers(-(1 << 31), 1 << 31, size=cols, dtype=np.int64).astype(np.int32)
    mat = ctx.upload_matrix(q, s)
    assert mat.storage == rd.DET_STORAGE_INT8
    got = gpu_linear(ctx, mat, act)[0]
    assert np.array_equal(got, oracle_gemv(expand(q, s), act))


# K of 12345 / 16384 takes two load batches per wave in the one-tile-per-
# workgroup kernel; 65552 rows (4097 tiles) goes to the persistent kernel
@pytest.mark.parametrize("rows,cols", [(2560, 2560), (10240, 2560), (2560, 10240), (385, 64), (17, 4096),
                                       (2048, 2560), (33, 16384), (100, 12345), (65552, 128), (65536, 130)])
def test_gemv_int8_decode_shapes(ctx, rows, cols):
    q, s, act = synthetic.gemv_problem(rows, cols, seed=rows * 7 + cols)
    mat = ctx.upload_matrix(q, s)
    got = gpu_linear(ctx, mat, act)[0]
    assert np.array_equal(got, oracle_gemv(expand(q, s), act))


def test_gemv_adversarial_activations(ctx):
    # |a| at the i32 edges and scales near the row-mass limit.
    rng = np.random.default_rng(99)
    cols = 1024
    q = rng.integers(-127, 128, size=(64, cols), dtype=np.int8)
    q[0, :] = 127
    q[1, :] = -127
    mass = np.abs(q.astype(np.int64)).sum(axis=1)
    s = ((2**31 - 1) // mass).astype(np.int32)  # largest scale that keeps the row mass < 2^31
    for act in (np.full(cols, 2**31 - 1, dtype=np.int32), np.full(cols, -(2**31), dtype=np.int32),
                rng.choice(np.array([-(2**31), 2**31 - 1, 0, 1, -1], dtype=np.int32), size=cols)):
        mat = ctx.upload_matrix(q, s)
        assert np.array_equal(gpu_linear(ctx, mat, act)[0], oracle_gemv(expand(q, s), act))


def test_gemv_raw_accumulators(ctx):
    q, s, act = synthetic.gemv_problem(300, 777, seed=5)
    mat = ctx.upload_matrix(q, s)
    a = ctx.to_device(act)
    out = ctx.empty(300, np.int64)
    ctx.det_linear_acc_i64(mat, a, out)
    exp = oracle_lib.det_linear_acc_i64(expand(q, s).astype(np.int32), act)
    assert np.array_equal(out.numpy(), exp)


@pytest.mark.parametrize("dtype", [np.int16, np.int32])
def test_gemv_wide_storage(ctx, dtype):
    # values that do not factor into int8 x scale take the wide path
    rng = np.random.default_rng(3)
    rows, cols = 129, 333
    hi = 30000 if dtype == np.int16 else 5_000_000
    w = rng.integers(-hi, hi, size=(rows, cols)).astype(dtype)
    w[:, 0] = 1  # gcd 1 with large entries: not int8-factorizable
    act = rng.integers(-(1 << 31), 1 << 31, size=cols, dtype=np.int64).astype(np.int32)
    mat = ctx.upload_matrix(w)
    assert mat.storage in (rd.DET_STORAGE_I16, rd.DET_STORAGE_I32)
    got = gpu_linear(ctx, mat, act)[0]
    assert np.array_equal(got, oracle_lib.det_linear(w, act))


def test_wgt_bits_factorize_to_int8(ctx):
    # detwgt v2 bits that are q*s exactly are stored as int8 x scale
    rng = np.random.default_rng(4)
    q, s = synthetic.random_int8_matrix(rng, 50, 96)
    w = expand(q, s).astype(np.int32)
    mat = ctx.upload_matrix(w)
    assert mat.storage == rd.DET_STORAGE_INT8
    act = rng.integers(-(1 << 20), 1 << 20, size=96).astype(np.int32)
    assert np.array_equal(gpu_linear(ctx, mat, act)[0], oracle_lib.det_linear(w, act))


@pytest.mark.parametrize("m", [1, 2, 3, 4, 5, 8, 9, 33])
def test_linear_slab(ctx, m):
    rng = np.random.default_rng(m)
    q, s = synthetic.random_int8_matrix(rng, 200, 300)
    acts = rng.integers(-(1 << 24), 1 << 24, size=(m, 300)).astype(np.int32)
    mat = ctx.upload_matrix(q, s)
    got = gpu_linear(ctx, mat, acts)
    w = expand(q, s)
    exp = oracle_lib.det_linear_slab(w.astype(np.int16) if np.abs(w).max() < 32768 else w.astype(np.int32), acts)
    assert np.array_equal(got, exp)


def test_row_mass_bound_is_enforced(ctx):
    q = np.full((2, 100), 127, dtype=np.int8)
    s = np.array([1, 2**31 // 12700 + 1], dtype=np.int32)
    with pytest.raises(rd.DetError) as e:
        ctx.upload_matrix(q, s)
    assert e.value.status == 1


@pytest.mark.parametrize("rows,cols,weighted", [(1, 1, True), (7, 2, True), (5, 64, False), (3, 2560, True),
                                                (40, 256, True), (2, 16, False)])
def test_rms_norm(ctx, rows, cols, weighted):
    rng = np.random.default_rng(rows * cols)
    x = rng.integers(-(1 << 24), 1 << 24, size=(rows, cols)).astype(np.int32)
    x[0, :] = 0 if rows > 1 else x[0, :]
    w = (65536 + rng.integers(-16, 17, size=cols) * 256).astype(np.int32)
    eps = 4295
    d = ctx.to_device(x)
    wd = ctx.to_device(w) if weighted else None
    ctx.rms_norm(d, rows, cols, wd, eps)
    exp = x.copy()
    L = oracle_lib.lib()
    for r in range(rows):
        row = np.ascontiguousarray(exp[r])
        if weighted:
            oracle_lib.check(L.orc_rms_norm(oracle_lib.ptr(row), oracle_lib.ptr(w), cols, eps), scalar=True)
        else:
            oracle_lib.check(L.orc_value_rms_norm(oracle_lib.ptr(row), cols, eps), scalar=True)
        exp[r] = row
    assert np.array_equal(d.numpy(), exp)


@pytest.mark.parametrize("hd,rotary,base,pos0", [(16, 16, 10000 << 32, 0), (16, 4, 1000000 << 32, 3),
                                                 (256, 256, 10000 << 32, 500), (256, 64, 1000000 << 32, 7),
                                                 (2, 2, 10000 << 32, 1)])
def test_rope(ctx, hd, rotary, base, pos0):
    rng = np.random.default_rng(hd + rotary)
    rows, heads = 6, 3
    x = rng.integers(-(1 << 18), 1 << 18, size=(rows, heads * hd)).astype(np.int32)
    d = ctx.to_device(x)
    ctx.rope_rotate_pairs(d, rows, heads, hd, rotary, hd, base, pos0, 1)
    exp = x.copy()
    L = oracle_lib.lib()
    for r in range(rows):
        for h in range(heads):
            seg = np.ascontiguousarray(exp[r, h * hd:(h + 1) * hd])
            oracle_lib.check(L.orc_rope_rotate_pairs(oracle_lib.ptr(seg), hd, rotary, hd, base, pos0 + r), scalar=True)
            exp[r, h * hd:(h + 1) * hd] = seg
    assert np.array_equal(d.numpy(), exp)


def oracle_attention(q, k, v, nq, nrows, nh, nkv, hd, window):
    L = oracle_lib.lib()
    out = np.zeros((nq, nh * hd), dtype=np.int32)
    g = nh // nkv
    for t in range(nq):
        start = max(0, t + 1 - window) if window else 0
        for h in range(nh):
            kvh = h // g
            rows = t + 1 - start
            qs = np.ascontiguousarray(q[t, h * hd:(h + 1) * hd])
            logits = np.array([0] * rows, dtype=np.int32)
            for r in range(rows):
                ks = np.ascontiguousarray(k[start + r, kvh * hd:(kvh + 1) * hd])
                o = oracle_lib.C.c_int32()
                L.orc_attention_score(oracle_lib.ptr(qs), oracle_lib.ptr(ks), hd, oracle_lib.C.byref(o))
                logits[r] = o.value
            w = np.empty_like(logits)
            L.orc_attention_softmax(oracle_lib.ptr(logits), rows, oracle_lib.ptr(w))
            vs = np.ascontiguousarray(v[start:start + rows, kvh * hd:(kvh + 1) * hd])
            o = np.empty(hd, dtype=np.int32)
            L.orc_attention_weighted_sum(oracle_lib.ptr(w), oracle_lib.ptr(vs), rows, hd, oracle_lib.ptr(o))
            out[t, h * hd:(h + 1) * hd] = o
    return out


@pytest.mark.parametrize("nq,nh,nkv,hd,window,mag", [(9, 4, 1, 16, 0, 18), (12, 2, 1, 2, 4, 16), (20, 8, 2, 256, 5, 16),
                                                     (7, 2, 2, 64, 0, 31),
                                                     # 16 queries or more, head dims a multiple of 64:
                                                     # the MFMA form, int32 extremes included
                                                     (40, 4, 2, 64, 0, 31), (33, 4, 4, 128, 7, 31),
                                                     (48, 2, 1, 512, 0, 24), (17, 8, 1, 64, 16, 31),
                                                     (70, 6, 3, 192, 0, 20)])
def test_attention_causal(ctx, nq, nh, nkv, hd, window, mag):
    rng = np.random.default_rng(nq * hd + mag)
    lim = 1 << mag
    q = rng.integers(-lim, lim, size=(nq, nh * hd), dtype=np.int64).astype(np.int32)
    k = rng.integers(-lim, lim, size=(nq, nkv * hd), dtype=np.int64).astype(np.int32)
    v = rng.integers(-lim, lim, size=(nq, nkv * hd), dtype=np.int64).astype(np.int32)
    out = ctx.empty((nq, nh * hd))
    ctx.attention(ctx.to_device(q), ctx.to_device(k), ctx.to_device(v), nq, nq, nh, nkv, hd, window, out)
    assert np.array_equal(out.numpy(), oracle_attention(q, k, v, nq, nq, nh, nkv, hd, window))


@pytest.mark.parametrize("n", [1, 5, 1023, 1024, 1025, 262144])
def test_argmax_first(ctx, n):
    rng = np.random.default_rng(n)
    x = rng.integers(-1000, 1000, size=n).astype(np.int32)
    if n > 10:
        x[[3, n - 2]] = 5000  # ties resolve to the first index
    assert ctx.argmax_first(ctx.to_device(x), n) == int(np.argmax(x))


@pytest.mark.parametrize("n", [3, 5000, 5003, 20483])
def test_elementwise_ops(ctx, n):
    # (n % 4 != 0: the quad-vector GELU kernel's scalar tail)
    rng = np.random.default_rng(1)
    x = rng.integers(-(1 << 31), 1 << 31, size=n, dtype=np.int64).astype(np.int32)
    y = rng.integers(-(1 << 20), 1 << 20, size=n).astype(np.int32)
    L = oracle_lib.lib()
    cases = [
        (rd.DET_EW_ADD, 0, lambda a, b: L.orc_add_sat(a, b)),
        (rd.DET_EW_GELU_MUL, 0, lambda a, b: L.orc_mul_sat(L.orc_gelu_pytorch_tanh_act(a), b)),
        (rd.DET_EW_SCALE, 46341, lambda a, b: L.orc_mul_sat(a, 46341)),
    ]
    for op, scalar, fn in cases:
        d = ctx.to_device(x)
        ctx.elementwise(op, d, ctx.to_device(y), n, scalar)
        exp = np.array([fn(int(a), int(b)) for a, b in zip(x, y)], dtype=np.int32)
        assert np.array_equal(d.numpy(), exp), op
    d = ctx.to_device(x)
    ctx.elementwise(rd.DET_EW_SOFTCAP, d, None, n, 7 << 16)
    exp = np.empty(n, dtype=np.int32)
    for i, a in enumerate(x):
        o = oracle_lib.C.c_int32()
        L.orc_softcap_act(int(a), 7 << 16, oracle_lib.C.byref(o))
        exp[i] = o.value
    assert np.array_equal(d.numpy(), exp)


# --------------------------- routine-level parity ---------------------------

@pytest.mark.parametrize("name", ["donor_ple", "no_donor_ple"])
def test_gpu_reproduces_reference_det_goldens(ctx, name):
    cfg, wgt, prompt, steps = fixtures.golden_fixture(name)
    model = rd.Model(ctx, cfg).load_detwgt(wgt).finalize()
    got = model.capture(prompt, steps)
    exp = fixtures.golden_expected(name)
    assert got["prefill"] == exp["prefill"]
    assert got["first_step_layers"] == exp["first_step_layers"]
    assert got["decode_steps"] == exp["decode_steps"]
    assert got["end_to_end"] == exp["end_to_end"]


def test_gpu_tiny_gemma_dev_matches_oracle(ctx):
    # committed detwgt asset: softcap 7.5, attention_k_eq_v, 2 KV-shared layers,
    # PLE, partial RoPE on full layers
    cfg, wgt = fixtures.tiny_gemma_dev()
    prompt = [2, 17, 100, 5, 250, 33, 7]
    exp = oracle_lib.OracleModel(cfg).load_detwgt(wgt).finalize().capture(prompt, 12)
    got = rd.Model(ctx, cfg).load_detwgt(wgt).finalize().capture(prompt, 12)
    assert got == exp


@pytest.mark.parametrize("head_dim", [16, 40, 384])
def test_gpu_tiny_baseline_model_matches_oracle(ctx, head_dim):
    # head dims up to 256 and 257-512 take the two forms of the prefill head
    # norm + RoPE kernel (40: rows that are not whole waves)
    cfg, tensors = synthetic.tiny_model(head_dim=head_dim)
    om = oracle_lib.OracleModel(cfg)
    gm = rd.Model(ctx, cfg)
    for name, v, s in tensors:
        om.set_tensor(name, v, 32 if s is None else 8, s)
        gm.set_tensor(name, v, s)
    om.finalize()
    gm.finalize()
    prompt = synthetic.tiny_prompt()
    exp = om.capture(prompt, 8)
    got = gm.capture(prompt, 8)
    assert got == exp

