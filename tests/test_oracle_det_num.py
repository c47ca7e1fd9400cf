"""Pins the oracle's scalar arithmetic.

1. Golden vectors transcribed from the reference's own unit tests
   (src/shared/numerics/det_num/tests.rs), stored in golden/det_num_vectors.json.
2. Closed forms the mathematics fixes, checked with Python big integers and
   exact rationals (a different computation from the oracle's i128 code):
   round-half-even division, acc_mul, inverse square root by integer search,
   wrapping MAC folds in any order.
"""
import ctypes as C
import json
import math
import random
from fractions import Fraction

import numpy as np
import pytest

import fixtures
import oracle_lib

L = oracle_lib.lib()
V = json.loads((fixtures.GOLDEN_DIR / "det_num_vectors.json").read_text())


def i32a(xs):
    return np.asarray(xs, dtype=np.int32)


def out32(fn, *args):
    o = C.c_int32()
    oracle_lib.check(fn(*args, C.byref(o)), scalar=True)
    return o.value


def out64(fn, *args):
    o = C.c_int64()
    oracle_lib.check(fn(*args, C.byref(o)), scalar=True)
    return o.value


def rte(fr: Fraction) -> int:
    """Round a rational to nearest, ties to even."""
    return round(fr)  # Python's round() on Fraction is half-to-even


def sat(v, lo, hi):
    return max(lo, min(hi, v))


def wrap64(v):
    v &= (1 << 64) - 1
    return v - (1 << 64) if v >> 63 else v


@pytest.mark.parametrize("acc,a,w,exp", V["mac"])
def test_mac_golden(acc, a, w, exp):
    assert L.orc_mac_bits(acc, a, w) == exp


@pytest.mark.parametrize("a,b,exp", V["acc_combine"])
def test_acc_combine_golden(a, b, exp):
    assert L.orc_acc_combine(a, b) == exp


@pytest.mark.parametrize("a,b,exp", V["add_sat"])
def test_add_sat_golden(a, b, exp):
    assert L.orc_add_sat(a, b) == exp


@pytest.mark.parametrize("a,b,exp", V["sub_sat"])
def test_sub_sat_golden(a, b, exp):
    assert L.orc_sub_sat(a, b) == exp


@pytest.mark.parametrize("a,b,exp", V["acc_add_sat"])
def test_acc_add_sat_golden(a, b, exp):
    assert L.orc_acc_add_sat(a, b) == exp


@pytest.mark.parametrize("a,b,exp", V["mul_sat"])
def test_mul_sat_golden(a, b, exp):
    assert L.orc_mul_sat(a, b) == exp


@pytest.mark.parametrize("n,d,exp", V["div_act"])
def test_div_act_golden(n, d, exp):
    assert out32(L.orc_div_act, n, d) == exp


@pytest.mark.parametrize("v,d,exp", V["div_acc_by_u32"])
def test_div_acc_by_u32_golden(v, d, exp):
    assert out64(L.orc_div_acc_by_u32, v, d) == exp


@pytest.mark.parametrize("acc,exp", V["requantize"])
def test_requantize_golden(acc, exp):
    assert L.orc_requantize(acc) == exp


@pytest.mark.parametrize("x,s,exp", V["rshift"])
def test_rshift_golden(x, s, exp):
    assert out64(L.orc_rshift_round_ties_even, x, s) == exp


def test_rshift_rejects_64():
    with pytest.raises(oracle_lib.OracleError):
        out64(L.orc_rshift_round_ties_even, 1, 64)


@pytest.mark.parametrize("xs,eps,exp", V["rms_norm_scale"])
def test_rms_norm_scale_golden(xs, eps, exp):
    x = i32a(xs)
    assert out32(L.orc_rms_norm_scale, oracle_lib.ptr(x), x.size, eps) == exp


@pytest.mark.parametrize("xs,ws,eps,exp", V["rms_norm"])
def test_rms_norm_golden(xs, ws, eps, exp):
    x, w = i32a(xs), i32a(ws)
    oracle_lib.check(L.orc_rms_norm(oracle_lib.ptr(x), oracle_lib.ptr(w), x.size, eps), scalar=True)
    assert x.tolist() == exp


@pytest.mark.parametrize("xs,eps,exp", V["value_rms_norm"])
def test_value_rms_norm_golden(xs, eps, exp):
    x = i32a(xs)
    oracle_lib.check(L.orc_value_rms_norm(oracle_lib.ptr(x), x.size, eps), scalar=True)
    assert x.tolist() == exp


@pytest.mark.parametrize("q,k,exp", V["attention_score"])
def test_attention_score_golden(q, k, exp):
    q, k = i32a(q), i32a(k)
    assert out32(L.orc_attention_score, oracle_lib.ptr(q), oracle_lib.ptr(k), q.size) == exp


@pytest.mark.parametrize("logits,exp", V["attention_softmax"])
def test_attention_softmax_golden(logits, exp):
    x = i32a(logits)
    w = np.empty_like(x)
    oracle_lib.check(L.orc_attention_softmax(oracle_lib.ptr(x), x.size, oracle_lib.ptr(w)), scalar=True)
    assert w.tolist() == exp


@pytest.mark.parametrize("weights,rows,exp", V["attention_weighted_sum"])
def test_weighted_sum_golden(weights, rows, exp):
    w, r = i32a(weights), i32a(rows)
    o = np.empty(r.shape[1], dtype=np.int32)
    oracle_lib.check(L.orc_attention_weighted_sum(oracle_lib.ptr(w), oracle_lib.ptr(r), r.shape[0], r.shape[1],
                                                  oracle_lib.ptr(o)), scalar=True)
    assert o.tolist() == exp


@pytest.mark.parametrize("x,exp", V["tanh"])
def test_tanh_golden(x, exp):
    assert L.orc_tanh_act(x) == exp


@pytest.mark.parametrize("x,c,exp", V["softcap"])
def test_softcap_golden(x, c, exp):
    assert out32(L.orc_softcap_act, x, c) == exp


def test_softcap_rejects_non_positive():
    with pytest.raises(oracle_lib.OracleError) as e:
        out32(L.orc_softcap_act, 65536, 0)
    assert e.value.status == 2


@pytest.mark.parametrize("x,exp", V["gelu"])
def test_gelu_golden(x, exp):
    assert L.orc_gelu_pytorch_tanh_act(x) == exp


@pytest.mark.parametrize("v,rd,fbd,base,pos,exp", V["rope"])
def test_rope_golden(v, rd, fbd, base, pos, exp):
    x = i32a(v)
    oracle_lib.check(L.orc_rope_rotate_pairs(oracle_lib.ptr(x), x.size, rd, fbd, base, pos), scalar=True)
    assert x.tolist() == exp


def test_rope_zero_position_and_tail_identity():
    # tests.rs:1086-1098 and :1100-1116
    base = [65536, 16384, 32768, -16384, 196608]
    x = i32a(base)
    oracle_lib.check(L.orc_rope_rotate_pairs(oracle_lib.ptr(x), 5, 4, 4, 16 << 32, 0), scalar=True)
    assert x.tolist() == base
    y = i32a([65536, 0, 32768, -32768, 196608])
    oracle_lib.check(L.orc_rope_rotate_pairs(oracle_lib.ptr(y), 5, 4, 4, 1_000_000 << 32, 4096), scalar=True)
    assert y[4] == 196608 and y[1] != 0


def test_rope_rejects_odd_rotary_dim():
    x = i32a([65536, 0, 32768])
    assert L.orc_rope_rotate_pairs(oracle_lib.ptr(x), 3, 3, 4, 16 << 32, 1) == 2


@pytest.mark.parametrize("xs,exp", V["argmax_first"])
def test_argmax_golden(xs, exp):
    x = i32a(xs)
    o = C.c_size_t()
    oracle_lib.check(L.orc_argmax_first(oracle_lib.ptr(x), x.size, C.byref(o)), scalar=True)
    assert o.value == exp


@pytest.mark.parametrize("x,exp", V["f32_to_wgt"])
def test_f32_to_wgt_golden(x, exp):
    assert out32(L.orc_f32_to_wgt, float(np.float32(x))) == exp
    assert out32(L.orc_f32_to_act, float(np.float32(x))) == exp


def test_f32_to_wgt_largest_subnormal():
    x = np.array([0x007FFFFF], dtype=np.uint32).view(np.float32)[0]
    assert out32(L.orc_f32_to_wgt, float(x)) == 0


@pytest.mark.parametrize("x,exp", V["f32_to_acc"])
def test_f32_to_acc_golden(x, exp):
    assert out64(L.orc_f32_to_acc, float(np.float32(x))) == exp


def test_f32_conversion_rejects_non_finite():
    for v in (float("nan"), float("inf")):
        with pytest.raises(oracle_lib.OracleError):
            out32(L.orc_f32_to_wgt, v)


# ---------------- closed forms (exact big-integer / rational checks) ----------------

def test_requantize_div_and_acc_mul_closed_forms():
    rng = random.Random(7)
    for _ in range(4000):
        x = rng.randrange(-(1 << 63), 1 << 63)
        assert L.orc_requantize(x) == sat(rte(Fraction(x, 1 << 16)), -(1 << 31), (1 << 31) - 1)
        a, b = rng.randrange(-(1 << 63), 1 << 63), rng.randrange(-(1 << 63), 1 << 63)
        assert L.orc_acc_mul(a, b) == sat(rte(Fraction(a * b, 1 << 32)), -(1 << 63), (1 << 63) - 1)
        d = rng.randrange(1, 1 << 32)
        assert out64(L.orc_div_acc_by_u32, x, d) == sat(rte(Fraction(x, d)), -(1 << 63), (1 << 63) - 1)
        n32, d32 = rng.randrange(-(1 << 31), 1 << 31), rng.choice([1, -1]) * rng.randrange(1, 1 << 31)
        assert out32(L.orc_div_act, n32, d32) == sat(rte(Fraction(n32 << 16, d32)), -(1 << 31), (1 << 31) - 1)
        den = rng.randrange(1, 1 << 62)
        num = rng.randrange(0, 1 << 33)
        assert out64(L.orc_div_acc, num, den) == sat(rte(Fraction(num << 32, den)), -(1 << 63), (1 << 63) - 1)


def test_inv_sqrt_matches_integer_search():
    # inv_sqrt_acc returns the integer c in [0, 2^31-1] minimising |c^2 x - 2^64|
    # (ties to even), with x = 0 and tiny x saturating at i32::MAX. Checked
    # against math.isqrt, an unrelated algorithm.
    rng = random.Random(11)
    xs = [1, 2, 3, 4, 5, 1 << 2, (1 << 2) + 1, 1 << 32, (1 << 63) - 1, 4295, 12345678901]
    xs += [rng.randrange(1, 1 << 63) for _ in range(3000)] + [rng.randrange(1, 1 << 20) for _ in range(500)]
    T = 1 << 64
    for x in xs:
        c0 = math.isqrt(T // x)
        best = None
        for c in (c0 - 1, c0, c0 + 1, c0 + 2):
            if c < 0:
                continue
            c = min(c, (1 << 31) - 1)
            err = abs(c * c * x - T)
            key = (err, c & 1, c)
            if best is None or key < best[0]:
                best = (key, c)
        exp = best[1]
        # the reference saturates when even i32::MAX is not large enough
        if ((1 << 31) - 1) ** 2 * x <= T:
            exp = (1 << 31) - 1
        assert out32(L.orc_inv_sqrt_acc, x) == exp, x


def test_wrapping_mac_is_order_independent():
    # tests.rs:330-411: fold, tree and chunked reductions agree under wrapping.
    rng = np.random.default_rng(3)
    a = rng.integers(-(1 << 31), 1 << 31, size=257, dtype=np.int64).astype(np.int32)
    w = rng.integers(-(1 << 31), 1 << 31, size=257, dtype=np.int64).astype(np.int32)
    exact = sum(int(x) * int(y) for x, y in zip(a, w))
    acc = 0
    for x, y in zip(a.tolist(), w.tolist()):
        acc = L.orc_mac_bits(acc, x, y)
    assert acc == wrap64(exact)
    out = oracle_lib.det_linear_acc_i64(w.reshape(1, -1), a)
    assert int(out[0]) == wrap64(exact)


def test_softmax_weights_sum_to_one():
    rng = np.random.default_rng(5)
    for n in (1, 2, 7, 64, 300):
        x = rng.integers(-(20 << 16), 20 << 16, size=n).astype(np.int32)
        w = np.empty_like(x)
        oracle_lib.check(L.orc_attention_softmax(oracle_lib.ptr(x), n, oracle_lib.ptr(w)), scalar=True)
        assert int(w.astype(np.int64).sum()) == 65536
        assert int(np.argmax(w)) == int(np.argmax(x))  # residual goes to the first max


def test_gemv_matches_brute_force_for_every_tail_length():
    # det_kernels.rs:1341-1367 fixtures (closed-form integer sequences).
    def fixture_matrix(rows, cols):
        idx = np.arange(rows * cols, dtype=np.int64)
        return (((idx * 2654435761) % 131072) - 65536).astype(np.int32).reshape(rows, cols)

    def fixture_input(cols):
        idx = np.arange(cols, dtype=np.int64)
        return (((idx * 40503) % 98304) - 49152).astype(np.int32)

    for cols in list(range(1, 41)) + [63, 64, 65, 129]:
        W, x = fixture_matrix(4, cols), fixture_input(cols)
        out = oracle_lib.det_linear(W, x)
        for r in range(4):
            acc = wrap64(sum(int(a) * int(b) for a, b in zip(x, W[r])))
            assert out[r] == sat(rte(Fraction(acc, 1 << 16)), -(1 << 31), (1 << 31) - 1)
    # row-parallel schedule equals serial (det_kernels.rs:1296-1320)
    W, x = fixture_matrix(128 * 3 + 17, 64), fixture_input(64)
    ref = oracle_lib.det_linear(W, x, threads=1)
    for t in (2, 3, 4, 8):
        assert np.array_equal(oracle_lib.det_linear(W, x, threads=t), ref)
    # i16 storage == i32 storage
    Wn = (fixture_matrix(6, 200) // 2).astype(np.int16)
    assert np.array_equal(oracle_lib.det_linear(Wn, fixture_input(200)),
                          oracle_lib.det_linear(Wn.astype(np.int32), fixture_input(200)))


def test_sin_cos_is_close_to_libm():
    # sin_cos_acc is a quadrant-reduced Taylor polynomial; it must track libm
    # to ~1e-3 over the whole circle (a wrong quadrant or sign fails this).
    for k in range(-200, 201):
        ang = k * 0.0417
        bits = int(round(ang * (1 << 32)))
        c, s = C.c_int32(), C.c_int32()
        L.orc_sin_cos_acc(bits, C.byref(c), C.byref(s))
        assert abs(c.value / 65536 - math.cos(ang)) < 2e-3
        assert abs(s.value / 65536 - math.sin(ang)) < 2e-3


def test_nth_root_and_frequency_step():
    for base, deg in [(16 << 32, 2), (10000 << 32, 8), (1_000_000 << 32, 128), (12345 << 32, 1)]:
        r = out64(L.orc_nth_root_acc, base, deg)
        assert abs(r / 2**32 - (base / 2**32) ** (1 / deg)) < 1e-6 * max(1, r / 2**32)
        step = out64(L.orc_rope_frequency_step, base, 2 * deg)
        assert abs(step / 2**32 - 1 / (r / 2**32)) < 1e-8
