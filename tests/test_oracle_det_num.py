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


# ---------------- nth_root_acc / RoPE frequencies, pinned exactly ----------------
# The reference (ops.rs:555-611) takes the largest Q32.32 value m in
# [0, max(value, one)] whose sequential power chain pow_acc_u32(m, degree)
# (one, then acc_mul by m degree times, each product rounded half to even and
# saturated to i64) does not exceed the value, then rounds to whichever of m and
# m + 1 (saturating) has the power nearest the value, ties to the even one.
# The restatement below shares no code with the oracle: acc_mul is the
# closed-form rational rounding (pinned above), and the floor is found by
# galloping from a floating-point estimate of the root instead of bisecting.
ONE = 1 << 32
I64MAX = (1 << 63) - 1


def py_acc_mul(a, b):
    return sat(rte(Fraction(a * b, ONE)), -(1 << 63), I64MAX)


def py_pow(m, degree):
    r = ONE
    for _ in range(degree):
        r = py_acc_mul(r, m)
    return r


def py_floor_root(value, degree):
    """Largest m in [0, max(value, one)] with py_pow(m, degree) <= value.

    py_pow is non-decreasing in m (acc_mul of non-negative operands is), so the
    values that qualify form a prefix of [0, hi]."""
    hi = max(value, ONE)
    est = min(hi, max(0, int((value / ONE) ** (1.0 / degree) * ONE)))
    m, step = est, 1
    while py_pow(m, degree) > value:  # gallop down to a qualifying m
        m, step = max(0, m - step), step * 2
    step = 1
    while m < hi and py_pow(min(hi, m + step), degree) <= value:  # gallop up
        m, step = min(hi, m + step), step * 2
    lo_ok, hi_bad = m, min(hi, m + step)  # py_pow(lo_ok) <= value, and hi_bad fails unless it is hi
    if py_pow(hi_bad, degree) <= value:
        return hi_bad
    while hi_bad - lo_ok > 1:
        mid = (lo_ok + hi_bad) // 2
        if py_pow(mid, degree) <= value:
            lo_ok = mid
        else:
            hi_bad = mid
    return lo_ok


def py_nth_root(value, degree):
    if degree == 1 or value == ONE:
        return value
    lower = py_floor_root(value, degree)
    upper = min(lower + 1, I64MAX)
    el, eu = abs(value - py_pow(lower, degree)), abs(py_pow(upper, degree) - value)
    if eu != el:
        return upper if eu < el else lower
    return lower if lower % 2 == 0 else upper


NTH_ROOT_BASES = [10000 * ONE, 1_000_000 * ONE, 12345 * ONE, 16 * ONE, int(3.5 * ONE), ONE + 1, ONE - 1,
                  ONE // 2, ONE // 1000, 7, I64MAX - 1, I64MAX - 12345, 5 * 10**17]


@pytest.mark.parametrize("base", NTH_ROOT_BASES)
def test_nth_root_equals_exact_restatement_for_every_degree(base):
    chosen_upper = 0
    for degree in list(range(1, 33)) + [47, 64, 100, 127, 128, 200, 256]:
        got = out64(L.orc_nth_root_acc, base, degree)
        exp = py_nth_root(base, degree)
        assert got == exp, (base, degree)
        if degree > 1 and got < I64MAX:
            # nearest power: no worse than the neighbouring Q32.32 values
            err = abs(base - py_pow(got, degree))
            assert err <= abs(base - py_pow(got + 1, degree)), (base, degree)
            assert got == 0 or err <= abs(base - py_pow(got - 1, degree)), (base, degree)
            chosen_upper += got != py_floor_root(base, degree)
    if base == 10000 * ONE:
        assert chosen_upper > 0  # the set exercises rounding up as well as down


def test_nth_root_saturating_search():
    # near i64::MAX every large candidate's power chain saturates to i64::MAX,
    # which exceeds the value, so the search stays below the saturation point
    for v in (I64MAX - 1, I64MAX - (1 << 40)):
        for degree in (2, 3, 128):
            assert out64(L.orc_nth_root_acc, v, degree) == py_nth_root(v, degree)


def test_nth_root_of_i64_max_is_the_reference_overflow_panic():
    # ops.rs:578 computes high - low + 1 = i64::MAX + 1 on the first step: the
    # reference panics (overflow checks) or bisects forever (wrapping), so the
    # oracle reports the panic as a contract violation, status 2
    o = C.c_int64()
    for degree in (2, 3, 128):
        assert L.orc_nth_root_acc(I64MAX, degree, C.byref(o)) == 2
    assert out64(L.orc_nth_root_acc, I64MAX, 1) == I64MAX  # degree 1 returns before the search


def test_nth_root_ties_go_to_the_even_candidate():
    # degree 2: pow(m) = acc_mul(m, m). A value exactly halfway between the
    # powers of consecutive candidates is a tie; both parities occur.
    parities = set()
    m = 3 * ONE // 2
    while len(parities) < 2:
        p0, p1 = py_pow(m, 2), py_pow(m + 1, 2)
        if (p0 + p1) % 2 == 0 and p1 > p0:
            v = (p0 + p1) // 2
            assert py_floor_root(v, 2) == m
            got = out64(L.orc_nth_root_acc, v, 2)
            assert got == (m if m % 2 == 0 else m + 1), m
            parities.add(m % 2)
        m += 1


@pytest.mark.parametrize("base", [10000 * ONE, 1_000_000 * ONE, 12345 * ONE, int(3.5 * ONE)])
@pytest.mark.parametrize("freq_base_dim", [2, 4, 16, 64, 256, 512])
def test_rope_frequency_step_and_inverse_frequency_chain(base, freq_base_dim):
    # rope_frequency_step = div_acc(one, nth_root_acc(base, fbd / 2)) (ops.rs:555-559),
    # div_acc rounding half to even; the chain multiplies by it after every pair
    # (ops.rs:184-195). E4B tables: fbd 256 with 128 pairs (sliding) and 32 (full).
    root = py_nth_root(base, freq_base_dim // 2)
    step = sat(rte(Fraction(ONE * ONE, root)), -(1 << 63), I64MAX)
    assert out64(L.orc_rope_frequency_step, base, freq_base_dim) == step
    half = freq_base_dim // 2
    chain, f = [], ONE
    for _ in range(half):
        chain.append(f)
        f = py_acc_mul(f, step)
    assert oracle_lib.rope_inv_frequencies(base, freq_base_dim, half).tolist() == chain
