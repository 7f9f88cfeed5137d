"""Closed-form and invariant checks that pin the oracle where the reference
has no implementation (mul, row/global reductions, argmax semantics, strided
views) or where its known answers leave room (GELU, RoPE, SwiGLU, RNG)."""
import math

import numpy as np
import pytest

from tests.helpers import assert_bits_equal

F16 = np.float16


def test_add_mul_are_single_ieee_ops(orc):
    a = orc.uniform((100000,), 0, 0, -1.0, 1.0)
    b = orc.uniform((100000,), 0, 1, -1.0, 1.0)
    assert_bits_equal(orc.add(a, b), a + b, "f32 add")
    assert_bits_equal(orc.mul(a, b), a * b, "f32 mul")
    ha, hb = a.astype(F16) * F16(300), b.astype(F16) * F16(300)
    # numpy float16 arithmetic widens to f32, operates, rounds once: the same rule
    with np.errstate(over="ignore"):
        assert_bits_equal(orc.add(ha, hb), ha + hb, "f16 add")
        assert_bits_equal(orc.mul(ha, hb), ha * hb, "f16 mul")


def test_denormal_and_special_arithmetic(orc):
    tiny = np.array([1e-45, -1e-45, 1e-40, 3e-39, 0.0, -0.0, np.inf, -np.inf], np.float32)
    other = np.array([1e-45, 1e-45, -2e-40, 1e-39, -0.0, -0.0, 5.0, 1.0], np.float32)
    assert_bits_equal(orc.add(tiny, other), tiny + other, "denormal add")
    assert_bits_equal(orc.mul(tiny, np.float32(3.0) * np.ones_like(tiny)), tiny * np.float32(3.0), "mul")


def test_bias_add_is_broadcast(orc):
    x = orc.uniform((7, 13), 1, 0, -1.0, 1.0)
    b = orc.uniform((13,), 1, 1, -1.0, 1.0)
    assert_bits_equal(orc.bias_add(x, b), x + b[None, :], "bias")
    hx, hb = x.astype(F16), b.astype(F16)
    assert_bits_equal(orc.bias_add(hx, hb), hx + hb[None, :], "bias f16")


def test_gelu_matches_double_formula_away_from_cancellation(orc):
    x = np.linspace(-6, 6, 20001, dtype=np.float32)
    y = orc.gelu(x).astype(np.float64)
    exact = orc.gelu_f64(x)
    pos = x >= 0  # 1 + tanh(u) >= 1: no cancellation
    assert np.all(np.abs(y[pos] - exact[pos]) <= 4e-7 * np.abs(exact[pos]) + 1e-37)
    # for x < 0 the float sum 1 + tanh(u) carries an absolute error of a few
    # ulp(1) = 2^-23, scaled by 0.5|x|: the bound a correct formula meets and a
    # dropped or mis-signed term would not
    neg = (x < 0) & (x > -5)
    assert np.all(np.abs(y[neg] - exact[neg]) <= 4e-7 * np.abs(exact[neg]) + 2.5e-7 * np.abs(x[neg]))
    assert np.all(y[x >= 5] == x[x >= 5]) and np.all(y[x <= -5] == 0)
    # the double formula itself equals x * Phi-like sigmoid form 2x*sigma(2u)/2
    u = (np.float64(np.float32(0.7978845608)) * (x + np.float64(np.float32(0.044715)) * x.astype(np.float64) ** 3))
    alt = x / (1.0 + np.exp(-2.0 * u))
    mid = (x > -5) & (x < 5)
    # (the double form still cancels near x = -5, to ~1e-9 relative)
    assert np.allclose(exact[mid], alt[mid], rtol=1e-8, atol=1e-300)


def test_silu_multiply_formula(orc):
    g = orc.normal((4096,), 2, 0, 0.0, 3.0, "f32")
    u = orc.normal((4096,), 2, 1, 0.0, 3.0, "f32")
    want = (g.astype(np.float64) / (1 + np.exp(-g.astype(np.float64)))) * u
    got = orc.silu_multiply(g, u).astype(np.float64)
    assert np.all(np.abs(got - want) <= 1e-6 * np.abs(want) + 1e-30)


def test_softmax_nan_rule(orc):
    """attention.c:346-372: NaN never becomes the max; exp(NaN) poisons the
    denominator unless a +inf is present, in which case NaN entries get 0."""
    nan, inf = np.nan, np.inf
    y = orc.softmax(np.array([[nan, 1, 2, 3], [nan, inf, 0, 1], [nan, -inf, -inf, -inf]], np.float32))
    assert np.all(np.isnan(y[0]))
    assert y[1].tolist() == [0.0, 1.0, 0.0, 0.0]
    assert y[2].tolist() == [0.0, 0.0, 0.0, 0.0]


def test_row_sum_and_max(orc):
    x = orc.normal((37, 129), 3, 0, 0.0, 3.0, "f16")
    s, a = orc.row_sum(x)
    x64 = x.astype(np.float64)
    assert np.array_equal(s, x64.sum(axis=1)) or np.allclose(s, x64.sum(axis=1), rtol=0, atol=1e-9)
    assert np.allclose(a, np.abs(x64).sum(axis=1), rtol=0, atol=1e-9)
    assert np.array_equal(orc.row_max(x), x.astype(np.float32).max(axis=1))
    y = x.astype(np.float32)
    y[3, 5] = np.nan
    m = orc.row_max(y)
    assert np.isnan(m[3]) and np.array_equal(np.delete(m, 3), np.delete(y.max(axis=1), 3))


def test_sum_max(orc):
    x = orc.uniform((1 << 20,), 4, 0, -1.0, 1.0)
    s, a, m = orc.sum_max(x)
    assert abs(s - x.astype(np.float64).sum()) < 1e-9
    assert m == x.max()
    x[77] = np.nan
    assert np.isnan(orc.sum_max(x)[2])


@pytest.mark.parametrize("values,want", [
    ([-2, 5, 5, 1], 1), ([np.nan, 1, 2], 0), ([1, np.nan, 3, 3], 2),
    ([-np.inf, -np.inf], 0), ([-np.inf, 5], 1), ([0.0, -0.0], 0), ([-0.0, 0.0], 0),
    ([3], 0), ([1, 2, np.inf, np.inf], 2)])
def test_argmax_scan_semantics(orc, values, want):
    assert orc.argmax(np.array(values, np.float32)) == want
    assert orc.argmax(np.array(values, np.float32).astype(F16)) == want


def test_rope_invariants(orc):
    seq, qh, kh, dim = 9, 3, 2, 16
    q = orc.normal((seq, qh, dim), 5, 0, 0.0, 1.0, "f32")
    k = orc.normal((seq, kh, dim), 5, 1, 0.0, 1.0, "f32")
    rq, rk = orc.rope(q, k, qh, kh, dim, 10000.0)
    assert np.array_equal(rq[0], q[0]) and np.array_equal(rk[0], k[0])  # position 0
    half = dim // 2
    for a, b in ((q, rq), (k, rk)):
        n0 = a[..., :half] ** 2 + a[..., half:] ** 2
        n1 = b[..., :half].astype(np.float64) ** 2 + b[..., half:].astype(np.float64) ** 2
        assert np.allclose(n0, n1, rtol=1e-5)
    # against a complex rotation with the same (float-rounded) angles
    p = np.arange(seq, dtype=np.float64)[:, None]
    d = np.arange(half, dtype=np.float64)[None, :]
    angle = (p / np.power(10000.0, 2 * d / dim)).astype(np.float32).astype(np.float64)
    z = (q[..., :half] + 1j * q[..., half:].astype(np.float64)) * np.exp(1j * angle)[:, None, :]
    assert np.allclose(rq[..., :half], z.real, atol=2e-6) and np.allclose(rq[..., half:], z.imag, atol=2e-6)
    # offset p0 equals positions p0..p0+seq-1
    rq2, _ = orc.rope(q, k, qh, kh, dim, 10000.0, offset=3)
    qq = np.concatenate([np.zeros((3, qh, dim), np.float32), q])
    kk = np.concatenate([np.zeros((3, kh, dim), np.float32), k])
    rq3, _ = orc.rope(qq, kk, qh, kh, dim, 10000.0)
    assert np.array_equal(rq2, rq3[3:])


def test_view_add_mul_brute_force(orc):
    B, S, H, D = 2, 5, 3, 8
    x = orc.normal((B, S, H, D), 6, 0, 0.0, 1.0, "f16")
    A = orc.uniform((1, H, 1, D), 6, 1, -1.0, 1.0, "f16")
    M = orc.uniform((B, 1, S, 1), 6, 2, -1.0, 1.0, "f16")
    shape = (B, H, S, D)
    strides = (S * H * D, D, H * D, 1)
    got = orc.view_add_mul(x, shape, strides, 0, A, M)
    want = ((x.transpose(0, 2, 1, 3).astype(np.float32) + A.astype(np.float32)) *
            M.astype(np.float32)).astype(F16)
    assert_bits_equal(got, want, "view add mul")
    got = orc.view_add_mul(x, shape, strides)
    assert_bits_equal(got, x.transpose(0, 2, 1, 3), "view copy")
    # offset slice with stride 2 in the last dim
    flat = orc.uniform((200,), 6, 3, -1, 1)
    got = orc.view_add_mul(flat, (4, 5), (40, 2), 3)
    want = np.lib.stride_tricks.as_strided(flat[3:], (4, 5), (160, 8))
    assert_bits_equal(got, want, "slice")


def test_rng_definition(orc):
    u = orc.uniform((100000,), 9, 3, -1.0, 1.0)
    assert u.min() >= -1.0 and u.max() < 1.0 and abs(u.mean()) < 0.01
    assert np.array_equal(u[500:600], orc.uniform((100,), 9, 3, -1.0, 1.0, first=500))
    n = orc.normal((200000,), 9, 4, 0.0, 3.0, "f32")
    assert abs(n.mean()) < 0.03 and abs(n.std() - 3.0) < 0.03
    assert not np.array_equal(orc.uniform((10,), 9, 3, 0, 1), orc.uniform((10,), 9, 4, 0, 1))
    h = orc.normal((1000,), 9, 4, 0.0, 3.0, "f16")
    assert_bits_equal(h, orc.normal((1000,), 9, 4, 0.0, 3.0, "f32").astype(F16), "f16 = rne(f32)")


_M64 = (1 << 64) - 1
_GAMMA = 0x9E3779B97F4A7C15


def _splitmix64(state: int, k: int) -> int:
    """Output k (k >= 1) of splitmix64 seeded with `state` (Steele, Lea and
    Flood, OOPSLA 2014; Vigna's splitmix64.c): state advances by the golden
    gamma, the output is the mixed state."""
    z = (state + _GAMMA * k) & _M64
    z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & _M64
    z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & _M64
    return z ^ (z >> 31)


def test_rng_bits_pinned_to_published_splitmix64():
    """The fills' generator, pinned without the oracle's code: this file's
    splitmix64 reproduces the published output sequences (seed 1234567:
    6457827717110365317, 3203168211198807973, 9817491932198370423,
    4593380528125082431, 16408922859458223821; seed 0: 0xE220A8397B1DCDAF),
    and orc_rng_bits(seed, stream, i) is output i + 1 of the generator whose
    state is output 2*stream + 1 of the generator seeded `seed` (one
    independent splitmix64 stream per (seed, tensor), indexed by element)."""
    import ctypes
    from oracle import ORACLE_PATH
    assert [_splitmix64(1234567, k) for k in range(1, 6)] == [
        6457827717110365317, 3203168211198807973, 9817491932198370423,
        4593380528125082431, 16408922859458223821]
    assert _splitmix64(0, 1) == 0xE220A8397B1DCDAF
    lib = ctypes.CDLL(ORACLE_PATH)
    lib.orc_rng_bits.argtypes = [ctypes.c_uint64] * 3
    lib.orc_rng_bits.restype = ctypes.c_uint64
    for seed, stream, index in [(0, 0, 0), (1, 2, 3), (5, 9, 123456789), (2**63 + 7, 1, 2**40),
                                (9, 4, 0)]:
        key = _splitmix64(seed, 2 * stream + 1)
        assert lib.orc_rng_bits(seed, stream, index) == _splitmix64(key, index + 1)


def test_rng_value_maps_from_the_definition(orc):
    """U[low, high] = low + (high - low) * (top 24 bits * 2^-24) in f32;
    N(mean, std) by Box-Muller in double on u1 = (bits >> 11 + 1) * 2^-53 in
    (0, 1] and u2 = (second >> 11) * 2^-53 in [0, 1), second = the mixed
    bits ^ 0xD1B54A32D192ED03, then f32, then f16 by RNE. Evaluated here
    with Python's float (C double, the C library's log/cos/sqrt) and
    numpy's f32 rounding, from splitmix64 pinned above."""
    import math
    def mix(z):
        return _splitmix64((z - _GAMMA) & _M64, 1)
    seed, stream, n = 11, 3, 2000
    key = _splitmix64(seed, 2 * stream + 1)
    bits = [_splitmix64(key, i + 1) for i in range(n)]
    low, high = np.float32(-1.5), np.float32(2.25)
    want_u = np.array([low + (high - low) * (np.float32(b >> 40) * np.float32(2.0 ** -24))
                       for b in bits], np.float32)
    assert_bits_equal(orc.uniform((n,), seed, stream, -1.5, 2.25), want_u, "uniform f32")
    mean, std = float(np.float32(0.25)), float(np.float32(3.0))
    want_n = []
    for b in bits:
        second = mix(b ^ 0xD1B54A32D192ED03)
        u1 = ((b >> 11) + 1) * 2.0 ** -53
        u2 = (second >> 11) * 2.0 ** -53
        z = math.sqrt(-2.0 * math.log(u1)) * math.cos(6.283185307179586 * u2)
        want_n.append(np.float32(mean + std * z))
    want_n = np.array(want_n, np.float32)
    assert_bits_equal(orc.normal((n,), seed, stream, 0.25, 3.0, "f32"), want_n, "normal f32")
    assert_bits_equal(orc.normal((n,), seed, stream, 0.25, 3.0, "f16"), want_n.astype(F16),
                      "normal f16")


def test_residual_rms_norm_is_add_then_norm(orc):
    x = orc.normal((8, 64), 10, 0, 0.0, 1.0)
    r = orc.normal((8, 64), 10, 1, 0.0, 1.0)
    w = orc.uniform((64,), 10, 2, 0.5, 1.5, "f16")
    s, y = orc.residual_rms_norm(x, r, w, 1e-6)
    assert_bits_equal(s, orc.add(x, r), "sum")
    assert_bits_equal(y, orc.rms_norm(orc.add(x, r), w, 1e-6), "norm")
