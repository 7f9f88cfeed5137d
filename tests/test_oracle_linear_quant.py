"""The oracle's matmul, linear and Q8_0/Q4_0 functions, pinned on the CPU.

- matmul / linear: bit-exact against the reference build's tensor_matmul_* /
  tensor_linear_* (src/common/tensor_ops.c:163-398, host loops), plus the
  reference's known answers (tests/test_tensor_ops.c:26-60,
  tests/test_tensor_device.c:115-135, tests/test_tensor_compute.c:103-109).
- quantize: byte-exact against the reference build's
  tensor_quantize_linear_weight_f16 (src/common/tensor_quant.c:48-100) on
  blocks chosen to hit every rounding branch, plus the reference test's
  known bytes (tests/test_tensor_quant.c:26-61).
- quantized linear (the CUDA kernel tensor_compute_cuda.cu:216-238, which
  no reference build here can run): the reference test's own tolerance check
  (tests/test_tensor_quant.c:10-24), and closed form: a double-precision dot
  product of the dequantized weights, which the f32 fmaf chain must match to
  within in * 2^-24 * sum|x w| plus half an f16 ulp.
"""
import numpy as np
import pytest

from tests.helpers import assert_bits_equal


@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("shape", [(1, 1, 1), (2, 3, 2), (7, 33, 5), (16, 128, 40)])
def test_matmul_matches_reference(orc, ref, dtype, shape):
    rows, inner, cols = shape
    a = orc.normal((rows, inner), 50, 0, 0.0, 1.0, dtype)
    b = orc.normal((inner, cols), 50, 1, 0.0, 1.0, dtype)
    ok, want, msg = ref.matmul(a, b)
    assert ok, msg
    assert_bits_equal(orc.matmul(a, b), want, "matmul")


@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("with_bias", [False, True])
@pytest.mark.parametrize("xshape,out", [((3,), 4), ((2, 5), 3), ((2, 3, 64), 17), ((9, 100), 33)])
def test_linear_matches_reference(orc, ref, dtype, with_bias, xshape, out):
    x = orc.normal(xshape, 51, 0, 0.0, 1.0, dtype)
    w = orc.normal((out, xshape[-1]), 51, 1, 0.0, 0.5, dtype)
    b = orc.normal((out,), 51, 2, 0.0, 1.0, dtype) if with_bias else None
    ok, want, msg = ref.linear(x, w, b)
    assert ok, msg
    assert_bits_equal(orc.linear(x, w, b), want, "linear")


def test_linear_and_matmul_known_answers(orc):
    # tests/test_tensor_ops.c:26-60
    left = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    right = np.array([[7, 8], [9, 10], [11, 12]], np.float32)
    assert orc.matmul(left, right).tolist() == [[58, 64], [139, 154]]
    w = np.array([[1, 0, -1], [0.5, 2, 1]], np.float32)
    b = np.array([0.25, -0.5], np.float32)
    assert np.allclose(orc.linear(left, w, b), [[-1.75, 7.0], [-1.75, 17.5]], atol=1e-5)
    # tests/test_tensor_device.c:115-135
    x = np.array([[1, 2, 3], [-1, 0.5, 2]], np.float32)
    w = np.array([[2, -1, 0.5], [-2, 3, 1]], np.float32)
    b = np.array([0.25, -0.75], np.float32)
    assert np.allclose(orc.linear(x, w, b), [[1.75, 6.25], [-1.25, 4.75]], atol=1e-5)
    # tests/test_tensor_compute.c:103-109 (linear slot, no bias)
    x = np.arange(1, 7, dtype=np.float32).reshape(2, 3)
    w = np.array([[1, 0, 0], [0, 1, 0]], np.float32)
    assert orc.linear(x, w).tolist() == [[1, 2], [4, 5]]


def quant_inputs(orc, out, inw, seed):
    """f16 weights whose blocks hit each branch of the quantizer: ordinary
    N(0,1) blocks, an all-zero block, a block with a tie between +m and -m
    for the largest magnitude, a block whose scale is subnormal, blocks near
    the f16 maximum, and values that land on exact .5 quotients."""
    w = orc.normal((out, inw), seed, 0, 0.0, 1.0, "f16")
    w[0, :32] = 0
    if out > 1:
        w[1, :32] = np.float16(0.25)
        w[1, 5] = np.float16(-3.0)
        w[1, 9] = np.float16(3.0)            # |-3| first: Q4 keeps the negative one
    if out > 2:
        w[2, :32] = orc.normal((32,), seed, 1, 0.0, 1e-4, "f16")  # scale below 2^-14
    if out > 3:
        w[3, :32] = np.float16(60000.0) * np.sign(orc.normal((32,), seed, 2, 0.0, 1.0, "f32")).astype(np.float16)
        w[3, 0] = np.float16(65504.0)
    if out > 4:
        w[4, :32] = (np.arange(32) - 16).astype(np.float16) / np.float16(8)  # the reference test's row
        w[4, 31] = np.float16(127.0 / 8)     # q = x * 127 / max lands on halves
    return w


@pytest.mark.parametrize("fmt", [1, 2])
@pytest.mark.parametrize("shape", [(1, 32), (5, 64), (8, 96), (33, 256)])
def test_quantize_matches_reference(orc, ref, fmt, shape):
    w = quant_inputs(orc, *shape, seed=52)
    ok, want, msg = ref.quantize(w, fmt)
    assert ok, msg
    got = orc.quantize(w, fmt)
    assert got is not None and got.shape == want.shape
    assert_bits_equal(got, want, f"format {fmt}")


@pytest.mark.parametrize("fmt", [1, 2])
def test_quantize_subnormal_and_tiny_scales(orc, ref, fmt):
    """Blocks whose largest magnitude makes the scale subnormal in f16 or
    smaller than 2^-25 (stored as zero), for every such magnitude class."""
    rows = []
    for e in range(-24, -9):
        row = np.zeros(32, np.float16)
        row[0] = np.float16(2.0 ** e)
        row[1] = np.float16(-(2.0 ** e) * 0.75)
        rows.append(row)
    w = np.stack(rows)
    ok, want, msg = ref.quantize(w, fmt)
    assert ok, msg
    assert_bits_equal(orc.quantize(w, fmt), want, "tiny scales")


def test_quantize_refusals(orc, ref):
    w = np.zeros((2, 33), np.float16)
    ok, _, msg = ref.quantize(w, 1)
    assert not ok and msg == ("quantized linear weight requires a valid format and input width "
                              "divisible by 32")
    assert orc.quantize(w, 1) is None
    w = np.zeros((2, 64), np.float16)
    w[1, 40] = np.float16(np.inf)
    for fmt in (1, 2):
        ok, _, msg = ref.quantize(w, fmt)
        assert not ok and msg == "quantized weights must contain only finite values"
        assert orc.quantize(w, fmt) is None
    w[1, 40] = np.float16(np.nan)
    assert not ref.quantize(w, 1)[0] and orc.quantize(w, 1) is None


def test_quantize_known_bytes(orc):
    # tests/test_tensor_quant.c:26-61: values[i] = ((i % 32) - 16) / 8
    values = ((np.arange(64) % 32) - 16).astype(np.float32) / 8
    w = values.astype(np.float16).reshape(2, 32)
    q8, q4 = orc.quantize(w, 1), orc.quantize(w, 2)
    assert q8.shape == (2, 1, 34) and q4.shape == (2, 1, 18)
    assert q8[0, 0, :2].any() and q4[0, 0, :2].any()
    assert int(np.int8(q8[0, 0, 2])) == -127 and int(np.int8(q8[0, 0, 33])) == 119
    assert q4[0, 0, 2] == 0x80


def test_quant_scale_rounding_closed_form(orc):
    """Normal range: round to nearest even (numpy's binary16 conversion).
    Below 2^-14 the reference's branch (src/common/tensor_quant.c:34-38)
    shifts one place short of IEEE binary16: the stored bits are
    floor(v * 2^25 + 0.5), twice the subnormal value v would round to (the
    quantize tests above pin this against the reference build); below 2^-25
    the scale is a signed zero."""
    f = orc.lib.orc_quant_scale_to_f16
    rng = np.random.default_rng(53)
    normal = np.concatenate([rng.uniform(6.2e-5, 65000, 2000),
                             np.float32(1 + np.arange(1, 64) * 2.0 ** -11)]).astype(np.float32)
    for v in normal:
        assert f(float(v)) == np.float32(v).astype(np.float16).view(np.uint16), v
        assert f(float(-v)) == np.float32(-v).astype(np.float16).view(np.uint16), v
    sub = np.concatenate([rng.uniform(2.0 ** -25, 2.0 ** -14, 2000),
                          (np.arange(1, 2048) + 0.5) * 2.0 ** -25]).astype(np.float32)
    for v in sub:
        want = int(np.floor(np.float64(v) * 2.0 ** 25 + 0.5))
        assert f(float(v)) == want, v
        assert f(float(-v)) == (want | 0x8000), v
    assert f(2.0 ** -26) == 0 and f(-(2.0 ** -26)) == 0x8000
    assert f(70000.0) == 0x7c00


def dequant_exact(x, packed, q8):
    """Double-precision sum_k x_k * scale_b * q_bk."""
    out, blocks = packed.shape[:2]
    scale = packed[:, :, :2].copy().view(np.float16)[:, :, 0].astype(np.float64)
    if q8:
        q = packed[:, :, 2:].view(np.int8).astype(np.float64)
    else:
        lo = (packed[:, :, 2:] & 15).astype(np.float64) - 8
        hi = (packed[:, :, 2:] >> 4).astype(np.float64) - 8
        q = np.concatenate([lo, hi], axis=2)
    wfull = (q * scale[:, :, None]).reshape(out, blocks * 32)
    return x.astype(np.float64).reshape(-1, blocks * 32) @ wfull.T


@pytest.mark.parametrize("fmt", [1, 2])
@pytest.mark.parametrize("rows,inw,out", [(1, 32, 3), (3, 256, 17), (2, 1024, 8)])
def test_quantized_linear_closed_form(orc, fmt, rows, inw, out):
    x = orc.normal((rows, inw), 54, 0, 0.0, 1.0, "f16")
    packed = orc.quantize(orc.normal((out, inw), 54, 1, 0.0, 1.0, "f16"), fmt)
    got = orc.linear_quant(x, packed, fmt == 1).astype(np.float64)
    exact = dequant_exact(x, packed, fmt == 1)
    weight = orc.linear_quant_abs_weight(x, packed, fmt == 1)
    half_ulp = np.spacing(np.abs(exact).astype(np.float16)).astype(np.float64) / 2
    bound = inw * 2.0 ** -24 * weight + half_ulp
    assert (np.abs(got - exact) <= bound).all()


def test_quantized_linear_reference_check(orc):
    """tests/test_tensor_quant.c:10-24 and :62-83: x[i] = 0.125 (i - 12),
    within 0.02 of the sequential f32 sum."""
    values = ((np.arange(64) % 32) - 16).astype(np.float32) / 8
    w = values.astype(np.float16).reshape(2, 32)
    x = (0.125 * (np.arange(32) - 12)).astype(np.float16).reshape(1, 32)
    for fmt in (1, 2):
        packed = orc.quantize(w, fmt)
        got = orc.linear_quant(x, packed, fmt == 1).astype(np.float32)
        expected = dequant_exact(x, packed, fmt == 1)
        assert np.abs(got - expected).max() <= 0.02


@pytest.mark.parametrize("fmt", [1, 2])
def test_quantized_linear_non_finite_closed_form(orc, fmt):
    """x = +-Inf / NaN through the fmaf chain: IEEE rules fix every output.
    One block, weights w_k = (k - 12) / 8 quantized (so q_12 = 0): an Inf at
    k = 12 meets a zero weight (NaN); an Inf at k = 20 gives the sign of x
    times the sign of its weight; +Inf at 20 and 21 (weights of one sign)
    stays +Inf; +Inf at 20 and -Inf at 21 is NaN; a NaN anywhere is NaN."""
    w = ((np.arange(32) - 12) / 8).astype(np.float16).reshape(1, 32)
    packed = orc.quantize(w, fmt)
    cases = [({12: np.inf}, "nan"), ({20: np.inf}, "+inf"), ({20: -np.inf}, "-inf"),
             ({4: np.inf}, "-inf"), ({20: np.inf, 21: np.inf}, "+inf"),
             ({20: np.inf, 21: -np.inf}, "nan"), ({7: np.nan}, "nan")]
    for cells, expect in cases:
        x = np.full((1, 32), 0.5, np.float16)
        for k, v in cells.items():
            x[0, k] = v
        y = float(orc.linear_quant(x, packed, fmt == 1)[0, 0])
        got = "nan" if np.isnan(y) else ("+inf" if y == np.inf else "-inf" if y == -np.inf else "finite")
        assert got == expect, (fmt, cells, y)
