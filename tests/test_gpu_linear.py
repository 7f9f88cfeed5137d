"""Linear, matmul and Q8_0/Q4_0 on the GPU against the CPU oracle.

The oracle follows the reference's host loops (src/common/tensor_ops.c:
163-398, one f32 sum per output in input order, started at the bias) and
the CUDA quantized-linear kernel (tensor_compute_cuda.cu:216-238). The GPU
sums in another order (hipBLASLt MFMA tiles; v_dot2 pairs per 32-weight
block), so outputs are compared against W = sum_k |x_k w_k| (+ |bias|):
  f32: |got - want| <= 1e-5 * W          (north-star f32 reduction bound)
  f16: within 1 f16 ulp of the oracle, or |got - want| <= 2e-3 * W
       (north-star f16 reduction bound).
The quantizer is integer/byte work and must match byte for byte."""
import ctypes
import os

import numpy as np
import pytest

from tests.helpers import assert_bits_equal, f16_ulps

pytestmark = pytest.mark.gpu


def check(got, want, weight, dtype, what):
    g, w = got.astype(np.float64), want.astype(np.float64)
    err = np.abs(g - w)
    if dtype == "f32":
        ok = err <= 1e-5 * weight + 1e-30
    else:
        ok = (f16_ulps(got, want) <= 1) | (err <= 2e-3 * weight)
    bad = np.flatnonzero(~ok)
    assert bad.size == 0, (f"{what}: {bad.size} of {ok.size} outside the bound; worst "
                           f"{float((err / np.maximum(weight, 1e-30)).max()):.3g} of sum|xw|")


def abs_weight(x, w, bias=None):
    xs = np.abs(x.astype(np.float64)).reshape(-1, x.shape[-1])
    out = xs @ np.abs(w.astype(np.float64)).T
    if bias is not None:
        out = out + np.abs(bias.astype(np.float64))
    return out.reshape(x.shape[:-1] + (w.shape[0],))


# ---- matmul / linear ---------------------------------------------------------

@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("shape", [(2, 3, 2), (37, 129, 65), (1, 4096, 3), (256, 256, 256), (5, 0, 4)])
def test_matmul(sdk, orc, dtype, shape):
    rows, inner, cols = shape
    a = orc.normal((rows, inner), 60, 0, 0.0, 1.0, dtype)
    b = orc.normal((inner, cols), 60, 1, 0.0, 1.0, dtype)
    out = sdk.tensor(dtype, (rows, cols), device=False)
    sdk.call(f"tensor_matmul_{dtype}", sdk.from_numpy(a, device=False),
             sdk.from_numpy(b, device=False), out)
    got = out.download()
    if inner == 0:
        assert (got == 0).all()
        return
    weight = np.abs(a.astype(np.float64)) @ np.abs(b.astype(np.float64))
    check(got, orc.matmul(a, b), weight, dtype, f"matmul {shape}")


LINEAR_SHAPES = [  # input shape, out features
    ((1, 64), 32),          # decode row
    ((3, 100), 77),         # widths that are not tile multiples
    ((2, 5, 256), 96),      # rank-3 input
    ((512, 1024), 768),     # prefill
    ((17,), 40),            # rank-1 input
    # the GEMV path (1-4 rows, in a whole number of 16-byte vectors): tail
    # vectors only, odd output counts; whole unrolled steps; steps and a tail
    ((4, 520), 130),
    ((2, 2048), 33),
    ((1, 8200), 9),
]


@pytest.mark.parametrize("device", [True, False])
@pytest.mark.parametrize("with_bias", [False, True])
@pytest.mark.parametrize("dtype", ["f32", "f16"])
@pytest.mark.parametrize("xshape,out", LINEAR_SHAPES)
def test_linear(sdk, orc, dtype, with_bias, device, xshape, out):
    x = orc.normal(xshape, 61, 0, 0.0, 1.0, dtype)
    w = orc.normal((out, xshape[-1]), 61, 1, 0.0, 0.5, dtype)
    b = orc.normal((out,), 61, 2, 0.0, 1.0, dtype) if with_bias else None
    y = sdk.tensor(dtype, xshape[:-1] + (out,), device=device)
    sdk.call(f"tensor_linear_{dtype}", sdk.from_numpy(x, device=device),
             sdk.from_numpy(w, device=device),
             None if b is None else sdk.from_numpy(b, device=device), y)
    check(y.download(), orc.linear(x, w, b), abs_weight(x, w, b), dtype,
          f"linear {xshape}x{out} bias={with_bias} device={device}")


def test_linear_known_answers(sdk):
    # tests/test_tensor_ops.c:26-60 (host) and tests/test_tensor_device.c:115-135 (device)
    left = np.array([[1, 2, 3], [4, 5, 6]], np.float32)
    right = np.array([[7, 8], [9, 10], [11, 12]], np.float32)
    out = sdk.tensor("f32", (2, 2), device=False)
    sdk.call("tensor_matmul_f32", sdk.from_numpy(left, device=False),
             sdk.from_numpy(right, device=False), out)
    assert np.allclose(out.download(), [[58, 64], [139, 154]], atol=1e-5, rtol=0)
    w = np.array([[1, 0, -1], [0.5, 2, 1]], np.float32)
    b = np.array([0.25, -0.5], np.float32)
    out = sdk.tensor("f32", (2, 2), device=False)
    sdk.call("tensor_linear_f32", sdk.from_numpy(left, device=False),
             sdk.from_numpy(w, device=False), sdk.from_numpy(b, device=False), out)
    assert np.allclose(out.download(), [[-1.75, 7.0], [-1.75, 17.5]], atol=1e-5, rtol=0)
    x = np.array([[1, 2, 3], [-1, 0.5, 2]], np.float32)
    w = np.array([[2, -1, 0.5], [-2, 3, 1]], np.float32)
    b = np.array([0.25, -0.75], np.float32)
    y = sdk.tensor("f32", (2, 2))
    sdk.call("tensor_linear_f32", sdk.from_numpy(x), sdk.from_numpy(w), sdk.from_numpy(b), y)
    assert np.allclose(y.download(), [[1.75, 6.25], [-1.25, 4.75]], atol=1e-5, rtol=0)


def test_device_linear_validation(sdk, monkeypatch):
    x = sdk.tensor("f32", (2, 3))
    w = sdk.tensor("f32", (4, 3))
    y = sdk.tensor("f32", (2, 4))
    host_w = sdk.tensor("f32", (4, 3), device=False)
    cases = [
        ((x, host_w, None, y), "device linear requires all operands on one device with F32 "
                               "dtype and compatible ranks"),
        ((x, w, sdk.tensor("f32", (5,)), y), "device linear dimensions do not match"),
        ((sdk.tensor("f32", (2, 5, 3)), w, None, sdk.tensor("f32", (2, 4, 4))),
         "device linear leading dimensions do not match"),
        ((sdk.tensor("f32", (0, 3)), w, None, sdk.tensor("f32", (0, 4))),
         "device linear backend operation failed"),
    ]
    for args, message in cases:
        ok, msg = sdk.try_call("tensor_linear_f32", *args)
        assert not ok and msg == message, (msg, message)
    ok, msg = sdk.try_call("tensor_linear_f16", x, w, None, y)
    assert not ok and msg == ("device linear requires all operands on one device with F16 dtype "
                              "and compatible ranks")
    # a backend selection naming another backend leaves no device linear
    monkeypatch.setenv("TENSOR_BACKEND", "cuda")
    ok, msg = sdk.try_call("tensor_linear_f32", x, w, None, y)
    assert not ok and msg == "device linear backend operation failed"


# ---- compute-table slots -----------------------------------------------------

def backend(sdk):
    from tests.test_gpu_vtable import Table
    return ctypes.cast(sdk.lib.tensor_compute_hip_backend(), ctypes.POINTER(Table)).contents


P, Z = ctypes.c_void_p, ctypes.c_size_t


def slot(sdk, name, *args):
    addr = getattr(backend(sdk), name)
    assert addr, f"slot {name} is NULL"
    return ctypes.CFUNCTYPE(ctypes.c_int, *args)(addr)


def release_cache(sdk):
    ctypes.CFUNCTYPE(None)(backend(sdk).release_cache)()


def test_linear_slot_known_answer(sdk):
    # tests/test_tensor_compute.c:103-109
    x = np.arange(1, 7, dtype=np.float32)
    w = np.array([1, 0, 0, 0, 1, 0], np.float32)
    y = np.zeros(4, np.float32)
    assert slot(sdk, "linear_f32", P, P, P, Z, Z, Z)(x.ctypes.data, w.ctypes.data, y.ctypes.data,
                                                     2, 3, 2)
    assert np.allclose(y, [1, 2, 4, 5], atol=1e-5, rtol=0)
    release_cache(sdk)


@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_linear_slots(sdk, orc, dtype):
    rows, inw, out = 9, 192, 70
    x = orc.normal((rows, inw), 62, 0, 0.0, 1.0, dtype)
    w = orc.normal((out, inw), 62, 1, 0.0, 0.5, dtype)
    want, weight = orc.linear(x, w), abs_weight(x, w)
    y = np.zeros((rows, out), x.dtype)
    fn = slot(sdk, f"linear_{dtype}", P, P, P, Z, Z, Z)
    assert fn(x.ctypes.data, w.ctypes.data, y.ctypes.data, rows, inw, out)
    check(y, want, weight, dtype, "host slot")
    # the weight stays cached per host address until release_cache
    w2 = w.copy()
    w[:] = 0
    y2 = np.zeros_like(y)
    assert fn(x.ctypes.data, w.ctypes.data, y2.ctypes.data, rows, inw, out)
    check(y2, want, weight, dtype, "host slot, cached weight")
    release_cache(sdk)
    assert fn(x.ctypes.data, w.ctypes.data, y2.ctypes.data, rows, inw, out)
    assert (y2 == 0).all()
    release_cache(sdk)
    assert fn(x.ctypes.data, w2.ctypes.data, y2.ctypes.data, 0, inw, out) == 0
    # device slot
    tx, tw, ty = sdk.from_numpy(x), sdk.from_numpy(w2), sdk.tensor(dtype, (rows, out))
    fn = slot(sdk, f"linear_{dtype}_device", P, P, P, Z, Z, Z)
    assert fn(tx.device_ptr(), tw.device_ptr(), ty.device_ptr(), rows, inw, out)
    check(ty.download(), want, weight, dtype, "device slot")
    release_cache(sdk)


def test_rms_norm_linear_slot(sdk, orc):
    rows, inw, out, eps = 6, 128, 40, 1e-6
    x = orc.normal((rows, inw), 63, 0, 0.0, 1.0, "f32")
    s = orc.uniform((inw,), 63, 1, 0.5, 1.5, "f32")
    w = orc.normal((out, inw), 63, 2, 0.0, 0.5, "f32")
    norm = np.zeros_like(x)
    y = np.zeros((rows, out), np.float32)
    fn = slot(sdk, "rms_norm_linear_f32", P, P, P, P, P, Z, Z, Z, ctypes.c_float)
    assert fn(x.ctypes.data, s.ctypes.data, norm.ctypes.data, w.ctypes.data, y.ctypes.data,
              rows, inw, out, eps)
    want_norm = orc.rms_norm(x, s, eps)
    assert np.abs(norm - want_norm).max() <= 1e-6 * np.abs(want_norm).max()
    check(y, orc.linear(want_norm, w), abs_weight(want_norm, w), "f32", "rms_norm_linear")
    release_cache(sdk)


def test_mlp_and_qkv_slots(sdk, orc):
    rows, inw, mid, out = 5, 64, 96, 48
    x = orc.normal((rows, inw), 64, 0, 0.0, 1.0, "f16")
    w1 = orc.normal((mid, inw), 64, 1, 0.0, 0.3, "f16")
    b1 = orc.normal((mid,), 64, 2, 0.0, 0.3, "f16")
    w2 = orc.normal((out, mid), 64, 3, 0.0, 0.3, "f16")
    b2 = orc.normal((out,), 64, 4, 0.0, 0.3, "f16")
    y = np.zeros((rows, out), np.float16)
    fn = slot(sdk, "mlp_f16", P, P, P, P, P, P, Z, Z, Z, Z)
    assert fn(x.ctypes.data, w1.ctypes.data, b1.ctypes.data, w2.ctypes.data, b2.ctypes.data,
              y.ctypes.data, rows, inw, mid, out)
    # the CUDA composition: f16 linear, f16 bias+GELU, f16 linear, f16 bias
    act = orc.bias_add(orc.linear(x, w1), b1, gelu=True)
    want = orc.linear(act, w2, b2)
    check(y, want, abs_weight(act, w2, b2), "f16", "mlp")
    q, k, v = (np.zeros((rows, mid), np.float16) for _ in range(3))
    wq, wk, wv = (orc.normal((mid, inw), 65, i, 0.0, 0.3, "f16") for i in range(3))
    bq = orc.normal((mid,), 65, 3, 0.0, 0.3, "f16")
    fn = slot(sdk, "qkv_f16", *([P] * 10), Z, Z, Z)
    assert fn(x.ctypes.data, wq.ctypes.data, wk.ctypes.data, wv.ctypes.data, bq.ctypes.data,
              None, None, q.ctypes.data, k.ctypes.data, v.ctypes.data, rows, inw, mid)
    check(q, orc.linear(x, wq, bq), abs_weight(x, wq, bq), "f16", "qkv q")
    check(k, orc.linear(x, wk), abs_weight(x, wk), "f16", "qkv k")
    check(v, orc.linear(x, wv), abs_weight(x, wv), "f16", "qkv v")
    release_cache(sdk)


# ---- Q8_0 / Q4_0 -------------------------------------------------------------

def quant_weights(orc, out, inw, seed):
    from tests.test_oracle_linear_quant import quant_inputs
    return quant_inputs(orc, out, inw, seed)


@pytest.mark.parametrize("fmt", [1, 2])
@pytest.mark.parametrize("shape", [(1, 32), (5, 64), (33, 256), (300, 4096)])
def test_quantize_matches_oracle(sdk, orc, fmt, shape):
    w = quant_weights(orc, *shape, seed=66)
    ok, packed, msg = sdk.quantize(w, fmt)
    assert ok, msg
    assert_bits_equal(packed, orc.quantize(w, fmt), f"quantize format {fmt} {shape}")


@pytest.mark.parametrize("fmt", [1, 2])
def test_quantize_rounding_edges(sdk, orc, fmt):
    """Every f16 magnitude class of block maximum (subnormal scales stored the
    reference's way), ties of +-max, and exact .5 quotients."""
    rows = []
    for e in range(-24, 16):
        for frac in (1.0, 1.5, 1.75):
            row = orc.normal((32,), 67, e + 40, 0.0, 1.0, "f32")
            row = row / np.abs(row).max() * (2.0 ** e) * frac
            rows.append(np.clip(row, -65504, 65504).astype(np.float16))
    tie = np.full(32, 0.5, np.float16)
    tie[3], tie[7] = -2.0, 2.0
    rows.append(tie)
    halves = (np.arange(32) - 15.5).astype(np.float16)
    rows.append(halves)
    w = np.stack(rows)
    ok, packed, msg = sdk.quantize(w, fmt)
    assert ok, msg
    assert_bits_equal(packed, orc.quantize(w, fmt), "rounding edges")


def test_quantize_rejects_non_finite(sdk):
    w = np.zeros((3, 64), np.float16)
    w[2, 63] = np.float16(np.inf)
    for fmt in (1, 2):
        ok, packed, msg = sdk.quantize(w, fmt)
        assert not ok and packed is None
        assert msg == "quantized weights must contain only finite values"
    w[2, 63] = np.float16(np.nan)
    assert not sdk.quantize(w, 1)[0]


def test_quantize_known_bytes(sdk):
    # tests/test_tensor_quant.c:26-61
    w = (((np.arange(64) % 32) - 16).astype(np.float32) / 8).astype(np.float16).reshape(2, 32)
    _, q8, _ = sdk.quantize(w, 1)
    _, q4, _ = sdk.quantize(w, 2)
    assert q8.shape == (2, 1, 34) and q4.shape == (2, 1, 18)
    assert int(np.int8(q8[0, 0, 2])) == -127 and int(np.int8(q8[0, 0, 33])) == 119
    assert q4[0, 0, 2] == 0x80


QUANT_SHAPES = [  # rows, in, out
    (1, 32, 1), (1, 64, 7), (1, 2048, 256), (2, 4096, 130), (3, 96, 33), (4, 1024, 64),
    (5, 512, 40), (8, 256, 16), (17, 2080, 24), (64, 768, 96), (1, 8192, 512),
    (6, 8192, 100), (33, 544, 50),
    # one row: a block's 4 waves split the 64-block chunks -- wave 1 with a
    # partial chunk; 6 chunks, so waves 0 and 1 take two (the second partial)
    (1, 2112, 5), (1, 10336, 9),
    # two rows: Q4_0 splits the chunks the same way, Q8_0 does not
    (2, 10336, 9), (2, 2112, 70),
    # the MFMA kernel (2+ rows): one weight block and one output; 16 rows over
    # 8 full chunks and a 1-block chunk, ragged tiles; a 4-row second group
    (2, 32, 1), (16, 4128, 70), (20, 1056, 130),
    # the MFMA kernel at in a multiple of 2048 (4, 8 and 12 16-block chunks
    # per row; Q8_0 from 7 rows on line windows); Q4_0 with 3 rows takes
    # one-wave blocks of 32-block chunks
    (3, 2048, 17), (16, 4096, 70), (20, 6144, 130), (7, 2048, 33),
    # drawn once with numpy's default_rng(5): rows 1-40, in up to 16384
    (16, 13216, 68), (17, 7712, 1546), (8, 4704, 2938), (1, 4576, 1150), (8, 6720, 394),
    (1, 16384, 573), (3, 7136, 790), (40, 2912, 2693), (4, 10304, 1479), (1, 15744, 1667),
]


@pytest.mark.parametrize("fmt", [1, 2])
@pytest.mark.parametrize("shape", QUANT_SHAPES)
def test_quantized_linear(sdk, orc, fmt, shape):
    rows, inw, out = shape
    x = orc.normal((rows, inw), 68, 0, 0.0, 1.0, "f16")
    packed = orc.quantize(orc.normal((out, inw), 68, 1, 0.0, 1.0, "f16"), fmt)
    y = sdk.tensor("f16", (rows, out))
    name = "tensor_linear_q8_0_f16" if fmt == 1 else "tensor_linear_q4_0_f16"
    sdk.call(name, sdk.from_numpy(x), sdk.from_numpy(packed, dtype="u8"), y)
    check(y.download(), orc.linear_quant(x, packed, fmt == 1),
          orc.linear_quant_abs_weight(x, packed, fmt == 1), "f16", f"{name} {shape}")


@pytest.mark.parametrize("fmt", [1, 2])
@pytest.mark.parametrize("shape", [(1, 2080, 96), (1, 10336, 9), (2, 1056, 40), (4, 4128, 70),
                                   (16, 2080, 33), (20, 1056, 130)])
def test_quantized_linear_non_finite(sdk, orc, fmt, shape):
    """+-Inf and NaN in x follow the reference's sum of x * (scale q)
    (tensor_compute_cuda.cu:216-238): +-Inf where every non-finite x meets a
    non-zero weight and the infinities agree in sign, NaN for a zero weight
    (Inf * 0), opposite infinities or a NaN input. Shapes cover the split
    one-row GEMV (an Inf in a partial last chunk, whose lanes past the end
    read that block's x), the two-row GEMV and the MFMA kernel (a 20-row
    input leaves a 4-row second tile). Rows with finite x keep the usual
    bound."""
    rows, inw, out = shape
    x = orc.normal((rows, inw), 69, 0, 0.0, 1.0, "f16").copy()
    w = orc.normal((out, inw), 69, 1, 0.0, 1.0, "f16").copy()
    planted = {0: [(inw - 5, np.inf)]}
    if rows > 1:
        planted[1] = [(3, -np.inf)]
    if rows > 2:
        planted[2] = [(40, np.inf), (41, -np.inf)]
    if rows > 3:
        planted[rows - 1] = [(inw // 2, np.nan)]
    for r, cells in planted.items():
        for k, value in cells:
            x[r, k] = value
    w[: min(out, 6) : 5, inw - 5] = 0.0   # Inf * 0 in row 0
    w[1 % out, 3] = 0.0
    packed = orc.quantize(w, fmt)
    y = sdk.tensor("f16", (rows, out))
    name = "tensor_linear_q8_0_f16" if fmt == 1 else "tensor_linear_q4_0_f16"
    sdk.call(name, sdk.from_numpy(x), sdk.from_numpy(packed, dtype="u8"), y)
    got = y.download().astype(np.float64)
    want = orc.linear_quant(x, packed, fmt == 1).astype(np.float64)
    for cls in (np.isnan, np.isposinf, np.isneginf):
        assert np.array_equal(cls(got), cls(want)), f"{name} {shape}: {cls.__name__} pattern"
    assert np.isnan(want).any() and np.isinf(want).any(), "the case must produce both outcomes"
    finite = [r for r in range(rows) if r not in planted]
    if finite:
        xf = x[finite]
        check(got[finite].astype(np.float16), want[finite].astype(np.float16),
              orc.linear_quant_abs_weight(xf, packed, fmt == 1), "f16", f"{name} {shape} finite rows")


@pytest.mark.parametrize("fmt", [1, 2])
@pytest.mark.parametrize("rows", [3, 5, 8])
def test_quantized_linear_weight_offsets(sdk, orc, fmt, rows):
    """The MFMA kernel (4-wave blocks; one-wave blocks for Q4_0 with 3 rows;
    for Q8_0 with 8 rows the line windows, each 128-byte line loaded once and
    a chunk's first bytes carried over from the chunk before) with the
    packed weights at byte offsets 4 .. 124 from a 256-byte boundary: every
    offset moves the chunks within their 16-byte segments and 128-byte
    lines. The decode and the sums do not depend on the offset, so every
    result equals the aligned one bit for bit."""
    inw, out = 2048, 37
    x = orc.normal((rows, inw), 70, 0, 0.0, 1.0, "f16")
    packed = orc.quantize(orc.normal((out, inw), 70, 1, 0.0, 1.0, "f16"), fmt)
    want = orc.linear_quant(x, packed, fmt == 1)
    weight = orc.linear_quant_abs_weight(x, packed, fmt == 1)
    tag = "q8_0" if fmt == 1 else "q4_0"
    dev = slot(sdk, f"linear_{tag}_f16_device", P, P, P, Z, Z, Z)
    tx = sdk.from_numpy(x)
    ty = sdk.tensor("f16", (rows, out))
    aligned = None
    for off in (0, 4, 12, 16, 64, 100, 124):
        tw = sdk.from_numpy(np.concatenate([np.zeros(off, np.uint8), packed.ravel()]), dtype="u8")
        assert tw.device_ptr() % 256 == 0
        assert dev(tx.device_ptr(), tw.device_ptr() + off, ty.device_ptr(), rows, inw, out)
        got = ty.download()
        if aligned is None:
            check(got, want, weight, "f16", f"{tag} weights at offset 0")
            aligned = got
        else:
            assert_bits_equal(got, aligned, f"{tag} weights at offset {off}")


def test_quantized_linear_reference_check(sdk, orc):
    """tests/test_tensor_quant.c:62-83 on the device path."""
    w = (((np.arange(64) % 32) - 16).astype(np.float32) / 8).astype(np.float16).reshape(2, 32)
    x = (0.125 * (np.arange(32) - 12)).astype(np.float16).reshape(1, 32)
    for fmt, name in ((1, "tensor_linear_q8_0_f16"), (2, "tensor_linear_q4_0_f16")):
        packed = orc.quantize(w, fmt)
        y = sdk.tensor("f16", (1, 2))
        sdk.call(name, sdk.from_numpy(x), sdk.from_numpy(packed, dtype="u8"), y)
        from tests.test_oracle_linear_quant import dequant_exact
        assert np.abs(y.download().astype(np.float64) - dequant_exact(x, packed, fmt == 1)).max() <= 0.02


def test_quantized_linear_validation(sdk, orc):
    x = sdk.tensor("f16", (2, 64))
    w8 = sdk.tensor("u8", (4, 2, 34))
    y = sdk.tensor("f16", (2, 4))
    cases = [
        (("tensor_linear_q8_0_f16", x, sdk.tensor("u8", (4, 2, 34), device=False), y),
         "quantized linear requires device-resident FP16 input/output and packed U8 weights"),
        (("tensor_linear_q4_0_f16", x, w8, y), "quantized linear shapes are incompatible"),
        (("tensor_linear_q8_0_f16", sdk.tensor("f16", (2, 48)), sdk.tensor("u8", (4, 1, 34)), y),
         "quantized linear shapes are incompatible"),
        (("tensor_linear_q8_0_f16", sdk.tensor("f16", (2, 3, 64)), w8, sdk.tensor("f16", (2, 4, 4))),
         "quantized linear leading dimensions do not match"),
        (("tensor_linear_q8_0_f16", sdk.tensor("f16", (0, 64)), w8, sdk.tensor("f16", (0, 4))),
         "quantized linear GPU kernel is unavailable"),
        (("tensor_linear_q8_0_f16", sdk.tensor("f16", (2, 0)), sdk.tensor("u8", (4, 0, 34)), y),
         "quantized linear GPU kernel is unavailable"),
    ]
    for args, message in cases:
        ok, msg = sdk.try_call(*args)
        assert not ok and msg == message, (args[0], msg)


@pytest.mark.parametrize("fmt", [1, 2])
def test_quantized_slots(sdk, orc, fmt):
    """Host slot (weight cached per host address) and device slot, including
    device addresses that are only 2-byte aligned (scalar kernel)."""
    rows, inw, out = 3, 160, 21
    x = orc.normal((rows, inw), 69, 0, 0.0, 1.0, "f16")
    packed = orc.quantize(orc.normal((out, inw), 69, 1, 0.0, 1.0, "f16"), fmt)
    want = orc.linear_quant(x, packed, fmt == 1)
    weight = orc.linear_quant_abs_weight(x, packed, fmt == 1)
    tag = "q8_0" if fmt == 1 else "q4_0"
    host = slot(sdk, f"linear_{tag}_f16", P, P, P, Z, Z, Z)
    y = np.zeros((rows, out), np.float16)
    assert host(x.ctypes.data, packed.ctypes.data, y.ctypes.data, rows, inw, out)
    check(y, want, weight, "f16", "host slot")
    assert host(x.ctypes.data, packed.ctypes.data, y.ctypes.data, rows, 33, out) == 0
    release_cache(sdk)
    dev = slot(sdk, f"linear_{tag}_f16_device", P, P, P, Z, Z, Z)
    tx, tw, ty = sdk.from_numpy(x), sdk.from_numpy(packed, dtype="u8"), sdk.tensor("f16", (rows, out))
    assert dev(tx.device_ptr(), tw.device_ptr(), ty.device_ptr(), rows, inw, out)
    check(ty.download(), want, weight, "f16", "device slot")
    # 2-byte offsets: weights at an address that is 2 mod 4, x not 16-byte aligned
    tx2 = sdk.from_numpy(np.concatenate([np.zeros(1, np.float16), x.ravel()]))
    tw2 = sdk.from_numpy(np.concatenate([np.zeros(2, np.uint8), packed.ravel()]), dtype="u8")
    ty2 = sdk.tensor("f16", (rows, out))
    assert dev(tx2.device_ptr() + 2, tw2.device_ptr() + 2, ty2.device_ptr(), rows, inw, out)
    check(ty2.download(), want, weight, "f16", "device slot, unaligned")
    # the scalar kernel runs the reference's chain operation for operation
    assert_bits_equal(ty2.download(), want, "device slot, unaligned: the reference's chain")
    assert dev(tx.device_ptr(), tw.device_ptr(), ty.device_ptr(), 0, inw, out) == 0
