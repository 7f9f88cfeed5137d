"""Row reductions on the GPU against the CPU oracle: RMSNorm, fused residual +
RMSNorm, LayerNorm, softmax (causal and plain, with the reference's special
rows), row sum and row max.

Bar: f16 outputs within 1 ulp of the oracle (the sum order differs), f32
within 1e-5 relative; row max bit-exact; row sums within 1e-5 * sum|x|.
Widths cover the one-wave register path, the four-wave LDS path and the
streaming path."""
import numpy as np
import pytest

from tests.helpers import assert_bits_equal, assert_f16_ulps, assert_f32_rel, f16_ulps

pytestmark = pytest.mark.gpu
F16 = np.float16

# (rows, width): register path 1 wave (<= 4096 f16), 4 waves (<= 16384), stream
SHAPES = [(1, 8), (3, 64), (37, 2048), (5, 1000), (4, 4096), (3, 8192), (2, 16384),
          (2, 1001), (2, 20000), (16384, 2048)]


def tensors(sdk, arrays, device=True):
    return [None if a is None else sdk.from_numpy(a, device=device) for a in arrays]


@pytest.mark.parametrize("device", [True, False])
@pytest.mark.parametrize("rows,width", SHAPES)
def test_rms_norm_f16(sdk, orc, rows, width, device):
    x = orc.normal((rows, width), 21, 0, 0.0, 1.0)
    w = orc.uniform((width,), 21, 1, 0.5, 1.5, "f16")
    tx, tw = tensors(sdk, [x, w], device)
    ty = sdk.tensor("f16", x.shape, device)
    sdk.call("tensor_rms_norm_f16", tx, tw, 1e-6, ty)
    assert_f16_ulps(ty.download(), orc.rms_norm(x, w, 1e-6), 1, "rms f16")


@pytest.mark.parametrize("rows,width", SHAPES[:8])
def test_rms_norm_f32(sdk, orc, rows, width):
    x = orc.normal((rows, width), 22, 0, 0.0, 1.0, "f32")
    w = orc.uniform((width,), 22, 1, 0.5, 1.5)
    tx, tw = tensors(sdk, [x, w])
    ty = sdk.tensor("f32", x.shape)
    sdk.call("tensor_rms_norm_f32", tx, tw, 1e-6, ty)
    assert_f32_rel(ty.download(), orc.rms_norm(x, w, 1e-6), 1e-5, "rms f32")


@pytest.mark.parametrize("dtype,rows,width", [
    ("f16", 8192, 2048),    # four waves per row, exact rows
    ("f16", 8200, 2056),    # four waves per row, 257 vectors (two per lane, ragged)
    ("f16", 9000, 64),      # many narrow rows: one wave per row
    ("f32", 8192, 1024),    # four waves per row, f32
    ("f16", 8191, 2048),    # just under the row threshold: one wave per row
])
def test_rms_norm_many_rows(sdk, orc, dtype, rows, width):
    """From 8192 rows of at least 256 vectors RMSNorm launches four waves per
    row; both sides of the rule, exact and ragged rows, f16 and f32, plain and
    with the residual."""
    if dtype == "f16":
        x = orc.normal((rows, width), 24, 0, 0.0, 1.0)
        r = orc.normal((rows, width), 24, 1, 0.0, 1.0)
        w = orc.uniform((width,), 24, 2, 0.5, 1.5, "f16")
    else:
        x = orc.normal((rows, width), 24, 0, 0.0, 1.0, "f32")
        w = orc.uniform((width,), 24, 2, 0.5, 1.5)
    tx, tw = tensors(sdk, [x, w])
    ty = sdk.tensor(dtype, x.shape)
    sdk.call(f"tensor_rms_norm_{dtype}", tx, tw, 1e-6, ty)
    if dtype == "f16":
        assert_f16_ulps(ty.download(), orc.rms_norm(x, w, 1e-6), 1, "rms f16")
        tr = sdk.from_numpy(r)
        ts, tn = sdk.tensor("f16", x.shape), sdk.tensor("f16", x.shape)
        sdk.call("tensor_residual_rms_norm_f16", tx, tr, tw, 1e-6, ts, tn)
        s_ref, y_ref = orc.residual_rms_norm(x, r, w, 1e-6)
        assert_bits_equal(ts.download(), s_ref, "sum")
        assert_f16_ulps(tn.download(), y_ref, 1, "norm of sum")
    else:
        assert_f32_rel(ty.download(), orc.rms_norm(x, w, 1e-6), 1e-5, "rms f32")


def test_rms_norm_known_answer(sdk):
    # reference tests/test_tensor_ops.c:84-97
    tx = sdk.from_numpy(np.array([[3, 4], [0, 2]], np.float32))
    tw = sdk.from_numpy(np.array([2, 0.5], np.float32))
    ty = sdk.tensor("f32", (2, 2))
    sdk.call("tensor_rms_norm_f32", tx, tw, 0.0, ty)
    assert np.allclose(ty.download().ravel(), [1.69705627, 0.56568545, 0.0, 0.70710678], atol=1e-5)


@pytest.mark.parametrize("device", [True, False])
@pytest.mark.parametrize("rows,width", [(4096, 2048), (3, 1000), (2, 1001), (2, 8192)])
def test_residual_rms_norm_f16(sdk, orc, rows, width, device):
    x = orc.normal((rows, width), 23, 0, 0.0, 1.0)
    r = orc.normal((rows, width), 23, 1, 0.0, 1.0)
    w = orc.uniform((width,), 23, 2, 0.5, 1.5, "f16")
    tx, tr, tw = tensors(sdk, [x, r, w], device)
    ts, ty = sdk.tensor("f16", x.shape, device), sdk.tensor("f16", x.shape, device)
    sdk.call("tensor_residual_rms_norm_f16", tx, tr, tw, 1e-6, ts, ty)
    s_ref, y_ref = orc.residual_rms_norm(x, r, w, 1e-6)
    assert_bits_equal(ts.download(), s_ref, "sum")
    assert_f16_ulps(ty.download(), y_ref, 1, "norm of sum")


@pytest.mark.parametrize("dtype", ["f16", "f32"])
@pytest.mark.parametrize("rows,width", [(3, 64), (37, 2048), (2, 1001), (3, 8192)])
@pytest.mark.parametrize("affine", ["none", "scale", "bias", "both"])
def test_layer_norm(sdk, orc, dtype, rows, width, affine):
    x = orc.normal((rows, width), 24, 0, 0.5, 2.0, dtype)
    s = orc.uniform((width,), 24, 1, 0.5, 1.5, dtype) if affine in ("scale", "both") else None
    b = orc.uniform((width,), 24, 2, -1.0, 1.0, dtype) if affine in ("bias", "both") else None
    tx, ts, tb = tensors(sdk, [x, s, b])
    ty = sdk.tensor(dtype, x.shape)
    sdk.call(f"tensor_layer_norm_{dtype}", tx, ts, tb, 1e-5, ty)
    want = orc.layer_norm(x, s, b, 1e-5)
    if dtype == "f16":
        # (x - mean) * inv * scale + bias can cancel: 1 ulp, or the north-star
        # f16 reduction bound 2e-3 relative with a small absolute floor
        got = ty.download()
        d = np.abs(got.astype(np.float64) - want.astype(np.float64))
        ok = (f16_ulps(got, want) <= 1) | (d <= 2e-3 * np.abs(want.astype(np.float64)) + 1e-5)
        assert ok.all(), f"{(~ok).sum()} layer-norm f16 values off"
    else:
        assert_f32_rel(ty.download(), want, 1e-5, "layer f32", floor=1e-5)


@pytest.mark.parametrize("device", [True, False])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("shape", [(1, 1, 8), (2, 64, 64), (4, 100, 2048), (1, 7, 1001),
                                   (2, 16, 4096), (1, 4, 8192), (1, 3, 20000)])
def test_softmax_f16(sdk, orc, shape, causal, device):
    x = orc.normal(shape, 25, 0, 0.0, 3.0)
    tx = sdk.from_numpy(x, device=device)
    ty = sdk.tensor("f16", shape, device)
    sdk.call("tensor_softmax_f16", tx, int(causal), ty)
    got, want = ty.download(), orc.softmax(x, causal)
    assert_f16_ulps(got, want, 1, "softmax f16")
    rel = np.abs(got.astype(np.float64) - want) <= 2e-3 * want.astype(np.float64) + 2.0 ** -24
    assert rel.all()


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("shape", [(2, 64, 64), (2, 33, 2048), (1, 5, 1001), (1, 3, 8192)])
def test_softmax_f32(sdk, orc, shape, causal):
    x = orc.normal(shape, 26, 0, 0.0, 3.0, "f32")
    tx = sdk.from_numpy(x)
    ty = sdk.tensor("f32", shape)
    sdk.call("tensor_softmax_f32", tx, int(causal), ty)
    assert_f32_rel(ty.download(), orc.softmax(x, causal), 1e-5, "softmax f32", floor=1e-38)


@pytest.mark.parametrize("dtype", ["f16", "f32"])
@pytest.mark.parametrize("width", [4, 64, 1001, 8192])
def test_softmax_special_rows(sdk, orc, dtype, width):
    """attention.c:335-380 rules: +inf rows share 1/count, all -inf rows are
    zero, NaN poisons a row unless +inf is present; causal masking of the
    rest."""
    rows = []
    base = orc.normal((width,), 27, 0, 0.0, 3.0, "f32")
    for specials in ({1: np.inf}, {0: np.inf, 2: np.inf}, {"all": -np.inf}, {1: np.nan},
                     {1: np.nan, 2: np.inf}, {0: -np.inf, 3: -np.inf}, {}):
        r = base.copy()
        for k, v in specials.items():
            if k == "all":
                r[:] = v
            else:
                r[k] = v
        rows.append(r)
    x = np.stack(rows).astype(np.float16 if dtype == "f16" else np.float32)
    for causal in (0, 1):
        tx = sdk.from_numpy(x)
        ty = sdk.tensor(dtype, x.shape)
        sdk.call(f"tensor_softmax_{dtype}", tx, causal, ty)
        got, want = ty.download(), orc.softmax(x, bool(causal))
        if dtype == "f16":
            assert_f16_ulps(got, want, 1, f"special rows causal={causal}")
        else:
            assert_f32_rel(got, want, 1e-5, f"special rows causal={causal}", floor=1e-38)


def test_softmax_first_causal_row_is_one(sdk, orc):
    """Square causal block (q_len == k_len, so the causal offset is 0)."""
    x = orc.normal((2, 256, 256), 28, 0, 0.0, 3.0)
    tx, ty = sdk.from_numpy(x), sdk.tensor("f16", x.shape)
    sdk.call("tensor_softmax_f16", tx, 1, ty)
    y = ty.download()
    assert np.all(y[:, 0, 0] == 1) and np.all(y[:, 0, 1:] == 0)
    assert np.all(np.triu(y[0].astype(np.float32), 1) == 0)
    # q_len < k_len aligns the mask to the end (attention.c causal_offset):
    # query row 0 sees keys 0..k_len-q_len
    x = orc.normal((1, 4, 64), 28, 1, 0.0, 3.0)
    tx, ty = sdk.from_numpy(x), sdk.tensor("f16", x.shape)
    sdk.call("tensor_softmax_f16", tx, 1, ty)
    y = ty.download()[0].astype(np.float32)
    assert np.all(y[0, 61:] == 0) and np.all(y[0, :61] > 0) and np.all(y[3] > 0)


@pytest.mark.parametrize("dtype", ["f16", "f32"])
@pytest.mark.parametrize("rows,width", [(1, 1), (3, 7), (37, 2048), (5, 1001), (3, 8192), (2, 20000)])
def test_row_sum_max(sdk, orc, dtype, rows, width):
    x = orc.normal((rows, width), 29, 0, 0.0, 3.0, dtype)
    tx = sdk.from_numpy(x)
    ts, tm = sdk.tensor("f32", (rows,)), sdk.tensor("f32", (rows,))
    sdk.call(f"tensor_row_sum_{dtype}", tx, ts)
    sdk.call(f"tensor_row_max_{dtype}", tx, tm)
    s, a = orc.row_sum(x)
    assert np.all(np.abs(ts.download().astype(np.float64) - s) <= 1e-5 * a + 1e-30)
    assert_bits_equal(tm.download(), orc.row_max(x), "row max")


def test_row_max_nan_and_inf(sdk, orc):
    x = orc.normal((4, 2048), 30, 0, 0.0, 3.0, "f32")
    x[1, 700] = np.nan
    x[2, 5] = np.inf
    x[3, :] = -np.inf
    tx, tm = sdk.from_numpy(x), sdk.tensor("f32", (4,))
    sdk.call("tensor_row_max_f32", tx, tm)
    assert_bits_equal(tm.download(), orc.row_max(x), "specials")


def test_config3_full_size(sdk, orc):
    x = sdk.tensor("f16", (16384, 2048))
    sdk.call("tensor_fill_normal", x, 3, 0, 0.0, 1.0)
    w = sdk.tensor("f16", (2048,))
    sdk.call("tensor_fill_uniform", w, 3, 1, 0.5, 1.5)
    y = sdk.tensor("f16", (16384, 2048))
    sdk.call("tensor_rms_norm_f16", x, w, 1e-6, y)
    assert_f16_ulps(y.download(), orc.rms_norm(x.download(), w.download(), 1e-6), 1, "rms cfg3")
    del y
    logits = sdk.tensor("f16", (32, 2048, 2048))
    sdk.call("tensor_fill_normal", logits, 3, 2, 0.0, 3.0)
    probs = sdk.tensor("f16", (32, 2048, 2048))
    sdk.call("tensor_softmax_f16", logits, 1, probs)
    xs = logits.download()
    assert_f16_ulps(probs.download(), orc.softmax(xs, True), 1, "softmax cfg3")
    sums, maxes = sdk.tensor("f32", (32, 2048)), sdk.tensor("f32", (32, 2048))
    sdk.call("tensor_row_sum_f16", logits, sums)
    sdk.call("tensor_row_max_f16", logits, maxes)
    s, a = orc.row_sum(xs)
    assert np.all(np.abs(sums.download().ravel().astype(np.float64) - s) <= 1e-5 * a)
    assert_bits_equal(maxes.download().ravel(), orc.row_max(xs), "row max cfg3")
