"""Whole-tensor reductions on the GPU: sum+max (two-pass grid reduction) and
argmax with the reference's scan semantics (tensor_compute_cuda.cu:386-397),
up to BASELINE config 5's 2^30 f32 elements."""
import numpy as np
import pytest

from tests.helpers import assert_bits_equal

pytestmark = pytest.mark.gpu


def sum_max(sdk, x, device=True):
    tx = sdk.from_numpy(x, device=device)
    ts, tm = sdk.tensor("f64", (1,), device), sdk.tensor("f32", (1,), device)
    sdk.call("tensor_sum_max_f32", tx, ts, tm)
    return float(ts.download()[0]), tm.download()[0]


@pytest.mark.parametrize("device", [True, False])
@pytest.mark.parametrize("n", [1, 3, 4, 5, 1000003, 1 << 24])
def test_sum_max(sdk, orc, n, device):
    x = orc.uniform((n,), 40, 0, -1.0, 1.0)
    s, m = sum_max(sdk, x, device)
    want_s, abs_s, want_m = orc.sum_max(x)
    assert abs(s - want_s) <= 1e-6 * abs_s + 1e-30
    assert m == want_m


def test_sum_max_specials(sdk, orc):
    x = orc.uniform((100000,), 41, 0, -1.0, 1.0)
    x[123] = np.nan
    s, m = sum_max(sdk, x)
    assert np.isnan(s) and np.isnan(m)
    x[123] = np.inf
    s, m = sum_max(sdk, x)
    assert s == np.inf and m == np.inf
    x = np.full(1000, -np.inf, np.float32)
    s, m = sum_max(sdk, x)
    assert s == -np.inf and m == -np.inf
    # only one output requested
    tx, tm = sdk.from_numpy(orc.uniform((77,), 41, 1, 0, 1)), sdk.tensor("f32", (1,))
    sdk.call("tensor_sum_max_f32", tx, None, tm)
    assert tm.download()[0] == orc.uniform((77,), 41, 1, 0, 1).max()


def test_sum_max_two_pow_30(sdk, orc):
    """2^30 f32 U[-1,1]."""
    n = 1 << 30
    t = sdk.tensor("f32", (n,))
    sdk.call("tensor_fill_uniform", t, 0, 0, -1.0, 1.0)
    ts, tm = sdk.tensor("f64", (1,)), sdk.tensor("f32", (1,))
    sdk.call("tensor_sum_max_f32", t, ts, tm)
    x = t.download()
    want_s, abs_s, want_m = orc.sum_max(x)
    assert abs(float(ts.download()[0]) - want_s) <= 1e-6 * abs_s
    assert tm.download()[0] == want_m


def test_sum_max_past_one_sweep(sdk, orc):
    """More than 4096 chunks of 2^18 floats (one sweep of the capped pass-1
    grid): pass-1 blocks stride over a second sweep of chunks, ending in a
    partial chunk and a ragged tail."""
    n = 4096 * (1 << 18) + 3 * (1 << 17) + 1000 * 4 + 3
    t = sdk.tensor("f32", (n,))
    sdk.call("tensor_fill_uniform", t, 0, 7, -1.0, 1.0)
    ts, tm = sdk.tensor("f64", (1,)), sdk.tensor("f32", (1,))
    sdk.call("tensor_sum_max_f32", t, ts, tm)
    x = t.download()
    want_s, abs_s, want_m = orc.sum_max(x)
    assert abs(float(ts.download()[0]) - want_s) <= 1e-6 * abs_s
    assert tm.download()[0] == want_m
    x[n - 2] = 7.5  # in the ragged tail
    x[4096 * (1 << 18) + 17] = 3.0  # in the second sweep
    s, m = sum_max(sdk, x)
    assert m == 7.5 and abs(s - orc.sum_max(x)[0]) <= 1e-6 * abs_s


def argmax(sdk, x, device=True):
    tx = sdk.from_numpy(x, device=device)
    ti = sdk.tensor("u32", (1,), device)
    sdk.call("tensor_argmax_f16" if x.dtype == np.float16 else "tensor_argmax_f32", tx, ti)
    return int(ti.download()[0])


@pytest.mark.parametrize("values", [
    [-2, 5, 5, 1], [np.nan, 1, 2], [1, np.nan, 3, 3], [-np.inf, -np.inf], [-np.inf, 5],
    [0.0, -0.0], [-0.0, 0.0], [3], [1, 2, np.inf, np.inf], [np.nan, np.nan, np.inf],
    [-np.inf, np.nan, -np.inf]])
def test_argmax_semantics(sdk, orc, values):
    x = np.array(values, np.float32)
    assert argmax(sdk, x) == orc.argmax(x)
    assert argmax(sdk, x.astype(np.float16)) == orc.argmax(x.astype(np.float16))


@pytest.mark.parametrize("device", [True, False])
@pytest.mark.parametrize("n", [9, 1000, 1000003, (1 << 24) + 5])
def test_argmax_random_and_ties(sdk, orc, n, device):
    x = orc.uniform((n,), 42, 0, -1.0, 1.0)
    assert argmax(sdk, x, device) == orc.argmax(x)
    x[n // 3] = x[n - 1] = 2.0  # tie: first index wins
    assert argmax(sdk, x, device) == n // 3
    h = orc.normal((n,), 42, 1, 0.0, 1.0)  # f16 has many exact ties
    assert argmax(sdk, h, device) == orc.argmax(h)
    x[:] = -np.inf
    x[n - 1] = -1.0
    assert argmax(sdk, x, device) == n - 1
