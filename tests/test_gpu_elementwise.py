"""Elementwise and row-broadcast kernels on the GPU against the CPU oracle.

Bar: add/mul bit-exact; f16 transcendental outputs
within 1 ulp of the reference, with the tanh-GELU arbitration rule (or no
farther from a double evaluation of the same formula than the reference);
f32 transcendentals within 1e-6 relative. Every op runs with device storage
and with host storage (staged through the device)."""
import numpy as np
import pytest

from tests.helpers import (arbitrated, assert_bits_equal, assert_f16_ulps, assert_f32_rel,
                           f16_ulps, f32_ulps)

pytestmark = pytest.mark.gpu

SIZES = [1, 7, 8, 9, 4096 + 3, 1 << 20]
F16 = np.float16
ALL_HALVES = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(F16)


def run(sdk, name, inputs, out_dtype, device=True):
    ts = [sdk.from_numpy(a, device=device) for a in inputs]
    out = sdk.tensor(out_dtype, inputs[0].shape, device)
    sdk.call(name, *ts, out)
    return out.download()


def specials_f32():
    return np.array([0.0, -0.0, 1.0, -1.0, np.inf, -np.inf, np.nan, 1e-45, -1e-45, 1e-38,
                     3.4e38, -3.4e38, 88.0, -88.0, 89.0, -104.0, 5.0, -5.0, 4.999999,
                     -4.999999, 1e-7, 20.0, -20.0, 10.375, -10.375], np.float32)


@pytest.mark.parametrize("device", [True, False])
@pytest.mark.parametrize("n", SIZES)
def test_add_mul_f32_bit_exact(sdk, orc, n, device):
    a = orc.uniform((n,), 0, 0, -1.0, 1.0)
    b = orc.uniform((n,), 0, 1, -1.0, 1.0)
    assert_bits_equal(run(sdk, "tensor_add_f32", [a, b], "f32", device), orc.add(a, b), "add")
    assert_bits_equal(run(sdk, "tensor_mul_f32", [a, b], "f32", device), orc.mul(a, b), "mul")


def test_add_mul_f32_specials_and_denormals(sdk, orc):
    s = specials_f32()
    a = np.repeat(s, s.size)
    b = np.tile(s, s.size)
    assert_bits_equal(run(sdk, "tensor_add_f32", [a, b], "f32"), orc.add(a, b), "add specials")
    assert_bits_equal(run(sdk, "tensor_mul_f32", [a, b], "f32"), orc.mul(a, b), "mul specials")


@pytest.mark.parametrize("partner", [0x0000, 0x8000, 0x3c00, 0xbc00, 0x0001, 0x03ff, 0x7bff,
                                     0xfbff, 0x7c00, 0x3555, 0x1400])
def test_add_mul_f16_every_half(sdk, orc, partner):
    b = np.full(65536, partner, np.uint16).view(F16)
    assert_bits_equal(run(sdk, "tensor_residual_add_f16", [ALL_HALVES, b], "f16"),
                      orc.add(ALL_HALVES, b), "f16 add")
    assert_bits_equal(run(sdk, "tensor_mul_f16", [ALL_HALVES, b], "f16"),
                      orc.mul(ALL_HALVES, b), "f16 mul")


@pytest.mark.parametrize("device", [True, False])
@pytest.mark.parametrize("n", SIZES)
def test_residual_add_f16_random(sdk, orc, n, device):
    a = orc.normal((n,), 1, 0, 0.0, 1.0)
    b = orc.normal((n,), 1, 1, 0.0, 1.0)
    assert_bits_equal(run(sdk, "tensor_residual_add_f16", [a, b], "f16", device), orc.add(a, b))


def test_silu_f16_every_half(sdk, orc):
    got = run(sdk, "tensor_silu_f16", [ALL_HALVES], "f16")
    assert_f16_ulps(got, orc.silu(ALL_HALVES), 1, "silu f16")


def test_relu_f16_every_half(sdk, orc):
    assert_bits_equal(run(sdk, "tensor_relu_f16", [ALL_HALVES], "f16"), orc.relu(ALL_HALVES), "relu")


def test_gelu_f16_every_half(sdk, orc):
    got = run(sdk, "tensor_gelu_f16", [ALL_HALVES], "f16")
    want = orc.gelu(ALL_HALVES)
    exact = orc.gelu_f64(ALL_HALVES.astype(np.float64))
    ok = arbitrated(got, want, exact, f16_ulps)
    assert ok.all(), f"{(~ok).sum()} halves fail the GELU rule, e.g. {ALL_HALVES[~ok][:5]}"
    # clamps are exact
    x = ALL_HALVES.astype(np.float32)
    assert_bits_equal(got[x >= 5], ALL_HALVES[x >= 5], "x >= 5 keeps x")
    assert np.all(got[x <= -5].view(np.uint16) == 0), "x <= -5 gives +0"


@pytest.mark.parametrize("device", [True, False])
def test_silu_gelu_f32(sdk, orc, device):
    x = np.concatenate([orc.normal((1 << 16,), 2, 0, 0.0, 6.0, "f32"), specials_f32()])
    got = run(sdk, "tensor_silu_f32", [x], "f32", device)
    assert_f32_rel(got, orc.silu(x), 1e-6, "silu f32", floor=1e-38)
    got = run(sdk, "tensor_gelu_f32", [x], "f32", device)
    want = orc.gelu(x)
    exact = orc.gelu_f64(x.astype(np.float64))
    with np.errstate(invalid="ignore"):   # Inf - Inf: NaN compares False; the rules below decide
        rel_ok = np.abs(got.astype(np.float64) - want) <= 1e-6 * np.abs(want) + 1e-38
    ok = rel_ok | arbitrated(got, want, exact, f32_ulps)
    ok |= np.isnan(got) & np.isnan(want)
    assert ok.all(), f"{(~ok).sum()} GELU f32 values fail, e.g. {x[~ok][:5]}"


@pytest.mark.parametrize("device", [True, False])
@pytest.mark.parametrize("n", SIZES)
def test_swiglu_f16(sdk, orc, n, device):
    gate = orc.normal((n,), 3, 0, 0.0, 1.0)
    up = orc.normal((n,), 3, 1, 0.0, 1.0)
    got = run(sdk, "tensor_silu_multiply_f16", [gate, up], "f16", device)
    assert_f16_ulps(got, orc.silu_multiply(gate, up), 1, "swiglu")


def test_swiglu_f16_specials(sdk, orc):
    g = np.repeat(ALL_HALVES[::97], 11)
    u = np.tile(np.array([0, 1, -1, 65504, -65504, np.inf, np.nan, 1e-7, 2, 0.5, -3], F16), g.size // 11)
    assert_f16_ulps(run(sdk, "tensor_silu_multiply_f16", [g, u], "f16"), orc.silu_multiply(g, u), 1)


def test_swiglu_f32(sdk, orc):
    g = orc.normal((100003,), 3, 2, 0.0, 4.0, "f32")
    u = orc.normal((100003,), 3, 3, 0.0, 4.0, "f32")
    assert_f32_rel(run(sdk, "tensor_silu_multiply_f32", [g, u], "f32"),
                   orc.silu_multiply(g, u), 1e-6, "swiglu f32", floor=1e-38)


def test_gelu_multiply_f16(sdk, orc):
    x = np.repeat(ALL_HALVES[::13], 3)
    g = np.tile(np.array([2, -0.25, 3.5], F16), x.size // 3)
    got = run(sdk, "tensor_gelu_multiply_f16", [x, g], "f16")
    want = orc.gelu_multiply(x, g)
    exact = orc.gelu_f64(x.astype(np.float64)) * g.astype(np.float64)
    ok = arbitrated(got, want, exact, f16_ulps)
    assert ok.all(), f"{(~ok).sum()} fail"


@pytest.mark.parametrize("device", [True, False])
@pytest.mark.parametrize("rows,width", [(1024, 4096), (3, 5), (7, 24), (5, 12), (1, 1)])
def test_bias_add(sdk, orc, rows, width, device):
    x = orc.uniform((rows, width), 0, 0, -1.0, 1.0)
    b = orc.uniform((width,), 0, 2, -1.0, 1.0)
    got = run_bias(sdk, "tensor_bias_add_f32", x, b, "f32", device)
    assert_bits_equal(got, orc.bias_add(x, b), "bias f32")
    hx, hb = x.astype(F16), b.astype(F16)
    assert_bits_equal(run_bias(sdk, "tensor_bias_add_f16", hx, hb, "f16", device),
                      orc.bias_add(hx, hb), "bias f16")
    got = run_bias(sdk, "tensor_bias_gelu_f16", hx * F16(6), hb, "f16", device)
    want = orc.bias_add(hx * F16(6), hb, gelu=True)
    exact = orc.gelu_f64((hx * F16(6)).astype(np.float64) + hb.astype(np.float64))
    assert arbitrated(got, want, exact, f16_ulps).all()
    got = run_bias(sdk, "tensor_bias_gelu_f32", x * 6, b, "f32", device)
    want = orc.bias_add(x * 6, b, gelu=True)
    exact = orc.gelu_f64((x * 6 + b).astype(np.float64))
    with np.errstate(invalid="ignore"):   # Inf - Inf: NaN compares False; the rules below decide
        rel_ok = np.abs(got.astype(np.float64) - want) <= 1e-6 * np.abs(want) + 1e-38
    assert (rel_ok | arbitrated(got, want, exact, f32_ulps)).all()


def run_bias(sdk, name, x, b, dtype, device):
    tx, tb = sdk.from_numpy(x, device=device), sdk.from_numpy(b, device=device)
    out = sdk.tensor(dtype, x.shape, device)
    sdk.call(name, tx, tb, out)
    return out.download()


def test_in_place_aliasing(sdk, orc):
    """vtable callers pass the output as one of the inputs (e.g.
    silu_multiply_f16(gate, up, gate), text_model.c:733)."""
    g = orc.normal((10007,), 4, 0, 0.0, 1.0)
    u = orc.normal((10007,), 4, 1, 0.0, 1.0)
    tg, tu = sdk.from_numpy(g), sdk.from_numpy(u)
    sdk.call("tensor_silu_multiply_f16", tg, tu, tg)
    assert_f16_ulps(tg.download(), orc.silu_multiply(g, u), 1)
    sdk.call("tensor_residual_add_f16", tu, tu, tu)
    assert_bits_equal(tu.download(), orc.add(u, u))


# ---- configuration-sized runs (BASELINE configs 1 and 2) ------------------

def test_config1_add_mul_bias_full_size(sdk, orc):
    a = orc.uniform((1024, 4096), 0, 0, -1.0, 1.0)
    b = orc.uniform((1024, 4096), 0, 1, -1.0, 1.0)
    bias = orc.uniform((4096,), 0, 2, -1.0, 1.0)
    assert_bits_equal(run(sdk, "tensor_add_f32", [a, b], "f32"), orc.add(a, b))
    assert_bits_equal(run(sdk, "tensor_mul_f32", [a, b], "f32"), orc.mul(a, b))
    assert_bits_equal(run_bias(sdk, "tensor_bias_add_f32", a, bias, "f32", True), orc.bias_add(a, bias))


def test_config2_full_size(sdk, orc):
    x = sdk.tensor("f16", (8192, 8192))
    sdk.call("tensor_fill_normal", x, 1, 0, 0.0, 1.0)
    xs = x.download()
    y = sdk.tensor("f16", (8192, 8192))
    sdk.call("tensor_silu_f16", x, y)
    assert_f16_ulps(y.download(), orc.silu(xs), 1, "silu cfg2")
    sdk.call("tensor_gelu_f16", x, y)
    got = y.download()
    ok = arbitrated(got, orc.gelu(xs), orc.gelu_f64(xs.astype(np.float64)), f16_ulps)
    assert ok.all(), f"{(~ok).sum()} fail"
    del xs, got
    a = sdk.tensor("f16", (4096, 16384))
    b = sdk.tensor("f16", (4096, 16384))
    sdk.call("tensor_fill_normal", a, 1, 1, 0.0, 1.0)
    sdk.call("tensor_fill_normal", b, 1, 2, 0.0, 1.0)
    out = sdk.tensor("f16", (4096, 16384))
    sdk.call("tensor_silu_multiply_f16", b, a, out)  # out = a * silu(b)
    assert_f16_ulps(out.download(), orc.silu_multiply(b.download(), a.download()), 1, "swiglu cfg2")


def test_add_f16_past_one_launch(sdk, orc):
    """2^34 + 43 f16 elements: more than 2^31 16-byte vectors, past what one
    one-shot launch may cover (a dispatch counts its work-items in 32 bits),
    so the map is split over launches. The start, both sides of the seam
    between the launches and the ragged tail are bit-exact (96 GiB of device
    operands; the windows are read back and checked against the oracle's
    fill of the same element indices)."""
    n = (1 << 34) + 8 * 5 + 3
    print(f"f16 add past one launch: {n} elements", flush=True)
    a, b, y = sdk.tensor("f16", (n,)), sdk.tensor("f16", (n,)), sdk.tensor("f16", (n,))
    sdk.call("tensor_fill_normal", a, 21, 0, 0.0, 1.0)
    sdk.call("tensor_fill_normal", b, 21, 1, 0.0, 1.0)
    sdk.call("tensor_residual_add_f16", a, b, y)
    sdk.synchronize()
    seam = (1 << 31) * 8
    for first in (0, seam - 4096, n - 4096):
        want = orc.add(orc.normal((4096,), 21, 0, 0.0, 1.0, first=first),
                       orc.normal((4096,), 21, 1, 0.0, 1.0, first=first))
        assert_bits_equal(y.download_range(first, 4096), want)
    for t in (a, b, y):
        t.free()
