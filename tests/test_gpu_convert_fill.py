"""tensor_buffer_convert on the GPU (bit rules of the reference's
tensor_f16.c / tensor_buffer.c, NaN payloads included) and the device
synthetic-input generator against its CPU definition."""
import ctypes

import numpy as np
import pytest

from tests.helpers import assert_bits_equal, f32_ulps

pytestmark = pytest.mark.gpu


def convert(sdk, array, src, dst, device):
    t = sdk.tensor(src, array.shape, device).upload(array)
    out = ctypes.c_void_p()
    err = ctypes.create_string_buffer(256)
    assert sdk.lib.tensor_buffer_convert(t.handle, {"f32": 14, "f16": 12, "bf16": 13}[dst],
                                         ctypes.byref(out), err, 256), err.value
    n = array.size
    res = np.empty(n, np.float32 if dst == "f32" else np.uint16)
    assert sdk.lib.tensor_buffer_download(out.value, 0, res.ctypes.data, res.nbytes, err, 256), err.value
    assert sdk.lib.tensor_buffer_storage(out.value) == (1 if device else 0)
    sdk.lib.tensor_buffer_free(out.value)
    return res.reshape(array.shape)


@pytest.mark.parametrize("device", [True, False])
def test_f16_to_f32_every_half(sdk, orc, device):
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = convert(sdk, h, "f16", "f32", device)
    assert np.array_equal(got.view(np.uint32), orc.f16_to_f32(h).view(np.uint32))


@pytest.mark.parametrize("device", [True, False])
def test_f32_to_f16_and_bf16_bit_patterns(sdk, orc, device):
    rng = np.random.default_rng(7)
    bits = rng.integers(0, 2**32, size=4_000_000, dtype=np.uint64).astype(np.uint32)
    edges = np.array([0x7f800001, 0xff800001, 0x7fc00000, 0x7f802000, 0x7fffe000, 0x477ff000,
                      0x477fefff, 0x38800000, 0x387fffff, 0x33000000, 0x33000001, 0x80000001,
                      0x7f800000, 0xff800000, 0, 0x80000000], np.uint32)
    bits = np.concatenate([bits, edges])
    # every rounding boundary region: low 13 bits set to the tie and neighbours
    hi = np.arange(0, 1 << 19, dtype=np.uint32) << 13
    for low in (0x0fff, 0x1000, 0x1001):
        bits = np.concatenate([bits, hi | low])
    f = bits.view(np.float32)
    assert np.array_equal(convert(sdk, f, "f32", "f16", device), orc.f32_to_f16(f))
    assert np.array_equal(convert(sdk, f, "f32", "bf16", device), orc.f32_to_bf16(f))


def test_same_dtype_is_a_copy(sdk):
    a = np.arange(1000, dtype=np.float32)
    assert np.array_equal(convert(sdk, a, "f32", "f32", True), a)


@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_fill_uniform_matches_cpu_definition(sdk, orc, dtype):
    n = 3_000_001
    t = sdk.tensor(dtype, (n,))
    sdk.call("tensor_fill_uniform", t, 0, 0, -1.0, 1.0)
    assert_bits_equal(t.download(), orc.uniform((n,), 0, 0, -1.0, 1.0, dtype), "uniform")


@pytest.mark.parametrize("dtype", ["f32", "f16"])
def test_fill_normal_matches_cpu_definition(sdk, orc, dtype):
    """Box-Muller in double on both sides; device and host libm may differ in
    the last double bit, which after rounding to f32 changes at most one ulp
    of a vanishing fraction of elements."""
    n = 2_000_003
    t = sdk.tensor(dtype, (n,))
    sdk.call("tensor_fill_normal", t, 1, 0, 0.0, 3.0)
    got, want = t.download(), orc.normal((n,), 1, 0, 0.0, 3.0, dtype)
    g32, w32 = got.astype(np.float32), want.astype(np.float32)
    diff = g32 != w32
    assert diff.sum() <= n * 1e-5
    assert np.all(f32_ulps(g32[diff], w32[diff]) <= (8192 if dtype == "f16" else 1))
