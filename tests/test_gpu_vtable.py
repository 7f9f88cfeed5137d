"""The "hip" TensorComputeBackend table through its C ABI.

The known answers are those of the reference's tests/test_tensor_compute.c
(which the reference only runs against Metal) and
tests/test_cuda_vision_sequence.cu, applied to the HIP table; the random
cases compare each host-pointer slot with the CPU oracle."""
import ctypes

import numpy as np
import pytest

from tests.helpers import arbitrated, assert_bits_equal, assert_f16_ulps, f16_ulps, rope_close

pytestmark = pytest.mark.gpu

from inference_c_amd import COMPUTE_SLOTS as SLOTS  # noqa: E402


P, Z, F, D, I = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_float, ctypes.c_double, ctypes.c_int
SIGS = {
    "rms_norm_f16": [P, P, P, Z, Z, F], "rms_norm_f32": [P, P, P, Z, Z, F],
    "layer_norm_f16": [P, P, P, P, Z, Z, F], "layer_norm_f32": [P, P, P, P, Z, Z, F],
    "bias_add_f16": [P, P, P, Z, Z], "bias_add_f32": [P, P, P, Z, Z],
    "gelu_f16": [P, P, Z], "gelu_f32": [P, P, Z], "relu_f16": [P, P, Z],
    "gelu_multiply_f16": [P, P, P, Z], "silu_multiply_f16": [P, P, P, Z],
    "silu_multiply_f32": [P, P, P, Z], "residual_add_f16": [P, P, P, Z],
    "residual_add_f32": [P, P, P, Z], "argmax_f16": [P, Z, P], "argmax_f32": [P, Z, P],
    "rope_f16": [P, P, Z, Z, Z, Z, D, Z], "rope_f32": [P, P, Z, Z, Z, Z, D],
    "bias_add_f32_device": [P, P, P, Z, Z], "bias_add_f16_device": [P, P, P, Z, Z],
    "residual_add_f16_device": [P, P, P, Z],
}


from inference_c_amd import ComputeBackend as Table  # noqa: E402,F401


@pytest.fixture(scope="module")
def hip(sdk):
    table = ctypes.cast(sdk.lib.tensor_compute_hip_backend(), ctypes.POINTER(Table)).contents
    fns = {}
    for name, args in SIGS.items():
        addr = getattr(table, name)
        assert addr, f"slot {name} is NULL"
        fns[name] = ctypes.CFUNCTYPE(I, *args)(addr)
    fns["table"] = table
    return fns


def p(a):
    return a.ctypes.data


def test_table_shape(hip):
    t = hip["table"]
    assert ctypes.cast(t.name, ctypes.c_char_p).value == b"hip"
    assert ctypes.CFUNCTYPE(I)(t.is_available)() == 1
    for slot in ("linear_f32", "linear_f16", "mlp_f16", "qkv_f16", "linear_f32_device",
                 "linear_f16_device", "rms_norm_linear_f32", "linear_q8_0_f16_device",
                 "linear_q4_0_f16_device", "linear_q8_0_f16", "linear_q4_0_f16"):
        assert getattr(t, slot), f"{slot} is NULL"
    # whole transformer layers (model harness code) are not provided
    for slot in ("mlp_f32", "vision_layer_f16", "vision_layer_f32", "vision_sequence_begin_f16",
                 "vision_sequence_layer_quant_f16", "vision_sequence_begin_f32"):
        assert getattr(t, slot) is None, f"{slot} should be NULL"
    assert t.release_cache


def test_reference_compute_known_answers(hip):
    """tests/test_tensor_compute.c:121-212 of the reference."""
    near = lambda a, b: abs(a - b) < 2e-4
    x = np.array([1, 2, 3, 4], np.float32); w = np.ones(2, np.float32); y = np.zeros(4, np.float32)
    assert hip["rms_norm_f32"](p(x), p(w), p(y), 2, 2, 1e-5)
    assert all(near(a, b) for a, b in zip(y, [0.63245, 1.2649, 0.84853, 1.13137]))
    x = np.array([1, 3, 2, 4], np.float32); b = np.zeros(2, np.float32)
    assert hip["layer_norm_f32"](p(x), p(w), p(b), p(y), 2, 2, 1e-5)
    assert all(near(a, c) for a, c in zip(y, [-1, 1, -1, 1]))
    x = np.array([1, 2, 3, 4], np.float32); bias = np.array([10, 20], np.float32)
    assert hip["bias_add_f32"](p(x), p(bias), p(y), 2, 2)
    assert y.tolist() == [11, 22, 13, 24]
    g = np.array([0, 1, 10.375, -10.375, 20, -20], np.float32); gy = np.zeros(6, np.float32)
    assert hip["gelu_f32"](p(g), p(gy), 6)
    assert np.all(np.isfinite(gy)) and near(gy[0], 0) and near(gy[1], 0.84119)
    assert near(gy[2], 10.375) and near(gy[3], 0)
    q = np.array([1, 0, 1, 0], np.float32); k = q.copy()
    assert hip["rope_f32"](p(q), p(k), 2, 1, 1, 2, 10000.0)
    for v in (q, k):
        assert near(v[0], 1) and near(v[1], 0) and near(v[2], np.cos(1.0)) and near(v[3], np.sin(1.0))
    gate = np.array([0, 1], np.float32); up = np.array([2, 3], np.float32); out = np.zeros(2, np.float32)
    assert hip["silu_multiply_f32"](p(gate), p(up), p(out), 2)
    assert near(out[0], 0) and near(out[1], 2.19318)
    xs = np.array([0, 1, -1, 0.5, 10.375, -10.375], np.float32).astype(np.float16)
    ms = np.array([2, 3, 4, -2, 0.25, 1.5], np.float32).astype(np.float16)
    prod = np.zeros(6, np.float16)
    assert hip["gelu_multiply_f16"](p(xs), p(ms), p(prod), 6)
    for xi, mi, yi in zip(xs.astype(np.float64), ms.astype(np.float64), prod.astype(np.float64)):
        gelu = xi if xi >= 5 else 0.0 if xi <= -5 else 0.5 * xi * (1 + np.tanh(0.7978845608 * (xi + 0.044715 * xi ** 3)))
        assert abs(yi - gelu * mi) < 2e-3
    r = np.array([0xbc00, 0x0000, 0x4200], np.uint16); ro = np.zeros(3, np.uint16)
    assert hip["relu_f16"](p(r), p(ro), 3)
    assert ro.view(np.float16).astype(np.float32).tolist() == [0.0, 0.0, 3.0]
    a = np.array([1, 2, 3], np.float32); bb = np.array([4, 5, 6], np.float32); s = np.zeros(3, np.float32)
    assert hip["residual_add_f32"](p(a), p(bb), p(s), 3)
    assert s.tolist() == [5, 7, 9]
    logits = np.array([-2, 5, 5, 1], np.float32); best = np.array([0xffffffff], np.uint32)
    assert hip["argmax_f32"](p(logits), 4, p(best))
    assert best[0] == 1


def test_slots_reject_bad_arguments(hip):
    x = np.ones(4, np.float32)
    assert hip["gelu_f32"](p(x), None, 4) == 0
    assert hip["residual_add_f32"](p(x), p(x), p(x), 0) == 0
    assert hip["rope_f32"](p(x), p(x), 1, 1, 1, 3, 10000.0) == 0  # odd head_dim
    assert hip["rms_norm_f32"](p(x), None, p(x), 2, 2, 1e-5) == 0


def test_slots_vs_oracle(hip, orc):
    rows, width = 33, 2048
    x = orc.normal((rows, width), 60, 0, 0.0, 1.0)
    w = orc.uniform((width,), 60, 1, 0.5, 1.5, "f16")
    y = np.zeros_like(x)
    assert hip["rms_norm_f16"](p(x), p(w), p(y), rows, width, 1e-6)
    assert_f16_ulps(y, orc.rms_norm(x, w, 1e-6), 1, "rms slot")
    b = orc.uniform((width,), 60, 2, -1.0, 1.0, "f16")
    assert hip["layer_norm_f16"](p(x), p(w), p(b), p(y), rows, width, 1e-5)
    want = orc.layer_norm(x, w, b, 1e-5)
    d = np.abs(y.astype(np.float64) - want.astype(np.float64))
    assert ((f16_ulps(y, want) <= 1) | (d <= 2e-3 * np.abs(want.astype(np.float64)) + 1e-5)).all()
    assert hip["bias_add_f16"](p(x), p(b), p(y), rows, width)
    assert_bits_equal(y, orc.bias_add(x, b), "bias slot")
    g = orc.normal((rows * width,), 60, 3, 0.0, 1.0)
    u = orc.normal((rows * width,), 60, 4, 0.0, 1.0)
    out = np.zeros_like(g)
    assert hip["silu_multiply_f16"](p(g), p(u), p(out), g.size)
    assert_f16_ulps(out, orc.silu_multiply(g, u), 1, "swiglu slot")
    assert hip["residual_add_f16"](p(g), p(u), p(out), g.size)
    assert_bits_equal(out, orc.add(g, u), "residual slot")
    assert hip["gelu_f16"](p(g), p(out), g.size)
    assert arbitrated(out, orc.gelu(g), orc.gelu_f64(g.astype(np.float64)), f16_ulps).all()
    best = np.zeros(1, np.uint32)
    assert hip["argmax_f16"](p(g), g.size, p(best))
    assert best[0] == orc.argmax(g)
    # in place, as the model harness calls it (text_model.c:733)
    gg = g.copy()
    assert hip["silu_multiply_f16"](p(gg), p(u), p(gg), g.size)
    assert_f16_ulps(gg, orc.silu_multiply(g, u), 1, "in-place slot")
    seq, heads, dim = 50, 4, 64
    q = orc.normal((seq, heads, dim), 60, 5, 0.0, 1.0)
    k = orc.normal((seq, 2, dim), 60, 6, 0.0, 1.0)
    q0, k0 = q.copy(), k.copy()
    wq, wk = orc.rope(q, k, heads, 2, dim, 10000.0, 7)
    assert hip["rope_f16"](p(q), p(k), seq, heads, 2, dim, 10000.0, 7)
    rope_close(q, wq, q0)
    rope_close(k, wk, k0)
    hip["table"].release_cache and ctypes.CFUNCTYPE(None)(hip["table"].release_cache)()


def test_device_slots(hip, sdk, orc):
    rows, width = 64, 4096
    x = orc.uniform((rows, width), 61, 0, -1.0, 1.0)
    bias = orc.uniform((width,), 61, 1, -1.0, 1.0)
    tx, tb, ty = sdk.from_numpy(x), sdk.from_numpy(bias), sdk.tensor("f32", x.shape)
    assert hip["bias_add_f32_device"](tx.device_ptr(), tb.device_ptr(), ty.device_ptr(), rows, width)
    sdk.synchronize()
    assert_bits_equal(ty.download(), orc.bias_add(x, bias), "bias device f32")
    hx, hb = x.astype(np.float16), bias.astype(np.float16)
    tx, tb, ty = sdk.from_numpy(hx), sdk.from_numpy(hb), sdk.tensor("f16", x.shape)
    assert hip["bias_add_f16_device"](tx.device_ptr(), tb.device_ptr(), ty.device_ptr(), rows, width)
    assert_bits_equal(ty.download(), orc.bias_add(hx, hb), "bias device f16")
    assert hip["residual_add_f16_device"](tx.device_ptr(), ty.device_ptr(), tx.device_ptr(), hx.size)
    assert_bits_equal(tx.download(), orc.add(hx, orc.bias_add(hx, hb)), "residual device in place")
    assert hip["residual_add_f16_device"](None, ty.device_ptr(), tx.device_ptr(), 4) == 0
