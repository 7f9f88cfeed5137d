"""The committed reference vectors (tests/golden/reference_vectors.npz, written
by tests/golden/make_golden.py from the reference's own C path): the oracle
must reproduce them bit for bit on any machine, and the HIP library within
the north-star tolerances on the GPU."""
import ctypes
import os

import numpy as np
import pytest

from tests.helpers import assert_bits_equal, assert_f16_ulps, assert_f32_rel, f16_ulps

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "reference_vectors.npz")


@pytest.fixture(scope="module")
def g():
    with np.load(GOLDEN, allow_pickle=False) as data:
        return {k: data[k] for k in data.files}


def test_oracle_reproduces_reference_vectors(orc, g):
    assert_bits_equal(orc.silu(g["silu_f16_x"]), g["silu_f16_y"], "silu f16")
    assert_bits_equal(orc.silu(g["silu_f32_x"]), g["silu_f32_y"], "silu f32")
    for dt in ("f16", "f32"):
        assert_bits_equal(orc.rms_norm(g[f"rms_{dt}_x"], g[f"rms_{dt}_w"], 1e-6), g[f"rms_{dt}_y"], dt)
        assert_bits_equal(orc.layer_norm(g[f"layer_{dt}_x"], g[f"layer_{dt}_s"], g[f"layer_{dt}_b"], 1e-5),
                          g[f"layer_{dt}_y"], dt)
    assert_bits_equal(orc.add(g["residual_a"], g["residual_b"]), g["residual_y"], "residual")
    assert_bits_equal(orc.softmax(g["softmax_x"]), g["softmax_y"], "softmax")
    assert_bits_equal(orc.softmax(g["softmax_x"], True), g["softmax_causal_y"], "causal softmax")
    assert np.array_equal(orc.f32_to_f16(g["convert_f32"]), g["convert_f32_to_f16"])
    assert np.array_equal(orc.f32_to_bf16(g["convert_f32"]), g["convert_f32_to_bf16"])


@pytest.mark.gpu
def test_hip_library_on_reference_vectors(sdk, g):
    def call(name, args, out_dtype, shape):
        out = sdk.tensor(out_dtype, shape)
        sdk.call(name, *args, out)
        return out.download()

    T = sdk.from_numpy
    assert_f16_ulps(call("tensor_silu_f16", [T(g["silu_f16_x"])], "f16", g["silu_f16_x"].shape),
                    g["silu_f16_y"], 1, "silu f16")
    assert_f32_rel(call("tensor_silu_f32", [T(g["silu_f32_x"])], "f32", g["silu_f32_x"].shape),
                   g["silu_f32_y"], 1e-6, "silu f32", floor=1e-38)
    y = call("tensor_rms_norm_f16", [T(g["rms_f16_x"]), T(g["rms_f16_w"]), 1e-6], "f16", g["rms_f16_x"].shape)
    assert_f16_ulps(y, g["rms_f16_y"], 1, "rms f16")
    y = call("tensor_rms_norm_f32", [T(g["rms_f32_x"]), T(g["rms_f32_w"]), 1e-6], "f32", g["rms_f32_x"].shape)
    assert_f32_rel(y, g["rms_f32_y"], 1e-5, "rms f32")
    y = call("tensor_layer_norm_f16", [T(g["layer_f16_x"]), T(g["layer_f16_s"]), T(g["layer_f16_b"]), 1e-5],
             "f16", g["layer_f16_x"].shape)
    want = g["layer_f16_y"]
    d = np.abs(y.astype(np.float64) - want.astype(np.float64))
    assert ((f16_ulps(y, want) <= 1) | (d <= 2e-3 * np.abs(want.astype(np.float64)) + 1e-5)).all()
    y = call("tensor_layer_norm_f32", [T(g["layer_f32_x"]), T(g["layer_f32_s"]), T(g["layer_f32_b"]), 1e-5],
             "f32", g["layer_f32_x"].shape)
    assert_f32_rel(y, g["layer_f32_y"], 1e-5, "layer f32", floor=1e-5)
    y = call("tensor_residual_add_f16", [T(g["residual_a"]), T(g["residual_b"])], "f16", g["residual_a"].shape)
    assert_bits_equal(y, g["residual_y"], "residual")
    for causal, key in ((0, "softmax_y"), (1, "softmax_causal_y")):
        y = call("tensor_softmax_f32", [T(g["softmax_x"]), causal], "f32", g["softmax_x"].shape)
        assert_f32_rel(y, g[key], 1e-5, key, floor=1e-38)
    for dst, key, code in (("f16", "convert_f32_to_f16", 12), ("bf16", "convert_f32_to_bf16", 13)):
        src = T(g["convert_f32"])
        res = ctypes.c_void_p()
        err = ctypes.create_string_buffer(256)
        assert sdk.lib.tensor_buffer_convert(src.handle, code, ctypes.byref(res), err, 256), err.value
        got = np.empty(g[key].shape, np.uint16)
        assert sdk.lib.tensor_buffer_download(res.value, 0, got.ctypes.data, got.nbytes, err, 256)
        sdk.lib.tensor_buffer_free(res.value)
        assert np.array_equal(got, g[key]), key
