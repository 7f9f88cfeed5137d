"""Writes tests/golden/reference_vectors.npz: inputs and the outputs of the
reference's own portable C path (oracle/_ref/libref.so, compiled from the
reference sources by oracle/Makefile) on small seeded inputs.

Run in a container that has /root/reference:  make -C oracle && python tests/golden/make_golden.py
The fixture is data only (numpy arrays, loaded with allow_pickle=False).
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import Oracle, Reference  # noqa: E402


def main():
    orc, ref = Oracle(), Reference()
    out = {}
    # SiLU (tensor_ops.c:545-573)
    x16 = orc.normal((8, 129), 100, 0, 0.0, 4.0)
    x32 = orc.normal((8, 129), 100, 1, 0.0, 4.0, "f32")
    out["silu_f16_x"], out["silu_f16_y"] = x16, ref.silu(x16)
    out["silu_f32_x"], out["silu_f32_y"] = x32, ref.silu(x32)
    # RMSNorm (tensor_ops.c:400-459)
    for dt, width in (("f16", 2048), ("f32", 1000)):
        x = orc.normal((6, width), 101, 0, 0.0, 1.0, dt)
        w = orc.uniform((width,), 101, 1, 0.5, 1.5, dt)
        out[f"rms_{dt}_x"], out[f"rms_{dt}_w"] = x, w
        out[f"rms_{dt}_y"] = ref.rms_norm(x, w, 1e-6)
    # LayerNorm with scale and bias (tensor_ops.c:461-543)
    for dt in ("f16", "f32"):
        x = orc.normal((5, 256), 102, 0, 0.5, 2.0, dt)
        s = orc.uniform((256,), 102, 1, 0.5, 1.5, dt)
        b = orc.uniform((256,), 102, 2, -1.0, 1.0, dt)
        out[f"layer_{dt}_x"], out[f"layer_{dt}_s"], out[f"layer_{dt}_b"] = x, s, b
        out[f"layer_{dt}_y"] = ref.layer_norm(x, s, b, 1e-5)
    # F16 residual add (tensor_ops.c:575-622)
    a = orc.normal((4096,), 103, 0, 0.0, 50.0)
    b = orc.normal((4096,), 103, 1, 0.0, 50.0)
    out["residual_a"], out["residual_b"], out["residual_y"] = a, b, ref.residual_add_f16(a, b)
    # softmax inside tensor_sdpa_f32 (attention.c:335-380), plain and causal
    s = orc.normal((24, 128), 104, 0, 0.0, 3.0, "f32")
    s[3, 7] = np.inf
    s[5, :] = -np.inf
    s[9, ::3] = -np.inf
    out["softmax_x"] = s
    out["softmax_y"] = ref.softmax_rows_f32(s, False)
    out["softmax_causal_y"] = ref.softmax_rows_f32(s, True)
    # conversions (tensor_buffer.c:274-298)
    rng = np.random.default_rng(105)
    bits = rng.integers(0, 2**32, size=8192, dtype=np.uint64).astype(np.uint32)
    f = bits.view(np.float32)
    out["convert_f32"] = f
    out["convert_f32_to_f16"] = ref.convert(f, "f32", "f16")
    out["convert_f32_to_bf16"] = ref.convert(f, "f32", "bf16")
    path = os.path.join(HERE, "reference_vectors.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path}: {len(out)} arrays")


if __name__ == "__main__":
    main()
