"""Pins the oracle's f16/bf16 conversions (and the library's host scalar
conversions) against the reference build, exhaustively, and against the
reference's own known answers (tests/test_tensor_buffer.c:19-67)."""
import ctypes
import math
import os
import subprocess

import numpy as np
import pytest

from tests.conftest import REPO

CHECKER = os.path.join(REPO, "oracle", "check_conversions")
REF_LIB = os.path.join(REPO, "oracle", "_ref", "libref.so")
ORACLE_LIB = os.path.join(REPO, "oracle", "liboracle.so")
PRODUCT_LIB = os.path.join(REPO, "inference_c_amd", "lib", "libinference_sdk_hip.so")


def _run_checker(lib_b, narrow_b, widen_b, stride):
    if not os.path.exists(REF_LIB):
        pytest.skip("reference build absent")
    if not os.path.exists(CHECKER):
        pytest.skip("oracle/check_conversions not built")
    out = subprocess.run([CHECKER, REF_LIB, "tensor_f32_to_f16", "tensor_f16_to_f32",
                          lib_b, narrow_b, widen_b, str(stride)],
                         capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "mismatches 0 of 65536; f32->f16 mismatches 0" in out.stdout


def test_oracle_conversions_exhaustive_vs_reference():
    """All 65536 halves and all 2^32 floats, bit for bit."""
    _run_checker(ORACLE_LIB, "orc_f32_to_f16", "orc_f16_to_f32", 1)


def test_library_host_conversions_vs_reference():
    """include/tensor_f16.h of the HIP library: every f16, every 3rd f32."""
    _run_checker(PRODUCT_LIB, "tensor_f32_to_f16", "tensor_f16_to_f32", 3)


def test_library_bf16_widening_vs_reference():
    """include/tensor_f16.h tensor_bf16_to_f32 of the HIP library against the
    reference build's (src/common/tensor_f16.c): all 65536 bf16 patterns, the
    same value and sign (NaNs: both NaN). A host function: no GPU needed."""
    if not os.path.exists(REF_LIB):
        pytest.skip("reference build absent")
    ref, lib = ctypes.CDLL(REF_LIB), ctypes.CDLL(PRODUCT_LIB)
    for f in (ref.tensor_bf16_to_f32, lib.tensor_bf16_to_f32):
        f.argtypes, f.restype = [ctypes.c_uint16], ctypes.c_float
    bad = 0
    for bits in range(65536):
        a, b = ref.tensor_bf16_to_f32(bits), lib.tensor_bf16_to_f32(bits)
        if math.isnan(a) or math.isnan(b):
            bad += not (math.isnan(a) and math.isnan(b))
        else:
            bad += not (a == b and math.copysign(1.0, a) == math.copysign(1.0, b))
    assert bad == 0
    # exact widening: the pattern is the high half of the f32
    assert lib.tensor_bf16_to_f32(0x3F80) == 1.0 and lib.tensor_bf16_to_f32(0xC000) == -2.0


def test_reference_known_answers(orc):
    # tests/test_tensor_buffer.c:30-61 of the reference
    inputs = [0.0, 1.0, -2.0, 0.33325, 65504.0, 0.00006103515625, 5.96046448e-8, 1e-8,
              70000.0, -0.5]
    back = [orc.lib.orc_f16_to_f32(orc.lib.orc_f32_to_f16(v)) for v in inputs]
    assert back[0] == 0.0 and back[1] == 1.0 and back[2] == -2.0
    assert abs(back[3] - 0.33325) <= 0.001
    assert back[4] == 65504.0
    assert back[5] == np.float32(0.00006103515625)
    assert back[6] == np.float32(5.96046448e-8)
    assert back[7] == 0.0
    assert np.isinf(back[8])
    assert back[9] == -0.5
    # bf16 round trip (test_tensor_buffer.c:38-45)
    bf = [orc.lib.orc_bf16_to_f32(orc.lib.orc_f32_to_bf16(v)) for v in inputs[:4]]
    assert bf[:3] == [0.0, 1.0, -2.0] and abs(bf[3] - 0.33325) <= 0.002


def test_numpy_agrees_on_non_nan(orc):
    """IEEE binary16 RNE is also what numpy implements: an independent check
    on every non-NaN half and a dense f32 sample."""
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    wide = np.empty(65536, np.float32)
    orc.lib.orc_f16_to_f32_array(h.ctypes.data, wide.ctypes.data, 65536)
    ok = ~np.isnan(h.view(np.float16))
    assert np.array_equal(wide[ok], h.view(np.float16)[ok].astype(np.float32))
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2**32, size=2_000_000, dtype=np.uint64).astype(np.uint32)
    f = bits.view(np.float32)
    f = f[~np.isnan(f)]
    narrow = np.empty(f.size, np.uint16)
    orc.lib.orc_f32_to_f16_array(f.ctypes.data, narrow.ctypes.data, f.size)
    with np.errstate(over="ignore"):
        assert np.array_equal(narrow, f.astype(np.float16).view(np.uint16))


def test_nan_payload_rules(orc):
    # sign and top ten payload bits kept; zero payload forced to 1
    # (array entry point: a scalar ctypes float argument would quieten sNaN)
    cases = {0x7f800001: 0x7c01, 0xff800001: 0xfc01, 0x7fc00000: 0x7e00,
             0x7f802000: 0x7c01, 0x7fffe000: 0x7fff}
    f = np.array(list(cases), np.uint32).view(np.float32)
    out = np.empty(f.size, np.uint16)
    orc.lib.orc_f32_to_f16_array(f.ctypes.data, out.ctypes.data, f.size)
    assert out.tolist() == list(cases.values())
    # bf16 quietens NaN
    f = np.array([0x7f800001], np.uint32).view(np.float32)[0]
    assert orc.lib.orc_f32_to_bf16(f) == 0x7fc0


def test_bf16_vs_reference(orc, ref):
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 2**32, size=200_000, dtype=np.uint64).astype(np.uint32)
    f = bits.view(np.float32).copy()
    got = np.array([orc.lib.orc_f32_to_bf16(v) for v in f[:20000]], np.uint16)
    want = ref.convert(f[:20000], "f32", "bf16")
    assert np.array_equal(got, want)
