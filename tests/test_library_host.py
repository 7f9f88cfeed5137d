"""The HIP library on any machine: it loads, exports every function that
include/*.h declares, keeps the reference's struct layouts and enum values,
and its host logic (TensorBuffer bookkeeping, validation messages, backend
selection) behaves like the reference's. No compute call is made here."""
import ctypes
import os
import subprocess

import numpy as np
import pytest

from tests.conftest import REPO

REF_INCLUDE = "/root/reference/include"


def test_every_declared_function_is_exported(lib):
    from inference_c_amd import declared_functions
    names = declared_functions()
    assert len(names) >= 70
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def _layout(include_dir, tmp_path, tag):
    exe = tmp_path / f"abi_{tag}"
    subprocess.run(["gcc", "-std=c11", "-I", include_dir, "-o", str(exe),
                    os.path.join(REPO, "oracle", "abi_layout.c")], check=True)
    return subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout


def test_struct_layout_matches_reference_header(tmp_path):
    if not os.path.isdir(REF_INCLUDE):
        pytest.skip("reference headers absent")
    mine = _layout(os.path.join(REPO, "include"), tmp_path, "mine")
    theirs = _layout(REF_INCLUDE, tmp_path, "ref")
    assert mine == theirs
    assert "sizeof TensorComputeBackend 392" in mine


def test_attention_table_layout_matches_reference_header(tmp_path):
    """include/attention_backend.h keeps the reference's
    src/attention_backend.h layout (the table src/common/attention.c calls)."""
    ref_src = os.path.join(os.path.dirname(REF_INCLUDE), "src")
    if not os.path.isdir(ref_src):
        pytest.skip("reference sources absent")
    probe = os.path.join(REPO, "oracle", "abi_attention.c")

    def layout(include_dirs, tag):
        exe = tmp_path / f"attn_{tag}"
        args = ["gcc", "-std=c11"]
        for d in include_dirs:
            args += ["-I", d]
        subprocess.run(args + ["-o", str(exe), probe], check=True)
        return subprocess.run([str(exe)], capture_output=True, text=True, check=True).stdout

    mine = layout([os.path.join(REPO, "include")], "mine")
    theirs = layout([ref_src, REF_INCLUDE], "ref")
    assert mine == theirs
    assert "TensorAttentionBackendOps.run_f16 32" in mine


def test_attention_table_without_device(lib):
    """The HIP attention table occupies the reference's accelerator slot: its
    name is "hip", only run/run_f16 are filled, and without a device it
    reports itself unavailable."""
    from inference_c_amd import Sdk
    sdk = Sdk()
    lib.tensor_attention_cuda_backend.restype = ctypes.c_void_p
    lib.tensor_attention_hip_backend.restype = ctypes.c_void_p
    table = lib.tensor_attention_cuda_backend()
    assert table and table == lib.tensor_attention_hip_backend()
    slots = ctypes.cast(table, ctypes.POINTER(ctypes.c_void_p))
    assert ctypes.cast(table, ctypes.POINTER(ctypes.c_int))[0] == 2   # TENSOR_ATTENTION_BACKEND_CUDA
    assert ctypes.cast(slots[1], ctypes.c_char_p).value == b"hip"
    assert slots[3] and slots[4]                                      # run, run_f16
    assert not any(slots[i] for i in range(5, 14))                    # decode slots NULL
    if not sdk.available:
        assert ctypes.CFUNCTYPE(ctypes.c_int)(slots[2])() == 0


def test_device_sdpa_rejects_host_tensors(lib):
    from inference_c_amd import Sdk
    sdk = Sdk()
    for dtype in ("f32", "f16"):
        q = sdk.tensor(dtype, (1, 2, 3, 4), device=False)
        ok, msg = sdk.try_call(f"tensor_sdpa_device_{dtype}", q, q, q, None, 1.0, 0, q)
        up = dtype.upper()
        assert not ok and msg == (f"device SDPA requires rank-4 {up} device tensors, finite "
                                  f"scale, and optional rank-2 {up} device mask")


def test_dtype_helpers(lib):
    sizes = {"UNKNOWN": 0, "BOOL": 1, "U8": 1, "I16": 2, "F16": 2, "BF16": 2, "F32": 4,
             "U32": 4, "F64": 8, "U64": 8}
    for code in range(16):
        name = lib.tensor_dtype_name(code).decode()
        if name in sizes:
            assert lib.tensor_dtype_size(code) == sizes[name]
    assert lib.tensor_dtype_name(99).decode() == "UNKNOWN"
    assert lib.tensor_dtype_size(12) == 2 and lib.tensor_dtype_name(12) == b"F16"


def test_host_tensor_buffer_contract(lib):
    from inference_c_amd import Sdk, SdkError
    sdk = Sdk()
    t = sdk.tensor("f32", (2, 5), device=False)
    assert lib.tensor_buffer_rank(t.handle) == 2
    assert lib.tensor_buffer_element_count(t.handle) == 10
    assert lib.tensor_buffer_byte_length(t.handle) == 40
    assert lib.tensor_buffer_storage(t.handle) == 0
    assert lib.tensor_buffer_data(t.handle) and lib.tensor_buffer_device_handle_internal(t.handle) is None
    shape = ctypes.cast(lib.tensor_buffer_shape(t.handle), ctypes.POINTER(ctypes.c_uint64))
    assert [shape[0], shape[1]] == [2, 5]
    a = np.arange(10, dtype=np.float32).reshape(2, 5)
    assert np.array_equal(t.upload(a).download(), a)
    assert np.all(np.frombuffer(ctypes.string_at(lib.tensor_buffer_data(sdk.tensor("u8", (7,), False).handle), 7), np.uint8) == 0)
    err = ctypes.create_string_buffer(256)
    buf = np.zeros(4, np.float32)
    assert not lib.tensor_buffer_upload(t.handle, 36, buf.ctypes.data, 8, err, 256)
    assert err.value == b"invalid tensor upload range or pointer"
    assert not lib.tensor_buffer_download(t.handle, 41, buf.ctypes.data, 0, err, 256)
    assert err.value == b"invalid tensor download range or pointer"
    empty = sdk.tensor("f16", (0, 3), device=False)
    assert lib.tensor_buffer_byte_length(empty.handle) == 0
    with pytest.raises(SdkError, match="invalid tensor buffer dtype, rank, or shape"):
        sdk.tensor("f32", (1,) * 17, device=False)
    with pytest.raises(SdkError, match="exceeds addressable size"):
        sdk.tensor("f32", (1 << 40, 1 << 40), device=False)


def test_store_and_workspace_entry_points_without_that_code_linked(lib):
    """In a process without the reference's tensor_store.c / tensor_workspace.c
    (this Python process) the weak references stay null and both calls fail
    with a message instead of jumping through a null pointer. With that code
    linked, the reference's own test_tensor_store / test_tensor_workspace /
    test_tensor_prefetch exercise them (test_dropin_reference.py)."""
    err = ctypes.create_string_buffer(256)
    res = ctypes.c_void_p(1)
    assert not lib.tensor_buffer_load(None, b"w", ctypes.byref(res), err, 256)
    assert res.value is None
    assert err.value == b"tensor_buffer_load requires tensor_store.c linked into the program"
    res = ctypes.c_void_p(1)
    shape = (ctypes.c_uint64 * 1)(4)
    assert not lib.tensor_buffer_create_in_workspace(14, shape, 1, None, ctypes.byref(res), err, 256)
    assert res.value is None and err.value == b"workspace-backed tensor requires a workspace"
    assert not lib.tensor_buffer_create_in_workspace(14, shape, 1, ctypes.c_void_p(8),
                                                     ctypes.byref(res), err, 256)
    assert res.value is None
    assert err.value == b"workspace-backed tensor requires tensor_workspace.c linked into the program"


def test_linear_and_matmul_validation_matches_reference(lib, ref, orc):
    """tensor_matmul_* / tensor_linear_* refuse bad host operands with the
    reference's messages (src/common/tensor_ops.c:163-398) before any device
    work, and an empty batch succeeds without one."""
    from inference_c_amd import Sdk
    sdk = Sdk()
    f32 = lambda *shape: np.zeros(shape, np.float32)
    f16 = lambda *shape: np.zeros(shape, np.float16)
    cases = [
        ("tensor_matmul_f32", [f32(2, 3), f32(3, 2)], f32(4)),
        ("tensor_matmul_f32", [f32(2, 3), f32(4, 2)], f32(2, 2)),
        ("tensor_matmul_f16", [f16(2, 3), f16(3, 5)], f16(2, 4)),
        ("tensor_linear_f32", [f32(2, 3), f32(3), None], f32(2, 3)),
        ("tensor_linear_f32", [f32(2, 3), f32(4, 3), f32(5)], f32(2, 4)),
        ("tensor_linear_f16", [f16(2, 3), f16(4, 2), None], f16(2, 4)),
        ("tensor_linear_f16", [f16(2, 5, 3), f16(4, 3), None], f16(2, 4, 4)),
        ("tensor_linear_f32", [f32(2, 3), f32(4, 3), f32(4, 1)], f32(2, 4)),
        ("tensor_linear_f32", [f32(2, 0), f32(4, 0), None], f32(2, 4)),
    ]
    for name, operands, out in cases:
        dtype = "f16" if out.dtype == np.float16 else "f32"
        rok, _, rmsg = ref._call(name, operands, out.shape, dtype)
        args = [None if a is None else sdk.from_numpy(a, device=False) for a in operands]
        ok, msg = sdk.try_call(name, *args, sdk.from_numpy(out, device=False))
        assert not rok and not ok and msg == rmsg, (name, msg, rmsg)
    # mixed dtypes within one call
    ok, msg = sdk.try_call("tensor_matmul_f32", sdk.from_numpy(f32(2, 2), device=False),
                           sdk.from_numpy(f16(2, 2), device=False),
                           sdk.from_numpy(f32(2, 2), device=False))
    assert not ok and msg == "matmul requires rank-2 F32 tensors"
    # empty batches: nothing to compute, success with or without a device
    ok, _ = sdk.try_call("tensor_linear_f32", sdk.from_numpy(f32(0, 3), device=False),
                         sdk.from_numpy(f32(4, 3), device=False), None,
                         sdk.from_numpy(f32(0, 4), device=False))
    assert ok
    ok, _ = sdk.try_call("tensor_matmul_f16", sdk.from_numpy(f16(0, 3), device=False),
                         sdk.from_numpy(f16(3, 2), device=False),
                         sdk.from_numpy(f16(0, 2), device=False))
    assert ok
    if not sdk.available:
        ok, msg = sdk.try_call("tensor_matmul_f32", sdk.from_numpy(f32(2, 3), device=False),
                               sdk.from_numpy(f32(3, 2), device=False),
                               sdk.from_numpy(f32(2, 2), device=False))
        assert not ok and msg.startswith("HIP device unavailable")


def test_quantize_refusals_match_reference(lib, ref):
    """tensor_quantize_linear_weight_f16 argument checks (tensor_quant.c:
    48-60): the same message, no result, before any device work."""
    from inference_c_amd import Sdk
    sdk = Sdk()
    message = "quantized linear weight requires a valid format and input width divisible by 32"
    for shape, fmt in (((2, 33), 1), ((2, 64), 3), ((2, 16), 2)):
        w = np.zeros(shape, np.float16)
        rok, _, rmsg = ref.quantize(w, fmt)
        ok, packed, msg = sdk.quantize(w, fmt)
        assert not rok and not ok and packed is None and msg == rmsg == message
    result = ctypes.c_void_p(7)
    err = ctypes.create_string_buffer(256)
    assert not lib.tensor_quantize_linear_weight_f16(None, 2, 32, 1, ctypes.byref(result), err, 256)
    assert result.value is None and err.value.decode() == message


def test_validation_precedes_device_use(lib):
    """The reference's messages (src/common/tensor_ops.c) for bad operands,
    produced before any device is touched."""
    from inference_c_amd import Sdk
    sdk = Sdk()
    x16 = sdk.tensor("f16", (2, 4), device=False)
    w16 = sdk.tensor("f16", (4,), device=False)
    w3 = sdk.tensor("f16", (3,), device=False)
    x32 = sdk.tensor("f32", (2, 4), device=False)
    y16 = sdk.tensor("f16", (2, 4), device=False)
    cases = [
        (("tensor_rms_norm_f16", x16, w16, float("nan"), y16),
         "RMSNorm requires compatible F16 tensors and nonnegative epsilon"),
        (("tensor_rms_norm_f16", x16, w16, -1.0, y16),
         "RMSNorm requires compatible F16 tensors and nonnegative epsilon"),
        (("tensor_rms_norm_f16", x16, w3, 0.0, y16), "RMSNorm weight width does not match input"),
        (("tensor_rms_norm_f32", x16, w16, 0.0, y16),
         "RMSNorm requires compatible F32 tensors and nonnegative epsilon"),
        (("tensor_layer_norm_f16", x16, w3, None, 1e-5, y16),
         "LayerNorm affine parameter width does not match input"),
        (("tensor_silu_f16", x32, y16), "SiLU requires same-shaped F16 tensors"),
        (("tensor_silu_f32", x16, y16), "SiLU requires same-shaped F32 tensors"),
        (("tensor_residual_add_f16", x16, x32, y16), "F16 residual add requires same-shaped F16 tensors"),
        (("tensor_residual_add_f16", x16, w16, y16), "F16 residual add requires same-shaped F16 tensors"),
    ]
    for args, message in cases:
        ok, msg = sdk.try_call(*args)
        assert not ok and msg == message, (args[0], msg)


def test_view_refuses_negative_strides_and_views_outside_the_input(lib):
    """The strided-view kernels address x with unsigned offsets, so the entry
    point refuses negative strides (and views reaching past the input) before
    any device work, whatever the offset."""
    from inference_c_amd import Sdk, TensorView
    sdk = Sdk()
    x = sdk.tensor("f16", (4, 64), device=False)
    y = sdk.tensor("f16", (2, 64), device=False)
    message = ("view add/mul requires non-negative strides, a view that lies inside the input, "
               "and an output of the view's shape")
    for view in (TensorView.make((2, 64), (-64, 1), 128),
                 TensorView.make((2, 64), (-64, 1), (1 << 32) + 64),
                 TensorView.make((2, 64), (64, 1), 192)):
        ok, msg = sdk.try_call("tensor_view_add_mul_f16", x, view, None, None, y)
        assert not ok and msg == message


def test_embedding_validation_matches_reference(lib, ref, orc):
    """tensor_embedding_lookup_* reject bad operands and bad indices with the
    reference's messages (src/common/tensor_ops.c:86-161) before any device
    work: every index of a host call is checked on the host first."""
    from inference_c_amd import Sdk
    sdk = Sdk()
    rows, width = 6, 4
    for dtype, npt in (("f32", np.float32), ("f16", np.float16)):
        table = orc.normal((rows, width), 18, 0, 0.0, 1.0, dtype)
        t = sdk.from_numpy(table, device=False)
        for ids in (np.array([1, -1, 2], np.int32), np.array([1, 6], np.uint16),
                    np.array([0, 1 << 40], np.uint64), np.array([-5], np.int64)):
            ti = sdk.from_numpy(ids, device=False)
            out = sdk.tensor(dtype, (ids.size, width), device=False)
            ok, msg = sdk.try_call(f"tensor_embedding_lookup_{dtype}", t, ti, out)
            rok, _, rmsg = ref.embedding_lookup(table, ids)
            assert not ok and not rok and msg == rmsg, (dtype, ids, msg, rmsg)
        # dimension mismatch and a rank-2 index buffer
        ti = sdk.from_numpy(np.array([0, 1], np.uint32), device=False)
        bad_out = sdk.tensor(dtype, (3, width), device=False)
        ok, msg = sdk.try_call(f"tensor_embedding_lookup_{dtype}", t, ti, bad_out)
        assert not ok and msg == "embedding table and output dimensions do not match"
        ti2 = sdk.from_numpy(np.zeros((2, 1), np.uint32), device=False)
        out = sdk.tensor(dtype, (2, width), device=False)
        ok, msg = sdk.try_call(f"tensor_embedding_lookup_{dtype}", t, ti2, out)
        assert not ok and msg == (f"embedding lookup requires a rank-2 {dtype.upper()} table, "
                                  f"integer rank-1 indices, and rank-2 {dtype.upper()} output")
    # F32 checks the index dtype up front, F16 when it reads the first index
    t32 = sdk.from_numpy(np.zeros((rows, width), np.float32), device=False)
    tf = sdk.from_numpy(np.zeros(2, np.float32), device=False)
    out = sdk.tensor("f32", (2, width), device=False)
    ok, msg = sdk.try_call("tensor_embedding_lookup_f32", t32, tf, out)
    assert not ok and "integer rank-1 indices" in msg
    t16 = sdk.from_numpy(np.zeros((rows, width), np.float16), device=False)
    out16 = sdk.tensor("f16", (2, width), device=False)
    ok, msg = sdk.try_call("tensor_embedding_lookup_f16", t16, tf, out16)
    assert not ok and msg == "embedding index is negative or outside the table"
    # no indices: nothing to gather, success without a device
    te = sdk.from_numpy(np.zeros(0, np.uint32), device=False)
    empty = sdk.tensor("f16", (0, width), device=False)
    assert sdk.try_call("tensor_embedding_lookup_f16", t16, te, empty)[0] == 1


def test_empty_tensors_succeed_without_work(lib):
    from inference_c_amd import Sdk
    sdk = Sdk()
    e = sdk.tensor("f16", (0, 8), device=False)
    w = sdk.tensor("f16", (8,), device=False)
    assert sdk.try_call("tensor_silu_f16", e, e)[0] == 1
    assert sdk.try_call("tensor_residual_add_f16", e, e, e)[0] == 1
    assert sdk.try_call("tensor_rms_norm_f16", e, w, 1e-6, e)[0] == 1


def test_backend_selection_without_device(lib, monkeypatch):
    from inference_c_amd import Sdk
    sdk = Sdk()
    if sdk.available:
        pytest.skip("a HIP device is present; covered by the gpu tests")
    for value in (None, "", "auto", "hip", "cuda", "metal", "qnn", "bogus"):
        if value is None:
            monkeypatch.delenv("TENSOR_BACKEND", raising=False)
        else:
            monkeypatch.setenv("TENSOR_BACKEND", value)
        assert lib.tensor_compute_preferred_backend() is None
    name = ctypes.cast(lib.tensor_compute_hip_backend(), ctypes.POINTER(ctypes.c_char_p))[0]
    assert name == b"hip"
    for getter, label in (("tensor_compute_cuda_backend", b"cuda"), ("tensor_compute_metal_backend", b"metal")):
        table = ctypes.cast(getattr(lib, getter)(), ctypes.POINTER(ctypes.c_void_p))
        assert ctypes.cast(table[0], ctypes.c_char_p).value == label
        assert ctypes.CFUNCTYPE(ctypes.c_int)(table[1])() == 0


def test_compute_without_device_fails_loudly(lib):
    from inference_c_amd import Sdk
    sdk = Sdk()
    if sdk.available:
        pytest.skip("a HIP device is present")
    x = sdk.tensor("f16", (4,), device=False).upload(np.ones(4, np.float16))
    y = sdk.tensor("f16", (4,), device=False)
    ok, msg = sdk.try_call("tensor_silu_f16", x, y)
    assert not ok and msg.startswith("HIP device unavailable")
    ok, msg = sdk.try_call("tensor_residual_add_f16", x, x, y)
    assert not ok and msg.startswith("HIP device unavailable")
    err = ctypes.create_string_buffer(256)
    p = ctypes.c_void_p()
    assert not lib.tensor_device_buffer_create(16, ctypes.byref(p), err, 256)
    assert err.value.startswith(b"HIP device unavailable")
    assert not lib.tensor_device_buffer_create(0, ctypes.byref(p), err, 256)
    assert err.value == b"device buffer size must be nonzero"
    assert lib.tensor_device_hip_stream() is None
