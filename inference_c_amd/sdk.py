"""ctypes binding of libinference_sdk_hip.so (the C ABI in include/*.h).

This module only marshals arguments: every operation runs in the HIP library.
If the library has not been built, loading fails with an error naming the
missing file; there is no Python fallback for any operation.
"""
from __future__ import annotations

import ctypes
import os
from typing import Iterable, Optional, Sequence

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "lib", "libinference_sdk_hip.so")
REPO = os.path.dirname(HERE)
INCLUDE_DIR = os.path.join(REPO, "include")

# TensorDType values (include/safetensors.h)
DTYPE_CODES = {
    "bool": 1, "u8": 2, "i8": 3, "i16": 4, "u16": 5, "i32": 6, "u32": 7,
    "i64": 8, "u64": 9, "f16": 12, "bf16": 13, "f32": 14, "f64": 15,
}
NUMPY_DTYPES = {
    "bool": np.uint8, "u8": np.uint8, "i8": np.int8, "i16": np.int16, "u16": np.uint16,
    "i32": np.int32, "u32": np.uint32, "i64": np.int64, "u64": np.uint64,
    "f16": np.float16, "bf16": np.uint16, "f32": np.float32, "f64": np.float64,
}
HOST, DEVICE = 0, 1

_P, _F, _D = ctypes.c_void_p, ctypes.c_float, ctypes.c_double
_Z, _I, _U64 = ctypes.c_size_t, ctypes.c_int, ctypes.c_uint64

# Operation signatures, without the trailing (char *error, size_t capacity).
OP_ARGTYPES = {
    "tensor_matmul_f32": [_P, _P, _P], "tensor_matmul_f16": [_P, _P, _P],
    "tensor_linear_f32": [_P, _P, _P, _P], "tensor_linear_f16": [_P, _P, _P, _P],
    "tensor_embedding_lookup_f32": [_P, _P, _P], "tensor_embedding_lookup_f16": [_P, _P, _P],
    "tensor_rms_norm_f32": [_P, _P, _F, _P], "tensor_rms_norm_f16": [_P, _P, _F, _P],
    "tensor_layer_norm_f32": [_P, _P, _P, _F, _P], "tensor_layer_norm_f16": [_P, _P, _P, _F, _P],
    "tensor_silu_f32": [_P, _P], "tensor_silu_f16": [_P, _P],
    "tensor_residual_add_f16": [_P, _P, _P],
    "tensor_add_f32": [_P, _P, _P], "tensor_mul_f32": [_P, _P, _P], "tensor_mul_f16": [_P, _P, _P],
    "tensor_gelu_f32": [_P, _P], "tensor_gelu_f16": [_P, _P],
    "tensor_gelu_multiply_f16": [_P, _P, _P], "tensor_relu_f16": [_P, _P],
    "tensor_silu_multiply_f32": [_P, _P, _P], "tensor_silu_multiply_f16": [_P, _P, _P],
    "tensor_bias_add_f32": [_P, _P, _P], "tensor_bias_add_f16": [_P, _P, _P],
    "tensor_bias_gelu_f32": [_P, _P, _P], "tensor_bias_gelu_f16": [_P, _P, _P],
    "tensor_view_add_mul_f16": [_P, _P, _P, _P, _P], "tensor_view_add_mul_f32": [_P, _P, _P, _P, _P],
    "tensor_softmax_f32": [_P, _I, _P], "tensor_softmax_f16": [_P, _I, _P],
    "tensor_row_sum_f32": [_P, _P], "tensor_row_sum_f16": [_P, _P],
    "tensor_row_max_f32": [_P, _P], "tensor_row_max_f16": [_P, _P],
    "tensor_residual_rms_norm_f16": [_P, _P, _P, _F, _P, _P],
    "tensor_sum_max_f32": [_P, _P, _P], "tensor_sum_max_f32_no_alloc": [_P, _P, _P],
    "tensor_argmax_f32": [_P, _P], "tensor_argmax_f16": [_P, _P],
    "tensor_rope_f32": [_P, _P, _Z, _Z, _Z, _D, _Z], "tensor_rope_f16": [_P, _P, _Z, _Z, _Z, _D, _Z],
    "tensor_fill_uniform": [_P, _U64, _U64, _F, _F], "tensor_fill_normal": [_P, _U64, _U64, _F, _F],
    "tensor_sdpa_device_f32": [_P, _P, _P, _P, _F, _I, _P],
    "tensor_sdpa_device_f16": [_P, _P, _P, _P, _F, _I, _P],
    "tensor_linear_q8_0_f16": [_P, _P, _P], "tensor_linear_q4_0_f16": [_P, _P, _P],
    "tensor_device_synchronize": [],
}


# TensorComputeBackend (include/tensor_compute_backend.h) field order: the
# name, then one function pointer per slot.
COMPUTE_SLOTS = [
    "name", "is_available", "linear_f32", "linear_f16", "embedding_f16", "rms_norm_f16",
    "layer_norm_f16", "bias_add_f16", "gelu_f16", "gelu_multiply_f16", "relu_f16",
    "rope_f16", "silu_multiply_f16", "residual_add_f16", "argmax_f16", "embedding_f32",
    "rms_norm_f32", "rms_norm_linear_f32", "layer_norm_f32", "bias_add_f32", "gelu_f32",
    "rope_f32", "silu_multiply_f32", "residual_add_f32", "argmax_f32", "release_cache",
    "mlp_f32", "mlp_f16", "qkv_f16", "vision_layer_f16", "vision_layer_f32",
    "vision_sequence_begin_f16", "vision_sequence_layer_f16", "vision_sequence_finish_f16",
    "vision_sequence_release_f16", "vision_sequence_layer_quant_f16",
    "vision_sequence_begin_f32", "vision_sequence_layer_f32", "vision_sequence_finish_f32",
    "vision_sequence_release_f32", "linear_f32_device", "linear_f16_device",
    "linear_q8_0_f16_device", "linear_q4_0_f16_device", "linear_q8_0_f16",
    "linear_q4_0_f16", "bias_add_f32_device", "bias_add_f16_device",
    "residual_add_f16_device"]


class ComputeBackend(ctypes.Structure):
    """TensorComputeBackend as raw addresses (NULL slots read as None)."""
    _fields_ = [(s, ctypes.c_void_p) for s in COMPUTE_SLOTS]


class SdkError(RuntimeError):
    """A library call returned 0; the message is the library's error text."""


class TensorView(ctypes.Structure):
    """include/tensor_ops_ext.h TensorView (elements, rank <= 8)."""
    _fields_ = [("rank", ctypes.c_size_t), ("shape", ctypes.c_uint64 * 8),
                ("strides", ctypes.c_int64 * 8), ("offset", ctypes.c_uint64)]

    @classmethod
    def make(cls, shape: Sequence[int], strides: Sequence[int], offset: int = 0) -> "TensorView":
        v = cls()
        v.rank = len(shape)
        for i, (s, t) in enumerate(zip(shape, strides)):
            v.shape[i] = s
            v.strides[i] = t
        v.offset = offset
        return v


def load_library(path: str = LIB_PATH) -> ctypes.CDLL:
    if not os.path.exists(path):
        raise SdkError(f"HIP tensor-ops library not built: {path} "
                       "(run __graft_entry__.build())")
    lib = ctypes.CDLL(path)
    for name, args in OP_ARGTYPES.items():
        fn = getattr(lib, name)
        fn.argtypes = list(args) + [ctypes.c_char_p, ctypes.c_size_t]
        fn.restype = ctypes.c_int
    lib.tensor_device_available.restype = ctypes.c_int
    lib.tensor_device_available.argtypes = []
    lib.tensor_buffer_create.argtypes = [_I, ctypes.POINTER(ctypes.c_uint64), _Z,
                                         ctypes.POINTER(_P), ctypes.c_char_p, _Z]
    lib.tensor_buffer_create_device.argtypes = lib.tensor_buffer_create.argtypes
    lib.tensor_buffer_free.argtypes = [_P]
    lib.tensor_buffer_free.restype = None
    lib.tensor_buffer_upload.argtypes = [_P, _Z, _P, _Z, ctypes.c_char_p, _Z]
    lib.tensor_buffer_download.argtypes = [_P, _Z, _P, _Z, ctypes.c_char_p, _Z]
    lib.tensor_buffer_copy_device.argtypes = [_P, _Z, _P, _Z, _Z, ctypes.c_char_p, _Z]
    lib.tensor_buffer_convert.argtypes = [_P, _I, ctypes.POINTER(_P), ctypes.c_char_p, _Z]
    for name in ("tensor_buffer_data", "tensor_buffer_data_mut",
                 "tensor_buffer_device_handle_internal", "tensor_buffer_shape"):
        getattr(lib, name).argtypes = [_P]
        getattr(lib, name).restype = _P
    for name in ("tensor_buffer_rank", "tensor_buffer_element_count",
                 "tensor_buffer_byte_length"):
        getattr(lib, name).argtypes = [_P]
        getattr(lib, name).restype = _Z
    lib.tensor_buffer_dtype.argtypes = [_P]
    lib.tensor_buffer_dtype.restype = _I
    lib.tensor_buffer_storage.argtypes = [_P]
    lib.tensor_buffer_storage.restype = _I
    lib.tensor_device_hip_stream.argtypes = []
    lib.tensor_device_hip_stream.restype = _P
    for name in ("tensor_compute_preferred_backend", "tensor_compute_hip_backend",
                 "tensor_compute_cuda_backend", "tensor_compute_metal_backend"):
        getattr(lib, name).argtypes = []
        getattr(lib, name).restype = _P
    lib.tensor_f32_to_f16.argtypes = [_F]
    lib.tensor_f32_to_f16.restype = ctypes.c_uint16
    lib.tensor_f16_to_f32.argtypes = [ctypes.c_uint16]
    lib.tensor_f16_to_f32.restype = _F
    lib.tensor_bf16_to_f32.argtypes = [ctypes.c_uint16]
    lib.tensor_bf16_to_f32.restype = _F
    lib.tensor_dtype_size.argtypes = [_I]
    lib.tensor_dtype_size.restype = _Z
    lib.tensor_dtype_name.argtypes = [_I]
    lib.tensor_dtype_name.restype = ctypes.c_char_p
    lib.tensor_quantize_linear_weight_f16.argtypes = [_P, _Z, _Z, _I, ctypes.POINTER(_P),
                                                      ctypes.c_char_p, _Z]
    lib.tensor_quantize_linear_weight_f16.restype = _I
    return lib


class Tensor:
    """Owns one TensorBuffer (host or device storage)."""

    def __init__(self, sdk: "Sdk", dtype: str, shape: Sequence[int], device: bool = True):
        self.sdk, self.dtype, self.shape = sdk, dtype, tuple(int(s) for s in shape)
        self.device = device
        dims = (ctypes.c_uint64 * max(1, len(self.shape)))(*self.shape)
        handle = ctypes.c_void_p()
        err = ctypes.create_string_buffer(512)
        create = sdk.lib.tensor_buffer_create_device if device else sdk.lib.tensor_buffer_create
        if not create(DTYPE_CODES[dtype], dims, len(self.shape), ctypes.byref(handle), err, 512):
            raise SdkError(err.value.decode())
        self.handle = handle.value

    @property
    def nbytes(self) -> int:
        return int(self.sdk.lib.tensor_buffer_byte_length(self.handle))

    @property
    def numel(self) -> int:
        return int(np.prod(self.shape, dtype=np.int64)) if self.shape else 1

    def device_ptr(self) -> int:
        return self.sdk.lib.tensor_buffer_device_handle_internal(self.handle) or 0

    def upload(self, array: np.ndarray) -> "Tensor":
        a = np.ascontiguousarray(array)
        if a.nbytes != self.nbytes:
            raise SdkError(f"upload of {a.nbytes} bytes into a {self.nbytes}-byte tensor")
        err = ctypes.create_string_buffer(512)
        if not self.sdk.lib.tensor_buffer_upload(self.handle, 0, a.ctypes.data, a.nbytes, err, 512):
            raise SdkError(err.value.decode())
        return self

    def download(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=NUMPY_DTYPES[self.dtype])
        err = ctypes.create_string_buffer(512)
        if out.nbytes and not self.sdk.lib.tensor_buffer_download(self.handle, 0, out.ctypes.data,
                                                                  out.nbytes, err, 512):
            raise SdkError(err.value.decode())
        return out

    def download_range(self, first: int, count: int) -> np.ndarray:
        """Elements first .. first + count - 1 of the flattened tensor."""
        dt = np.dtype(NUMPY_DTYPES[self.dtype])
        out = np.empty(count, dtype=dt)
        err = ctypes.create_string_buffer(512)
        if out.nbytes and not self.sdk.lib.tensor_buffer_download(
                self.handle, first * dt.itemsize, out.ctypes.data, out.nbytes, err, 512):
            raise SdkError(err.value.decode())
        return out

    def free(self) -> None:
        if self.handle:
            self.sdk.lib.tensor_buffer_free(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Sdk:
    """Library handle with Tensor construction and checked op calls."""

    def __init__(self, path: str = LIB_PATH):
        self.lib = load_library(path)

    @property
    def available(self) -> bool:
        return bool(self.lib.tensor_device_available())

    def require_device(self) -> None:
        if not self.available:
            raise SdkError("no HIP device: the tensor-ops library needs an MI355X (gfx950)")

    def tensor(self, dtype: str, shape: Sequence[int], device: bool = True) -> Tensor:
        return Tensor(self, dtype, shape, device)

    def from_numpy(self, array: np.ndarray, dtype: Optional[str] = None,
                   device: bool = True) -> Tensor:
        if dtype is None:
            dtype = {np.dtype(np.float32): "f32", np.dtype(np.float16): "f16",
                     np.dtype(np.float64): "f64", np.dtype(np.int16): "i16",
                     np.dtype(np.uint16): "u16", np.dtype(np.int32): "i32",
                     np.dtype(np.uint32): "u32", np.dtype(np.int64): "i64",
                     np.dtype(np.uint64): "u64"}[array.dtype]
        return self.tensor(dtype, array.shape, device).upload(array)

    def call(self, name: str, *args) -> None:
        """Calls op `name`; Tensor arguments are passed as their handles,
        None as NULL. Raises SdkError with the library's message on failure."""
        conv = [self._arg(a) for a in args]
        err = ctypes.create_string_buffer(512)
        if not getattr(self.lib, name)(*conv, err, 512):
            raise SdkError(f"{name}: {err.value.decode()}")

    def try_call(self, name: str, *args) -> tuple[int, str]:
        conv = [self._arg(a) for a in args]
        err = ctypes.create_string_buffer(512)
        ok = getattr(self.lib, name)(*conv, err, 512)
        return ok, err.value.decode()

    @staticmethod
    def _arg(a):
        if isinstance(a, Tensor):
            return a.handle
        if isinstance(a, ctypes.Structure):
            return ctypes.addressof(a)
        return a

    def quantize(self, weight: np.ndarray, fmt: int) -> tuple[int, Optional[np.ndarray], str]:
        """tensor_quantize_linear_weight_f16 on an f16 [out, in] matrix
        (fmt 1 = Q8_0, 2 = Q4_0): (ok, packed uint8 [out, in/32, block], message)."""
        w = np.ascontiguousarray(weight, np.float16)
        result = _P()
        err = ctypes.create_string_buffer(512)
        ok = self.lib.tensor_quantize_linear_weight_f16(w.ctypes.data, w.shape[0], w.shape[1], fmt,
                                                        ctypes.byref(result), err, 512)
        if not ok:
            return 0, None, err.value.decode()
        try:
            shape = ctypes.cast(self.lib.tensor_buffer_shape(result),
                                ctypes.POINTER(ctypes.c_uint64))
            packed = np.empty((shape[0], shape[1], shape[2]), np.uint8)
            ctypes.memmove(packed.ctypes.data, self.lib.tensor_buffer_data(result), packed.nbytes)
            return 1, packed, ""
        finally:
            self.lib.tensor_buffer_free(result)

    def compute_table(self) -> ComputeBackend:
        """The library's "hip" TensorComputeBackend."""
        return ctypes.cast(self.lib.tensor_compute_hip_backend(),
                           ctypes.POINTER(ComputeBackend)).contents

    def synchronize(self) -> None:
        self.call("tensor_device_synchronize")

    def stream(self) -> int:
        return self.lib.tensor_device_hip_stream() or 0


# Headers whose functions the calling program defines (the reference's
# tensor_store.c); the library only references them weakly.
PROGRAM_HEADERS = ("tensor_store.h",)


def declared_functions(include_dir: str = INCLUDE_DIR) -> list[str]:
    """Names of every function the library exports, as declared in include/*.h
    (all headers but PROGRAM_HEADERS)."""
    import re
    names = []
    pattern = re.compile(r"^[A-Za-z_][\w\s\*]*?\b([a-z_][a-z0-9_]*)\s*\(", re.M)
    for fname in sorted(os.listdir(include_dir)):
        if not fname.endswith(".h") or fname in PROGRAM_HEADERS:
            continue
        text = open(os.path.join(include_dir, fname)).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        text = re.sub(r"//[^\n]*", "", text)
        # drop struct bodies (function-pointer members are not exports)
        text = re.sub(r"typedef struct \{.*?\}\s*\w+\s*;", "", text, flags=re.S)
        for m in pattern.finditer(text):
            if m.group(1) not in ("if", "return", "sizeof"):
                names.append(m.group(1))
    return sorted(set(names))
