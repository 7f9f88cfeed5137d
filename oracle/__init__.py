"""CPU oracle for the tensor-ops hot path -- TEST INFRASTRUCTURE ONLY.

numpy wrappers over oracle/liboracle.so (the C11 restatement in oracle.c) and
over oracle/_ref/libref.so (the reference's own portable C path, compiled from
/root/reference sources by oracle/Makefile). Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg import this module;
the product library never does.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libref.so")

_P, _F, _D, _Z = ctypes.c_void_p, ctypes.c_float, ctypes.c_double, ctypes.c_size_t
_U64, _U16, _U32, _I = ctypes.c_uint64, ctypes.c_uint16, ctypes.c_uint32, ctypes.c_int

_SIGS = {
    "orc_f16_to_f32": ([_U16], _F), "orc_f32_to_f16": ([_F], _U16),
    "orc_bf16_to_f32": ([_U16], _F), "orc_f32_to_bf16": ([_F], _U16),
    "orc_f16_to_f32_array": ([_P, _P, _Z], None), "orc_f32_to_f16_array": ([_P, _P, _Z], None),
    "orc_f32_to_bf16_array": ([_P, _P, _Z], None),
    "orc_rng_bits": ([_U64, _U64, _U64], _U64),
    "orc_fill_uniform_f32": ([_P, _Z, _U64, _U64, _U64, _F, _F], None),
    "orc_fill_uniform_f16": ([_P, _Z, _U64, _U64, _U64, _F, _F], None),
    "orc_fill_normal_f32": ([_P, _Z, _U64, _U64, _U64, _F, _F], None),
    "orc_fill_normal_f16": ([_P, _Z, _U64, _U64, _U64, _F, _F], None),
    "orc_add_f32": ([_P, _P, _P, _Z], None), "orc_mul_f32": ([_P, _P, _P, _Z], None),
    "orc_add_f16": ([_P, _P, _P, _Z], None), "orc_mul_f16": ([_P, _P, _P, _Z], None),
    "orc_silu_f32": ([_P, _P, _Z], None), "orc_silu_f16": ([_P, _P, _Z], None),
    "orc_gelu_scalar": ([_F], _F), "orc_gelu_scalar_f64": ([_D], _D),
    "orc_gelu_f32": ([_P, _P, _Z], None), "orc_gelu_f16": ([_P, _P, _Z], None),
    "orc_gelu_f64": ([_P, _P, _Z], None),
    "orc_gelu_multiply_f16": ([_P, _P, _P, _Z], None), "orc_relu_f16": ([_P, _P, _Z], None),
    "orc_silu_multiply_f32": ([_P, _P, _P, _Z], None),
    "orc_silu_multiply_f16": ([_P, _P, _P, _Z], None),
    "orc_bias_add_f32": ([_P, _P, _P, _Z, _Z, _I], None),
    "orc_bias_add_f16": ([_P, _P, _P, _Z, _Z, _I], None),
    "orc_rms_norm_f32": ([_P, _P, _P, _Z, _Z, _F], None),
    "orc_rms_norm_f16": ([_P, _P, _P, _Z, _Z, _F], None),
    "orc_layer_norm_f32": ([_P, _P, _P, _P, _Z, _Z, _F], None),
    "orc_layer_norm_f16": ([_P, _P, _P, _P, _Z, _Z, _F], None),
    "orc_residual_rms_norm_f16": ([_P, _P, _P, _P, _P, _Z, _Z, _F], None),
    "orc_softmax_f32": ([_P, _P, _Z, _Z, _Z], None), "orc_softmax_f16": ([_P, _P, _Z, _Z, _Z], None),
    "orc_row_sum_f32": ([_P, _P, _P, _Z, _Z], None), "orc_row_sum_f16": ([_P, _P, _P, _Z, _Z], None),
    "orc_row_max_f32": ([_P, _P, _Z, _Z], None), "orc_row_max_f16": ([_P, _P, _Z, _Z], None),
    "orc_sum_max_f32": ([_P, _Z, _P, _P, _P], None),
    "orc_argmax_f32": ([_P, _Z], _U32), "orc_argmax_f16": ([_P, _Z], _U32),
    "orc_rope_f32": ([_P, _P, _Z, _Z, _Z, _Z, _D, _Z], None),
    "orc_rope_f16": ([_P, _P, _Z, _Z, _Z, _Z, _D, _Z], None),
    "orc_view_add_mul_f16": ([_P, _Z, _P, _P, _U64, _P, _P, _P, _P, _P], None),
    "orc_view_add_mul_f32": ([_P, _Z, _P, _P, _U64, _P, _P, _P, _P, _P], None),
    "orc_embedding_lookup": ([_P, _Z, _Z, _P, _I, _Z, _P], _I),
    "orc_embedding_gather_u32": ([_P, _Z, _Z, _P, _Z, _P], None),
    "orc_sdpa_f32": ([_P] * 5 + [_Z] * 7 + [_F, _I, _P], None),
    "orc_sdpa_f16": ([_P] * 5 + [_Z] * 7 + [_F, _I, _P], None),
    "orc_sdpa_abs_weight": ([_P] * 5 + [_I] + [_Z] * 7 + [_F, _I, _P], None),
    "orc_matmul_f32": ([_P, _P, _P, _Z, _Z, _Z], None),
    "orc_matmul_f16": ([_P, _P, _P, _Z, _Z, _Z], None),
    "orc_linear_f32": ([_P, _P, _P, _P, _Z, _Z, _Z], None),
    "orc_linear_f16": ([_P, _P, _P, _P, _Z, _Z, _Z], None),
    "orc_quant_scale_to_f16": ([_F], _U16),
    "orc_quantize_f16": ([_P, _Z, _Z, _I, _P], _I),
    "orc_linear_quant_f16": ([_P, _P, _P, _Z, _Z, _Z, _I], None),
    "orc_linear_quant_abs_weight": ([_P, _P, _P, _Z, _Z, _Z, _I], None),
}

# bytes per 32-weight block of each TensorWeightQuantization format
QUANT_BLOCK_BYTES = {1: 34, 2: 18}

# TensorDType numbering (include/safetensors.h) of numpy index and value types
INDEX_DTYPES = {np.dtype(np.int16): 4, np.dtype(np.uint16): 5, np.dtype(np.int32): 6,
                np.dtype(np.uint32): 7, np.dtype(np.int64): 8, np.dtype(np.uint64): 9,
                np.dtype(np.float16): 12, np.dtype(np.float32): 14}


def _ptr(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data


def _h(a: np.ndarray) -> np.ndarray:
    """f16 array as contiguous uint16 bits."""
    return np.ascontiguousarray(a).view(np.uint16) if a.dtype == np.float16 else np.ascontiguousarray(a)


class Oracle:
    """numpy-level interface to liboracle.so. f16 arrays are np.float16."""

    def __init__(self, path: str = ORACLE_PATH):
        if not os.path.exists(path):
            raise FileNotFoundError(f"oracle library not built: {path} (make -C oracle)")
        self.lib = ctypes.CDLL(path)
        for name, (args, res) in _SIGS.items():
            fn = getattr(self.lib, name)
            fn.argtypes, fn.restype = args, res

    # ---- synthetic inputs ----
    def uniform(self, shape, seed, stream, low, high, dtype="f32", first=0):
        n = int(np.prod(shape))
        if dtype == "f32":
            out = np.empty(n, np.float32)
            self.lib.orc_fill_uniform_f32(out.ctypes.data, n, seed, stream, first, low, high)
        else:
            out = np.empty(n, np.uint16)
            self.lib.orc_fill_uniform_f16(out.ctypes.data, n, seed, stream, first, low, high)
            out = out.view(np.float16)
        return out.reshape(shape)

    def normal(self, shape, seed, stream, mean, std, dtype="f16", first=0):
        n = int(np.prod(shape))
        if dtype == "f32":
            out = np.empty(n, np.float32)
            self.lib.orc_fill_normal_f32(out.ctypes.data, n, seed, stream, first, mean, std)
        else:
            out = np.empty(n, np.uint16)
            self.lib.orc_fill_normal_f16(out.ctypes.data, n, seed, stream, first, mean, std)
            out = out.view(np.float16)
        return out.reshape(shape)

    # ---- conversions (bit patterns in, bit patterns out) ----
    def f16_to_f32(self, bits):
        bits = np.ascontiguousarray(bits, np.uint16)
        out = np.empty(bits.shape, np.float32)
        self.lib.orc_f16_to_f32_array(bits.ctypes.data, out.ctypes.data, bits.size)
        return out

    def f32_to_f16(self, values):
        values = np.ascontiguousarray(values, np.float32)
        out = np.empty(values.shape, np.uint16)
        self.lib.orc_f32_to_f16_array(values.ctypes.data, out.ctypes.data, values.size)
        return out

    def f32_to_bf16(self, values):
        values = np.ascontiguousarray(values, np.float32)
        out = np.empty(values.shape, np.uint16)
        self.lib.orc_f32_to_bf16_array(values.ctypes.data, out.ctypes.data, values.size)
        return out

    # ---- elementwise ----
    def _map(self, name, out_dtype, *arrays):
        arrays = [_h(a) for a in arrays]
        out = np.empty(arrays[0].shape, np.uint16 if out_dtype == np.float16 else out_dtype)
        getattr(self.lib, name)(*[a.ctypes.data for a in arrays], out.ctypes.data, arrays[0].size)
        return out.view(np.float16) if out_dtype == np.float16 else out

    def add(self, a, b):
        return self._map("orc_add_f16" if a.dtype == np.float16 else "orc_add_f32", a.dtype.type, a, b)

    def mul(self, a, b):
        return self._map("orc_mul_f16" if a.dtype == np.float16 else "orc_mul_f32", a.dtype.type, a, b)

    def silu(self, x):
        return self._map("orc_silu_f16" if x.dtype == np.float16 else "orc_silu_f32", x.dtype.type, x)

    def gelu(self, x):
        return self._map("orc_gelu_f16" if x.dtype == np.float16 else "orc_gelu_f32", x.dtype.type, x)

    def gelu_f64(self, x):
        return self._map("orc_gelu_f64", np.float64, np.ascontiguousarray(x, np.float64))

    def gelu_multiply(self, x, gate):
        return self._map("orc_gelu_multiply_f16", np.float16, x, gate)

    def relu(self, x):
        return self._map("orc_relu_f16", np.float16, x)

    def silu_multiply(self, gate, up):
        if gate.dtype == np.float16:
            return self._map("orc_silu_multiply_f16", np.float16, gate, up)
        return self._map("orc_silu_multiply_f32", np.float32, gate, up)

    def bias_add(self, x, bias, gelu=False):
        width = bias.size
        rows = x.size // width
        xs, bs = _h(x), _h(bias)
        out = np.empty(x.shape, xs.dtype)
        name = "orc_bias_add_f16" if x.dtype == np.float16 else "orc_bias_add_f32"
        getattr(self.lib, name)(xs.ctypes.data, bs.ctypes.data, out.ctypes.data, rows, width, int(gelu))
        return out.view(np.float16) if x.dtype == np.float16 else out

    # ---- rows ----
    def rms_norm(self, x, w, eps):
        width = x.shape[-1]
        xs, ws = _h(x), _h(w)
        out = np.empty(x.shape, xs.dtype)
        name = "orc_rms_norm_f16" if x.dtype == np.float16 else "orc_rms_norm_f32"
        getattr(self.lib, name)(xs.ctypes.data, ws.ctypes.data, out.ctypes.data, x.size // width, width, eps)
        return out.view(np.float16) if x.dtype == np.float16 else out

    def layer_norm(self, x, scale, bias, eps):
        width = x.shape[-1]
        xs = _h(x)
        ss = None if scale is None else _h(scale)
        bs = None if bias is None else _h(bias)
        out = np.empty(x.shape, xs.dtype)
        name = "orc_layer_norm_f16" if x.dtype == np.float16 else "orc_layer_norm_f32"
        getattr(self.lib, name)(xs.ctypes.data, _ptr(ss), _ptr(bs), out.ctypes.data,
                                x.size // width, width, eps)
        return out.view(np.float16) if x.dtype == np.float16 else out

    def residual_rms_norm(self, x, r, w, eps):
        width = x.shape[-1]
        xs, rs, ws = _h(x), _h(r), _h(w)
        s = np.empty(x.shape, np.uint16)
        y = np.empty(x.shape, np.uint16)
        self.lib.orc_residual_rms_norm_f16(xs.ctypes.data, rs.ctypes.data, ws.ctypes.data,
                                           s.ctypes.data, y.ctypes.data, x.size // width, width, eps)
        return s.view(np.float16), y.view(np.float16)

    def softmax(self, x, causal=False):
        width = x.shape[-1]
        q_len = x.shape[-2] if causal else 0
        xs = _h(x)
        out = np.empty(x.shape, xs.dtype)
        name = "orc_softmax_f16" if x.dtype == np.float16 else "orc_softmax_f32"
        getattr(self.lib, name)(xs.ctypes.data, out.ctypes.data, x.size // width, width, q_len)
        return out.view(np.float16) if x.dtype == np.float16 else out

    def row_sum(self, x):
        """(sum as float64, sum |x| as float64) per row."""
        width = x.shape[-1]
        rows = x.size // width
        xs = _h(x)
        s = np.empty(rows, np.float64)
        a = np.empty(rows, np.float64)
        name = "orc_row_sum_f16" if x.dtype == np.float16 else "orc_row_sum_f32"
        getattr(self.lib, name)(xs.ctypes.data, s.ctypes.data, a.ctypes.data, rows, width)
        return s, a

    def row_max(self, x):
        width = x.shape[-1]
        rows = x.size // width
        xs = _h(x)
        out = np.empty(rows, np.float32)
        name = "orc_row_max_f16" if x.dtype == np.float16 else "orc_row_max_f32"
        getattr(self.lib, name)(xs.ctypes.data, out.ctypes.data, rows, width)
        return out

    # ---- whole tensor ----
    def sum_max(self, x):
        x = np.ascontiguousarray(x, np.float32)
        s, a, m = ctypes.c_double(), ctypes.c_double(), ctypes.c_float()
        self.lib.orc_sum_max_f32(x.ctypes.data, x.size, ctypes.byref(s), ctypes.byref(a), ctypes.byref(m))
        return s.value, a.value, np.float32(m.value)

    def argmax(self, x):
        xs = _h(x)
        name = "orc_argmax_f16" if x.dtype == np.float16 else "orc_argmax_f32"
        return int(getattr(self.lib, name)(xs.ctypes.data, x.size))

    # ---- rope ----
    def rope(self, q, k, qh, kh, dim, theta, offset=0):
        qs, ks = _h(q).copy(), _h(k).copy()
        seq = q.size // (qh * dim)
        name = "orc_rope_f16" if q.dtype == np.float16 else "orc_rope_f32"
        getattr(self.lib, name)(qs.ctypes.data, ks.ctypes.data, seq, qh, kh, dim, theta, offset)
        if q.dtype == np.float16:
            return qs.view(np.float16), ks.view(np.float16)
        return qs, ks

    # ---- views ----
    def view_add_mul(self, x, shape, strides, offset=0, addend=None, mult=None):
        rank = len(shape)
        shp = np.array(shape, np.uint64)
        st = np.array(strides, np.int64)
        xs = _h(x.reshape(-1))
        ad = None if addend is None else _h(addend)
        mu = None if mult is None else _h(mult)
        ash = None if addend is None else np.array(addend.shape, np.uint64)
        msh = None if mult is None else np.array(mult.shape, np.uint64)
        out = np.empty(tuple(shape), xs.dtype)
        name = "orc_view_add_mul_f16" if x.dtype == np.float16 else "orc_view_add_mul_f32"
        getattr(self.lib, name)(xs.ctypes.data, rank, shp.ctypes.data, st.ctypes.data, offset,
                                _ptr(ad), _ptr(ash), _ptr(mu), _ptr(msh), out.ctypes.data)
        return out.view(np.float16) if x.dtype == np.float16 else out

    def embedding_lookup(self, table, indices):
        """Rows of `table` [rows, width] picked by `indices` (any numpy dtype;
        the reference accepts int16/uint16/int32/uint32/int64/uint64), or
        None when the reference would fail (an index unreadable, negative or
        outside the table)."""
        t = np.ascontiguousarray(table)
        ids = np.ascontiguousarray(indices)
        out = np.zeros((ids.size, t.shape[1]), t.dtype)
        ok = self.lib.orc_embedding_lookup(t.ctypes.data, t.shape[0], t.shape[1] * t.itemsize,
                                           ids.ctypes.data, INDEX_DTYPES.get(ids.dtype, 0),
                                           ids.size, out.ctypes.data)
        return out if ok else None

    @staticmethod
    def _sdpa_dims(q, k, v):
        batch, qh, ql, dim = q.shape
        _, kvh, kl, _ = k.shape
        return batch, qh, kvh, ql, kl, dim, v.shape[3]

    def sdpa(self, q, k, v, mask, scale, causal):
        """Accelerator-semantics attention (f16 in -> f16 out, f32 -> f32)."""
        dims = self._sdpa_dims(q, k, v)
        f16 = q.dtype == np.float16
        qs, ks, vs = _h(q), _h(k), _h(v)
        ms = None if mask is None else _h(mask)
        out = np.empty(dims[:2] + (dims[3], dims[6]), qs.dtype)
        scratch = np.empty(max(1, dims[4]), np.float32)
        name = "orc_sdpa_f16" if f16 else "orc_sdpa_f32"
        getattr(self.lib, name)(qs.ctypes.data, ks.ctypes.data, vs.ctypes.data, _ptr(ms),
                                out.ctypes.data, *dims, scale, int(causal), scratch.ctypes.data)
        return out.view(np.float16) if f16 else out

    def sdpa_abs_weight(self, q, k, v, mask, scale, causal):
        """sum_j p_j |v_j| per output element (f64), the error scale of a
        reordered accumulation."""
        dims = self._sdpa_dims(q, k, v)
        qs, ks, vs = _h(q), _h(k), _h(v)
        ms = None if mask is None else _h(mask)
        out = np.empty(dims[:2] + (dims[3], dims[6]), np.float64)
        scratch = np.empty(max(1, dims[4]), np.float32)
        self.lib.orc_sdpa_abs_weight(qs.ctypes.data, ks.ctypes.data, vs.ctypes.data, _ptr(ms),
                                     out.ctypes.data, int(q.dtype == np.float16), *dims, scale,
                                     int(causal), scratch.ctypes.data)
        return out

    def matmul(self, a, b):
        """tensor_matmul_* host loop: [rows, inner] x [inner, cols]."""
        f16 = a.dtype == np.float16
        out = np.empty((a.shape[0], b.shape[1]), np.uint16 if f16 else np.float32)
        name = "orc_matmul_f16" if f16 else "orc_matmul_f32"
        getattr(self.lib, name)(_h(a).ctypes.data, _h(b).ctypes.data, out.ctypes.data,
                                a.shape[0], a.shape[1], b.shape[1])
        return out.view(np.float16) if f16 else out

    def linear(self, x, w, bias=None):
        """tensor_linear_* host loop: x [..., in] times w [out, in]^T plus bias."""
        f16 = x.dtype == np.float16
        rows = int(np.prod(x.shape[:-1]))
        out = np.empty(x.shape[:-1] + (w.shape[0],), np.uint16 if f16 else np.float32)
        name = "orc_linear_f16" if f16 else "orc_linear_f32"
        getattr(self.lib, name)(_h(x).ctypes.data, _h(w).ctypes.data,
                                None if bias is None else _h(bias).ctypes.data, out.ctypes.data,
                                rows, w.shape[1], w.shape[0])
        return out.view(np.float16) if f16 else out

    def quantize(self, w, fmt):
        """tensor_quantize_linear_weight_f16: packed uint8 [out, in/32, block]
        for an f16 [out, in] matrix, or None when refused."""
        out, inw = w.shape
        if inw % 32:
            return None
        packed = np.zeros((out, inw // 32, QUANT_BLOCK_BYTES[fmt]), np.uint8)
        ok = self.lib.orc_quantize_f16(_h(w).ctypes.data, out, inw, fmt, packed.ctypes.data)
        return packed if ok else None

    def linear_quant(self, x, packed, q8):
        """The CUDA backend's quantized linear: f16 x [..., in], packed
        weights [out, in/32, block] -> f16 [..., out]."""
        rows, inw = int(np.prod(x.shape[:-1])), x.shape[-1]
        out = np.empty(x.shape[:-1] + (packed.shape[0],), np.uint16)
        self.lib.orc_linear_quant_f16(_h(x).ctypes.data, np.ascontiguousarray(packed).ctypes.data,
                                      out.ctypes.data, rows, inw, packed.shape[0], int(q8))
        return out.view(np.float16)

    def linear_quant_abs_weight(self, x, packed, q8):
        rows, inw = int(np.prod(x.shape[:-1])), x.shape[-1]
        out = np.empty(x.shape[:-1] + (packed.shape[0],), np.float64)
        self.lib.orc_linear_quant_abs_weight(_h(x).ctypes.data,
                                             np.ascontiguousarray(packed).ctypes.data,
                                             out.ctypes.data, rows, inw, packed.shape[0], int(q8))
        return out

    def embedding_gather_u32(self, table, ids):
        """Compute-table slot semantics: uint32 ids, zero rows past the table."""
        t = np.ascontiguousarray(table)
        i = np.ascontiguousarray(ids, np.uint32)
        out = np.empty((i.size, t.shape[1]), t.dtype)
        self.lib.orc_embedding_gather_u32(t.ctypes.data, t.shape[0], t.shape[1] * t.itemsize,
                                          i.ctypes.data, i.size, out.ctypes.data)
        return out


class Reference:
    """The reference's portable C path (oracle/_ref/libref.so), driven through
    its own public API: host TensorBuffers and tensor_ops functions."""

    DT = {"f32": 14, "f16": 12, "bf16": 13, "u32": 7}

    def __init__(self, path: str = REF_PATH):
        if not os.path.exists(path):
            raise FileNotFoundError(f"reference build absent: {path} (make -C oracle ref)")
        lib = ctypes.CDLL(path)
        lib.tensor_buffer_create.argtypes = [_I, ctypes.POINTER(_U64), _Z, ctypes.POINTER(_P),
                                             ctypes.c_char_p, _Z]
        lib.tensor_buffer_data_mut.argtypes = [_P]
        lib.tensor_buffer_data_mut.restype = _P
        lib.tensor_buffer_free.argtypes = [_P]
        lib.tensor_buffer_free.restype = None
        lib.tensor_buffer_convert.argtypes = [_P, _I, ctypes.POINTER(_P), ctypes.c_char_p, _Z]
        lib.tensor_buffer_byte_length.argtypes = [_P]
        lib.tensor_buffer_byte_length.restype = _Z
        lib.tensor_f32_to_f16.argtypes = [_F]
        lib.tensor_f32_to_f16.restype = _U16
        lib.tensor_f16_to_f32.argtypes = [_U16]
        lib.tensor_f16_to_f32.restype = _F
        lib.tensor_workspace_create.argtypes = [_Z, ctypes.POINTER(_P), ctypes.c_char_p, _Z]
        lib.tensor_workspace_free.argtypes = [_P]
        lib.tensor_workspace_free.restype = None
        lib.tensor_sdpa_f32.argtypes = [_P, _P, _P, _P, _F, _I, _P, _P, _P, ctypes.c_char_p, _Z]
        for name in ("tensor_rms_norm_f32", "tensor_rms_norm_f16"):
            getattr(lib, name).argtypes = [_P, _P, _F, _P, ctypes.c_char_p, _Z]
        for name in ("tensor_layer_norm_f32", "tensor_layer_norm_f16"):
            getattr(lib, name).argtypes = [_P, _P, _P, _F, _P, ctypes.c_char_p, _Z]
        for name in ("tensor_silu_f32", "tensor_silu_f16"):
            getattr(lib, name).argtypes = [_P, _P, ctypes.c_char_p, _Z]
        lib.tensor_residual_add_f16.argtypes = [_P, _P, _P, ctypes.c_char_p, _Z]
        for name in ("tensor_embedding_lookup_f32", "tensor_embedding_lookup_f16",
                     "tensor_matmul_f32", "tensor_matmul_f16"):
            getattr(lib, name).argtypes = [_P, _P, _P, ctypes.c_char_p, _Z]
        for name in ("tensor_linear_f32", "tensor_linear_f16"):
            getattr(lib, name).argtypes = [_P, _P, _P, _P, ctypes.c_char_p, _Z]
        lib.tensor_quantize_linear_weight_f16.argtypes = [_P, _Z, _Z, _I, ctypes.POINTER(_P),
                                                          ctypes.c_char_p, _Z]
        lib.tensor_buffer_shape.argtypes = [_P]
        lib.tensor_buffer_shape.restype = ctypes.POINTER(_U64)
        self.lib = lib

    def _make(self, dtype, array):
        a = _h(np.ascontiguousarray(array))
        shape = (ctypes.c_uint64 * max(1, a.ndim))(*a.shape)
        handle = ctypes.c_void_p()
        err = ctypes.create_string_buffer(256)
        assert self.lib.tensor_buffer_create(self.DT[dtype], shape, a.ndim, ctypes.byref(handle), err, 256), err.value
        ctypes.memmove(self.lib.tensor_buffer_data_mut(handle), a.ctypes.data, a.nbytes)
        return handle.value

    def _read(self, handle, shape, dtype):
        out = np.empty(shape, np.uint16 if dtype == "f16" else np.float32)
        ctypes.memmove(out.ctypes.data, self.lib.tensor_buffer_data_mut(handle), out.nbytes)
        return out.view(np.float16) if dtype == "f16" else out

    def unary(self, name, x):
        dtype = "f16" if x.dtype == np.float16 else "f32"
        hx, hy = self._make(dtype, x), self._make(dtype, np.zeros_like(x))
        err = ctypes.create_string_buffer(256)
        try:
            assert getattr(self.lib, name)(hx, hy, err, 256), err.value
            return self._read(hy, x.shape, dtype)
        finally:
            self.lib.tensor_buffer_free(hx)
            self.lib.tensor_buffer_free(hy)

    def silu(self, x):
        return self.unary("tensor_silu_f16" if x.dtype == np.float16 else "tensor_silu_f32", x)

    def residual_add_f16(self, a, b):
        ha, hb, hy = self._make("f16", a), self._make("f16", b), self._make("f16", np.zeros_like(a))
        err = ctypes.create_string_buffer(256)
        try:
            assert self.lib.tensor_residual_add_f16(ha, hb, hy, err, 256), err.value
            return self._read(hy, a.shape, "f16")
        finally:
            for h in (ha, hb, hy):
                self.lib.tensor_buffer_free(h)

    def rms_norm(self, x, w, eps):
        dtype = "f16" if x.dtype == np.float16 else "f32"
        hx, hw, hy = self._make(dtype, x), self._make(dtype, w), self._make(dtype, np.zeros_like(x))
        err = ctypes.create_string_buffer(256)
        try:
            name = "tensor_rms_norm_f16" if dtype == "f16" else "tensor_rms_norm_f32"
            assert getattr(self.lib, name)(hx, hw, eps, hy, err, 256), err.value
            return self._read(hy, x.shape, dtype)
        finally:
            for h in (hx, hw, hy):
                self.lib.tensor_buffer_free(h)

    def layer_norm(self, x, scale, bias, eps):
        dtype = "f16" if x.dtype == np.float16 else "f32"
        hx, hy = self._make(dtype, x), self._make(dtype, np.zeros_like(x))
        hs = None if scale is None else self._make(dtype, scale)
        hb = None if bias is None else self._make(dtype, bias)
        err = ctypes.create_string_buffer(256)
        try:
            name = "tensor_layer_norm_f16" if dtype == "f16" else "tensor_layer_norm_f32"
            assert getattr(self.lib, name)(hx, hs, hb, eps, hy, err, 256), err.value
            return self._read(hy, x.shape, dtype)
        finally:
            for h in (hx, hs, hb, hy):
                if h is not None:
                    self.lib.tensor_buffer_free(h)

    def softmax_rows_f32(self, scores, causal):
        """Row softmax of a [q_len, k_len] f32 score matrix through the
        reference's tensor_sdpa_f32 with scale 1, K = 2I and V = I
        (head_dim = value_dim = k_len), so every score is one exact product
        and every output the probability itself:
          finite s -> Q = s/2 (exact for normal floats),
          +inf     -> Q = 3e38, whose product with 2 overflows to +inf,
          -inf     -> Q = 0 and -inf in the additive mask.
        NaN scores cannot be produced this way (NaN * 0 poisons the row)."""
        q_len, k_len = scores.shape
        s = np.ascontiguousarray(scores, np.float32)
        if np.isnan(s).any():
            raise ValueError("NaN scores are not reachable through tensor_sdpa_f32")
        q = np.where(np.isposinf(s), np.float32(3e38), np.where(np.isneginf(s), 0, s * 0.5))
        q = q.astype(np.float32).reshape(1, 1, q_len, k_len)
        mask = np.where(np.isneginf(s), np.float32(-np.inf), np.float32(0)).astype(np.float32)
        two_eye = (2 * np.eye(k_len, dtype=np.float32)).reshape(1, 1, k_len, k_len)
        eye = np.eye(k_len, dtype=np.float32).reshape(1, 1, k_len, k_len)
        hq, hk, hv = self._make("f32", q), self._make("f32", two_eye), self._make("f32", eye)
        hm = self._make("f32", mask)
        ho = self._make("f32", np.zeros((1, 1, q_len, k_len), np.float32))
        ws = ctypes.c_void_p()
        err = ctypes.create_string_buffer(256)
        assert self.lib.tensor_workspace_create(q_len * k_len * 4 + 4096, ctypes.byref(ws), err, 256), err.value
        try:
            assert self.lib.tensor_sdpa_f32(hq, hk, hv, hm, 1.0, int(causal), ho, ws, None, err, 256), err.value
            return self._read(ho, (q_len, k_len), "f32")
        finally:
            for h in (hq, hk, hv, hm, ho):
                self.lib.tensor_buffer_free(h)
            self.lib.tensor_workspace_free(ws)

    def embedding_lookup(self, table, indices):
        """tensor_embedding_lookup_f32/f16 on host buffers: (ok, rows, message)."""
        dtype = "f16" if table.dtype == np.float16 else "f32"
        ids = np.ascontiguousarray(indices)
        shape = (ctypes.c_uint64 * 1)(ids.size)
        hi = ctypes.c_void_p()
        err = ctypes.create_string_buffer(256)
        assert self.lib.tensor_buffer_create(INDEX_DTYPES[ids.dtype], shape, 1, ctypes.byref(hi),
                                             err, 256), err.value
        if ids.nbytes:
            ctypes.memmove(self.lib.tensor_buffer_data_mut(hi), ids.ctypes.data, ids.nbytes)
        ht = self._make(dtype, table)
        ho = self._make(dtype, np.zeros((ids.size, table.shape[1]), table.dtype))
        try:
            name = f"tensor_embedding_lookup_{dtype}"
            ok = bool(getattr(self.lib, name)(ht, hi.value, ho, err, 256))
            return ok, self._read(ho, (ids.size, table.shape[1]), dtype), err.value.decode()
        finally:
            for h in (ht, hi.value, ho):
                self.lib.tensor_buffer_free(h)

    def sdpa_f32(self, q, k, v, mask, scale, causal):
        """tensor_sdpa_f32 of the reference build (its CPU path: no accelerator
        backend is linked): (ok, out, message)."""
        hq, hk, hv = self._make("f32", q), self._make("f32", k), self._make("f32", v)
        hm = None if mask is None else self._make("f32", mask)
        shape = q.shape[:3] + (v.shape[3],)
        ho = self._make("f32", np.zeros(shape, np.float32))
        ws = ctypes.c_void_p()
        err = ctypes.create_string_buffer(256)
        assert self.lib.tensor_workspace_create(q.shape[2] * k.shape[2] * 4 + 4096,
                                                ctypes.byref(ws), err, 256), err.value
        try:
            ok = bool(self.lib.tensor_sdpa_f32(hq, hk, hv, hm, scale, int(causal), ho, ws, None,
                                               err, 256))
            return ok, self._read(ho, shape, "f32"), err.value.decode()
        finally:
            for h in (hq, hk, hv, hm, ho):
                if h is not None:
                    self.lib.tensor_buffer_free(h)
            self.lib.tensor_workspace_free(ws)

    def _call(self, name, operands, out_shape, dtype):
        """Runs a tensor_ops entry point on host buffers: (ok, out, message)."""
        handles = [None if a is None else self._make(dtype, a) for a in operands]
        ho = self._make(dtype, np.zeros(out_shape, np.float16 if dtype == "f16" else np.float32))
        err = ctypes.create_string_buffer(256)
        try:
            ok = bool(getattr(self.lib, name)(*handles, ho, err, 256))
            return ok, self._read(ho, out_shape, dtype), err.value.decode()
        finally:
            for h in handles + [ho]:
                if h is not None:
                    self.lib.tensor_buffer_free(h)

    def matmul(self, a, b):
        dtype = "f16" if a.dtype == np.float16 else "f32"
        return self._call(f"tensor_matmul_{dtype}", [a, b], (a.shape[0], b.shape[1]), dtype)

    def linear(self, x, w, bias=None):
        dtype = "f16" if x.dtype == np.float16 else "f32"
        return self._call(f"tensor_linear_{dtype}", [x, w, bias], x.shape[:-1] + (w.shape[0],),
                          dtype)

    def quantize(self, w, fmt):
        """tensor_quantize_linear_weight_f16: (ok, packed uint8 or None, message)."""
        bits = _h(np.ascontiguousarray(w, np.float16))
        result = _P()
        err = ctypes.create_string_buffer(256)
        ok = bool(self.lib.tensor_quantize_linear_weight_f16(bits.ctypes.data, w.shape[0],
                                                              w.shape[1], fmt,
                                                              ctypes.byref(result), err, 256))
        if not ok:
            return False, None, err.value.decode()
        try:
            shape = self.lib.tensor_buffer_shape(result)
            dims = (shape[0], shape[1], shape[2])
            packed = np.empty(dims, np.uint8)
            ctypes.memmove(packed.ctypes.data, self.lib.tensor_buffer_data_mut(result), packed.nbytes)
            return True, packed, ""
        finally:
            self.lib.tensor_buffer_free(result)

    def convert(self, array, src, dst):
        h = self._make(src, array)
        out = ctypes.c_void_p()
        err = ctypes.create_string_buffer(256)
        try:
            assert self.lib.tensor_buffer_convert(h, self.DT[dst], ctypes.byref(out), err, 256), err.value
            n = array.size
            res = np.empty(n, np.float32 if dst == "f32" else np.uint16)
            ctypes.memmove(res.ctypes.data, self.lib.tensor_buffer_data_mut(out), res.nbytes)
            return res.reshape(array.shape)
        finally:
            self.lib.tensor_buffer_free(h)
            if out.value:
                self.lib.tensor_buffer_free(out.value)


def load_oracle() -> Oracle:
    return Oracle()


def load_reference() -> Optional[Reference]:
    return Reference() if os.path.exists(REF_PATH) else None
