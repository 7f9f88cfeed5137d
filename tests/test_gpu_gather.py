"""Embedding lookup (row gather) on the GPU against the CPU oracle.

Rows are copied bytes, so every case is bit-exact: the public entry points
(tensor_embedding_lookup_*, reference src/common/tensor_ops.c:86-161) for
every index dtype, host and device storage, vector and scalar row widths;
rejected calls leave the output untouched; and the compute-table slots
(reference src/platform/cuda/tensor_compute_cuda.cu:53-67, 484-495), whose
out-of-range ids give zero rows and whose table stays cached per host address
until release_cache."""
import ctypes

import numpy as np
import pytest

from tests.helpers import assert_bits_equal

pytestmark = pytest.mark.gpu

INDEX_TYPES = [np.int16, np.uint16, np.int32, np.uint32, np.int64, np.uint64]


def ids_for(orc, count, rows, seed):
    return orc.uniform((count,), seed, 7, 0.0, rows - 0.001, "f32").astype(np.int64)


@pytest.mark.parametrize("device", [True, False])
@pytest.mark.parametrize("index_type", INDEX_TYPES)
@pytest.mark.parametrize("dtype", ["f16", "f32"])
def test_lookup_index_types(sdk, orc, dtype, index_type, device):
    rows, width, count = 300, 64, 257
    table = orc.normal((rows, width), 40, 0, 0.0, 1.0, dtype)
    ids = ids_for(orc, count, rows, 40).astype(index_type)
    ids[0], ids[-1] = rows - 1, 0
    t, i = sdk.from_numpy(table, device=device), sdk.from_numpy(ids, device=device)
    out = sdk.tensor(dtype, (count, width), device=device)
    sdk.call(f"tensor_embedding_lookup_{dtype}", t, i, out)
    assert_bits_equal(out.download(), orc.embedding_lookup(table, ids), "embedding")


@pytest.mark.parametrize("dtype,width", [("f32", 3), ("f32", 1), ("f16", 5), ("f16", 8),
                                         ("f32", 4), ("f16", 2048), ("f32", 1000)])
def test_lookup_row_widths(sdk, orc, dtype, width):
    """Scalar path (rows not whole 16-byte vectors) and vector path."""
    rows, count = 97, 129
    table = orc.normal((rows, width), 41, 0, 0.0, 1.0, dtype)
    ids = ids_for(orc, count, rows, 41).astype(np.uint32)
    t, i = sdk.from_numpy(table), sdk.from_numpy(ids)
    out = sdk.tensor(dtype, (count, width))
    sdk.call(f"tensor_embedding_lookup_{dtype}", t, i, out)
    assert_bits_equal(out.download(), orc.embedding_lookup(table, ids), f"width {width}")


def test_lookup_decoder_shape(sdk, orc):
    """A prefill batch: 4096 token ids into a 32000 x 2048 f16 table."""
    rows, width, count = 32000, 2048, 4096
    table = sdk.tensor("f16", (rows, width))
    sdk.call("tensor_fill_normal", table, 42, 0, 0.0, 1.0)
    ids = ids_for(orc, count, rows, 42).astype(np.int32)
    out = sdk.tensor("f16", (count, width))
    sdk.call("tensor_embedding_lookup_f16", table, sdk.from_numpy(ids), out)
    got = out.download()
    host_table = table.download()
    assert_bits_equal(got, orc.embedding_lookup(host_table, ids), "decoder-shape embedding")


@pytest.mark.parametrize("device", [True, False])
@pytest.mark.parametrize("bad", ["negative", "past_end"])
def test_rejected_lookup_leaves_output(sdk, orc, device, bad):
    rows, width = 50, 16
    table = orc.normal((rows, width), 43, 0, 0.0, 1.0, "f32")
    ids = ids_for(orc, 40, rows, 43).astype(np.int64)
    ids[17] = -3 if bad == "negative" else rows
    before = orc.normal((40, width), 43, 2, 0.0, 1.0, "f32")
    out = sdk.from_numpy(before, device=device)
    ok, msg = sdk.try_call("tensor_embedding_lookup_f32", sdk.from_numpy(table, device=device),
                           sdk.from_numpy(ids, device=device), out)
    assert not ok and msg == "embedding index is negative or outside the table"
    assert_bits_equal(out.download(), before, "output after a rejected call")


@pytest.mark.parametrize("index_type", INDEX_TYPES)
@pytest.mark.parametrize("count,position", [(1, 0), (45, 0), (45, 44), (45, 21),
                                            (70001, 70000), (70001, 65537)])
def test_device_index_check_positions(sdk, orc, index_type, count, position):
    """The device check scans 16-byte vectors of ids, several per lane per
    step, then a scalar tail: a bad id anywhere is found, a good batch
    passes. The gather is enqueued behind the check and skips every row on
    a rejected call: the previous output stays."""
    rows, width = 1000, 8
    table = sdk.from_numpy(orc.normal((rows, width), 45, 0, 0.0, 1.0, "f16"))
    ids = ids_for(orc, count, rows, 45).astype(index_type)
    out = sdk.tensor("f16", (count, width))
    assert sdk.try_call("tensor_embedding_lookup_f16", table, sdk.from_numpy(ids), out)[0] == 1
    good = out.download()
    ids[position] = rows if not np.issubdtype(index_type, np.signedinteger) or position % 2 else -1
    ok, msg = sdk.try_call("tensor_embedding_lookup_f16", table, sdk.from_numpy(ids), out)
    assert not ok and msg == "embedding index is negative or outside the table"
    assert_bits_equal(out.download(), good, "output after a rejected call")


def test_lookup_mixed_storage_rejected(sdk, orc):
    table = sdk.from_numpy(np.zeros((4, 8), np.float16))
    ids = sdk.from_numpy(np.array([1, 2], np.uint32), device=False)
    out = sdk.tensor("f16", (2, 8))
    ok, msg = sdk.try_call("tensor_embedding_lookup_f16", table, ids, out)
    assert not ok and "same storage type" in msg


def backend(sdk):
    from tests.test_gpu_vtable import Table
    return ctypes.cast(sdk.lib.tensor_compute_hip_backend(), ctypes.POINTER(Table)).contents


def slot(sdk, name):
    addr = getattr(backend(sdk), name)
    assert addr, f"slot {name} is NULL"
    args = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_size_t,
            ctypes.c_size_t]
    return ctypes.CFUNCTYPE(ctypes.c_int, *args)(addr)


def release_cache(sdk):
    ctypes.CFUNCTYPE(None)(backend(sdk).release_cache)()


def test_compute_slot_known_answer(sdk):
    # reference tests/test_tensor_compute.c:112-119
    table = np.arange(8, dtype=np.float32)
    ids = np.array([2, 0], np.uint32)
    out = np.zeros(4, np.float32)
    assert slot(sdk, "embedding_f32")(table.ctypes.data, ids.ctypes.data, out.ctypes.data, 2, 2, 4)
    assert out.tolist() == [4, 5, 0, 1]
    release_cache(sdk)


@pytest.mark.parametrize("dtype", ["f16", "f32"])
def test_compute_slot_zero_rows_and_cache(sdk, orc, dtype):
    rows, width, count = 40, 24, 33
    table = orc.normal((rows, width), 44, 0, 0.0, 1.0, dtype)
    ids = ids_for(orc, count, rows, 44).astype(np.uint32)
    ids[3], ids[9] = rows, 0xffffffff
    out = np.zeros((count, width), table.dtype)
    fn = slot(sdk, f"embedding_{dtype}")
    assert fn(table.ctypes.data, ids.ctypes.data, out.ctypes.data, count, width, rows)
    assert_bits_equal(out, orc.embedding_gather_u32(table, ids), "slot")
    # the table stays cached per host address: a changed host table is not
    # seen until release_cache (the CUDA backend's behaviour)
    cached = table.copy()
    table[:] = table * 2
    out2 = np.zeros_like(out)
    assert fn(table.ctypes.data, ids.ctypes.data, out2.ctypes.data, count, width, rows)
    assert_bits_equal(out2, orc.embedding_gather_u32(cached, ids), "slot (cached table)")
    # same address with another size is refused
    assert fn(table.ctypes.data, ids.ctypes.data, out2.ctypes.data, count, width, rows - 1) == 0
    release_cache(sdk)
    assert fn(table.ctypes.data, ids.ctypes.data, out2.ctypes.data, count, width, rows)
    assert_bits_equal(out2, orc.embedding_gather_u32(table, ids), "slot after release_cache")
    release_cache(sdk)
    assert fn(table.ctypes.data, ids.ctypes.data, out2.ctypes.data, 0, width, rows) == 0
