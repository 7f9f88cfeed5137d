"""RoPE and strided-view kernels on the GPU against the CPU oracle.

RoPE: f16 within 1 ulp of the oracle (cosf/sinf of the same float angle may
differ in the last f32 bit); f32 within 2e-6 of the pair magnitude.
Strided views: bit-exact (one f32 add and one multiply per element)."""
import numpy as np
import pytest

from inference_c_amd import TensorView
from tests.helpers import assert_bits_equal, assert_f16_ulps, rope_close

pytestmark = pytest.mark.gpu
F16 = np.float16


@pytest.mark.parametrize("device", [True, False])
@pytest.mark.parametrize("seq,qh,kh,dim,offset", [
    (4096, 32, 32, 64, 0), (17, 8, 2, 128, 5), (3, 1, 1, 2, 0), (9, 3, 5, 6, 1000),
    (5, 2, 2, 256, 123456),
    # fused path: waves straddling the q/k rows, a ragged last block, and
    # positions of more than 1024 (row, chunk) items split over blocks
    (33, 5, 3, 64, 7), (3, 200, 100, 64, 0), (70, 1, 1, 16, 2)])
def test_rope_f16(sdk, orc, seq, qh, kh, dim, offset, device):
    q = orc.normal((seq, qh, dim), 50, 0, 0.0, 1.0)
    k = orc.normal((seq, kh, dim), 50, 1, 0.0, 1.0)
    tq, tk = sdk.from_numpy(q, device=device), sdk.from_numpy(k, device=device)
    sdk.call("tensor_rope_f16", tq, tk, qh, kh, dim, 10000.0, offset)
    wq, wk = orc.rope(q, k, qh, kh, dim, 10000.0, offset)
    rope_close(tq.download(), wq, q)
    rope_close(tk.download(), wk, k)


# Shapes of the 1 KB-group path (half a row a whole number of 16-byte vectors,
# a power of two of them, and heads x vectors a multiple of 32 in both
# tensors): 1, 2, 4 and 8 groups per wave, positions of 1, 2, 4 and 8
# groups, more q blocks than k blocks and the reverse, and ragged tensors
# whose last waves hold groups past the end.
GROUP_SHAPES = [
    ("f16", 3, 16, 8, 64, 0),          # 1 group per wave, dead waves and groups
    ("f16", 70, 32, 64, 16, 2),        # one vector per half row
    ("f16", 300, 16, 32, 32, 9),       # two vectors per half row
    ("f16", 700, 2, 4, 256, 0),        # 16 vectors per half row
    ("f16", 4001, 8, 16, 64, 11),      # 2 groups per wave, k has twice q's blocks
    ("f16", 1501, 32, 16, 128, 77),    # 4 groups per wave, 2 positions per wave
    ("f16", 20001, 8, 8, 64, 1 << 20),  # 8 groups per wave over 8 positions
    ("f32", 64, 8, 4, 64, 3),
    ("f32", 33, 1, 1, 256, 0),         # 32 vectors per half row
    ("f32", 4096, 32, 8, 64, 0),       # 8 groups per wave, q has 4x k's blocks
]


@pytest.mark.parametrize("dtype,seq,qh,kh,dim,offset", GROUP_SHAPES)
def test_rope_group_path(sdk, orc, dtype, seq, qh, kh, dim, offset):
    q = orc.normal((seq, qh, dim), 52, 0, 0.0, 1.0, dtype)
    k = orc.normal((seq, kh, dim), 52, 1, 0.0, 1.0, dtype)
    tq, tk = sdk.from_numpy(q), sdk.from_numpy(k)
    sdk.call(f"tensor_rope_{dtype}", tq, tk, qh, kh, dim, 10000.0, offset)
    wq, wk = orc.rope(q, k, qh, kh, dim, 10000.0, offset)
    if dtype == "f16":
        rope_close(tq.download(), wq, q)
        rope_close(tk.download(), wk, k)
        return
    half = dim // 2
    for got, want, src in ((tq.download(), wq, q), (tk.download(), wk, k)):
        mag = np.sqrt(src[..., :half] ** 2 + src[..., half:] ** 2)
        mag = np.concatenate([mag, mag], axis=-1)
        assert np.all(np.abs(got - want) <= 2e-6 * mag + 1e-30)


@pytest.mark.parametrize("seq,qh,kh,dim,offset", [(64, 4, 2, 64, 0), (7, 3, 3, 10, 77),
                                                   (2, 150, 150, 64, 3), (45, 3, 1, 8, 9)])
def test_rope_f32(sdk, orc, seq, qh, kh, dim, offset):
    q = orc.normal((seq, qh, dim), 51, 0, 0.0, 1.0, "f32")
    k = orc.normal((seq, kh, dim), 51, 1, 0.0, 1.0, "f32")
    tq, tk = sdk.from_numpy(q), sdk.from_numpy(k)
    sdk.call("tensor_rope_f32", tq, tk, qh, kh, dim, 500000.0, offset)
    wq, wk = orc.rope(q, k, qh, kh, dim, 500000.0, offset)
    half = dim // 2
    for got, want, src in ((tq.download(), wq, q), (tk.download(), wk, k)):
        mag = np.sqrt(src[..., :half] ** 2 + src[..., half:] ** 2)
        mag = np.concatenate([mag, mag], axis=-1)
        assert np.all(np.abs(got - want) <= 2e-6 * mag + 1e-30)


def test_rope_known_answer(sdk):
    # reference tests/test_tensor_compute.c:160-168
    tq = sdk.from_numpy(np.array([1, 0, 1, 0], np.float32))
    tk = sdk.from_numpy(np.array([1, 0, 1, 0], np.float32))
    sdk.call("tensor_rope_f32", tq, tk, 1, 1, 2, 10000.0, 0)
    for t in (tq, tk):
        assert np.allclose(t.download(), [1, 0, np.cos(1.0), np.sin(1.0)], atol=2e-4)


def test_rope_rejects_bad_shapes(sdk):
    q = sdk.tensor("f16", (10, 4, 64))
    k = sdk.tensor("f16", (10, 3, 64))
    ok, msg = sdk.try_call("tensor_rope_f16", q, k, 4, 2, 64, 10000.0, 0)
    assert not ok and "RoPE requires" in msg
    ok, _ = sdk.try_call("tensor_rope_f16", q, q, 4, 4, 63, 10000.0, 0)
    assert not ok


def view_case(sdk, orc, x, shape, strides, offset, addend, mult, dtype="f16", device=True):
    tx = sdk.from_numpy(x, device=device)
    ta = None if addend is None else sdk.from_numpy(addend, device=device)
    tm = None if mult is None else sdk.from_numpy(mult, device=device)
    ty = sdk.tensor(dtype, shape, device)
    view = TensorView.make(shape, strides, offset)
    sdk.call(f"tensor_view_add_mul_{dtype}", tx, view, ta, tm, ty)
    want = orc.view_add_mul(x, shape, strides, offset, addend, mult)
    assert_bits_equal(ty.download(), want, f"view {shape} {strides}")


@pytest.mark.parametrize("device", [True, False])
def test_config4_permuted_broadcast(sdk, orc, device):
    """x [16,1024,32,64] read as (0,2,1,3), + A[1,32,1,64],
    * M[16,1,1024,1], written contiguous [16,32,1024,64]."""
    B, S, H, D = 16, 1024, 32, 64
    x = orc.normal((B, S, H, D), 1, 0, 0.0, 1.0)
    A = orc.uniform((1, H, 1, D), 1, 1, -1.0, 1.0, "f16")
    M = orc.uniform((B, 1, S, 1), 1, 2, -1.0, 1.0, "f16")
    view_case(sdk, orc, x, (B, H, S, D), (S * H * D, D, H * D, 1), 0, A, M, device=device)


@pytest.mark.parametrize("case", ["vector_tile", "vector_tile_ragged", "vector_rows", "tile",
                                  "tile_vec", "tile_vec_offset", "scalar", "broadcast_x", "offset", "rank1", "coalesce_contig",
                                  "rank6", "unit_dims", "one_vector_runs", "addend_inner_bcast",
                                  "short_rank4", "short_rank3_offset", "short_rank2",
                                  "copy_whole", "copy_ragged", "copy_unaligned"])
@pytest.mark.parametrize("dtype", ["f16", "f32"])
def test_view_paths(sdk, orc, case, dtype):
    dt = "f16" if dtype == "f16" else "f32"
    if case == "vector_tile":  # (0,2,1,3) permutation, 16-element runs
        x = orc.normal((3, 40, 5, 16), 52, 0, 0.0, 1.0, dt)
        shape, strides, off = (3, 5, 40, 16), (3200, 16, 80, 1), 0
        A = orc.uniform((1, 5, 1, 16), 52, 1, -1, 1, dt)
        M = orc.uniform((3, 1, 40, 1), 52, 2, -1, 1, dt)
    elif case == "vector_tile_ragged":  # rank-5 permutation with odd extents
        x = orc.normal((2, 3, 13, 11, 32), 58, 0, 0.0, 1.0, dt)
        shape = (2, 3, 11, 13, 32)
        strides = (3 * 13 * 11 * 32, 13 * 11 * 32, 32, 11 * 32, 1)
        off = 0
        A = orc.uniform((1, 3, 11, 1, 32), 58, 1, -1, 1, dt)
        M = orc.uniform((2, 1, 1, 13, 1), 58, 2, -1, 1, dt)
    elif case == "vector_rows":  # strided rows, last dim contiguous, no tile partner
        x = orc.normal((4, 6, 16), 59, 0, 0.0, 1.0, dt)
        shape, strides, off = (4, 3, 16), (96, 32, 1), 0
        A = orc.uniform((4, 3, 16), 59, 1, -1, 1, dt)
        M = orc.uniform((1, 3, 1), 59, 2, -1, 1, dt)
    elif case == "tile":       # transpose of the last two dims
        x = orc.normal((2, 3, 70, 130), 53, 0, 0.0, 1.0, dt)
        shape, strides, off = (2, 3, 130, 70), (3 * 70 * 130, 70 * 130, 1, 130), 0
        A = orc.uniform((1, 3, 130, 1), 53, 1, -1, 1, dt)
        M = orc.uniform((2, 1, 1, 70), 53, 2, -1, 1, dt)
    elif case == "tile_vec":   # transpose in whole 16-byte vectors (f16 without
        # operands: the vector tile kernel), partial 64 x 64 tiles, two batch dims
        x = orc.normal((2, 3, 72, 136), 71, 0, 0.0, 1.0, dt)
        shape, strides, off = (2, 3, 136, 72), (3 * 72 * 136, 72 * 136, 1, 136), 0
        A = orc.uniform((1, 3, 136, 1), 71, 1, -1, 1, dt)
        M = orc.uniform((2, 1, 1, 72), 71, 2, -1, 1, dt)
    elif case == "tile_vec_offset":  # a 16-column slice at an offset, transposed
        x = orc.normal((1000, 24), 72, 0, 0.0, 1.0, dt)
        shape, strides, off = (16, 1000), (1, 24), 8
        A, M = orc.uniform((16, 1), 72, 1, -1, 1, dt), None
    elif case == "scalar":     # odd strides
        x = orc.normal((1000,), 54, 0, 0.0, 1.0, dt)
        shape, strides, off = (7, 9), (101, 3), 5
        A = orc.uniform((7, 1), 54, 1, -1, 1, dt)
        M = None
    elif case == "broadcast_x":  # stride 0 repeats x along a dim
        x = orc.normal((64,), 55, 0, 0.0, 1.0, dt)
        shape, strides, off = (5, 64), (0, 1), 0
        A, M = None, orc.uniform((5, 64), 55, 2, -1, 1, dt)
    elif case == "offset":     # sliced, vector-aligned
        x = orc.normal((10, 48), 56, 0, 0.0, 1.0, dt)
        shape, strides, off = (4, 32), (96, 1), 8 if dt == "f16" else 4
        A, M = orc.uniform((1, 32), 56, 1, -1, 1, dt), orc.uniform((4, 32), 56, 2, -1, 1, dt)
    elif case == "coalesce_contig":  # contiguous view: x and A merge to one dim, M splits it
        x = orc.normal((3, 4, 5, 32), 60, 0, 0.0, 1.0, dt)
        shape, strides, off = (3, 4, 5, 32), (640, 160, 32, 1), 0
        A = orc.uniform((3, 4, 5, 32), 60, 1, -1, 1, dt)
        M = orc.uniform((3, 4, 1, 1), 60, 2, -1, 1, dt)
    elif case == "rank6":  # six dims that cannot merge: the any-rank gather kernel
        x = orc.normal((2, 3, 2, 3, 2, 16), 61, 0, 0.0, 1.0, dt)
        phys = (2, 3, 2, 3, 2, 16)
        cstr = [1] * 6
        for d in range(4, -1, -1):
            cstr[d] = cstr[d + 1] * phys[d + 1]
        perm = (4, 2, 0, 3, 1, 5)
        shape = tuple(phys[p] for p in perm)
        strides = tuple(cstr[p] for p in perm)
        off = 0
        A = orc.uniform((1,) + shape[1:], 61, 1, -1, 1, dt)
        M = orc.uniform(shape[:5] + (1,), 61, 2, -1, 1, dt)
    elif case == "unit_dims":  # extents of 1 between permuted dims
        x = orc.normal((4, 1, 6, 1, 24), 62, 0, 0.0, 1.0, dt)
        shape, strides, off = (6, 1, 4, 1, 24), (24, 999, 144, 5, 1), 0
        A = orc.uniform((6, 1, 1, 1, 24), 62, 1, -1, 1, dt)
        M = orc.uniform((1, 1, 4, 1, 1), 62, 2, -1, 1, dt)
    elif case == "one_vector_runs":  # innermost run of exactly one 16-byte vector
        e = 8 if dt == "f16" else 4
        x = orc.normal((5, 7, 3, e), 63, 0, 0.0, 1.0, dt)
        shape, strides, off = (5, 3, 7, e), (7 * 3 * e, e, 3 * e, 1), 0
        A = orc.uniform((1, 3, 1, e), 63, 1, -1, 1, dt)
        M = orc.uniform((5, 1, 7, 1), 63, 2, -1, 1, dt)
    elif case == "addend_inner_bcast":  # addend a scalar per vector, multiplier a vector
        x = orc.normal((6, 4, 32), 64, 0, 0.0, 1.0, dt)
        shape, strides, off = (4, 6, 32), (32, 128, 1), 0
        A = orc.uniform((4, 6, 1), 64, 1, -1, 1, dt)
        M = orc.uniform((1, 6, 32), 64, 2, -1, 1, dt)
    # the short gather kernel: <= 2 outer dims, whole 256-vector blocks per
    # plane, a power-of-two number of vectors per row
    elif case == "short_rank4":  # (0,2,1,3) permutation, vector addend, scalar multiplier
        x = orc.normal((2, 64, 3, 64), 65, 0, 0.0, 1.0, dt)
        shape, strides, off = (2, 3, 64, 64), (64 * 3 * 64, 64, 3 * 64, 1), 0
        A = orc.uniform((1, 3, 1, 64), 65, 1, -1, 1, dt)
        M = orc.uniform((2, 1, 64, 1), 65, 2, -1, 1, dt)
    elif case == "short_rank3_offset":  # sliced rows at an offset, scalar addend, vector multiplier
        x = orc.normal((4, 130, 32), 66, 0, 0.0, 1.0, dt)
        shape, strides, off = (3, 128, 32), (130 * 32, 32, 1), 2 * 32
        A = orc.uniform((1, 128, 1), 66, 1, -1, 1, dt)
        M = orc.uniform((3, 1, 32), 66, 2, -1, 1, dt)
    elif case == "short_rank2":  # strided rows, no outer dims
        x = orc.normal((300, 128), 67, 0, 0.0, 1.0, dt)
        shape, strides, off = (256, 64), (128, 1), 64
        A, M = orc.uniform((256, 1), 67, 1, -1, 1, dt), None
    # a contiguous view without operands is a copy (its own kernel): whole
    # 256-vector blocks at an aligned offset, a ragged last block, and an
    # offset off the 16-byte grid (the gather path takes that one)
    elif case == "copy_whole":  # 2048 vectors: 8 whole blocks
        e = 8 if dt == "f16" else 4
        x = orc.normal((4 * 512 * 8 + 64,), 68, 0, 0.0, 1.0, dt)
        shape, strides, off = (4, 512 * e), (512 * e, 1), 64
        A = orc.uniform((4, 1), 68, 1, -1, 1, dt)
        M = None
    elif case == "copy_ragged":  # 521 (f16) or 1042 (f32) vectors
        x = orc.normal((4200,), 69, 0, 0.0, 1.0, dt)
        shape, strides, off = (4168,), (1,), 16
        A, M = None, orc.uniform((1,), 69, 2, -1, 1, dt)
    elif case == "copy_unaligned":
        x = orc.normal((4000,), 70, 0, 0.0, 1.0, dt)
        shape, strides, off = (3000,), (1,), 3
        A, M = orc.uniform((3000,), 70, 1, -1, 1, dt), None
    else:
        x = orc.normal((100,), 57, 0, 0.0, 1.0, dt)
        shape, strides, off = (33,), (3,), 1
        A, M = orc.uniform((33,), 57, 1, -1, 1, dt), orc.uniform((1,), 57, 2, -1, 1, dt)
    view_case(sdk, orc, x, shape, strides, off, A, M, dt)
    view_case(sdk, orc, x, shape, strides, off, None, None, dt)


def test_view_rejects_out_of_bounds(sdk):
    x = sdk.tensor("f16", (100,))
    y = sdk.tensor("f16", (10, 10))
    ok, msg = sdk.try_call("tensor_view_add_mul_f16", x, TensorView.make((10, 10), (10, 1), 1), None, None, y)
    assert not ok and "lies inside the input" in msg
    ok, msg = sdk.try_call("tensor_view_add_mul_f16", x, TensorView.make((10, 10), (-10, 1), 99), None, None, y)
    assert not ok
    bad = sdk.tensor("f16", (3, 10))
    ok, msg = sdk.try_call("tensor_view_add_mul_f16", x, TensorView.make((10, 10), (10, 1), 0), bad, None, y)
    assert not ok and "1 or equal" in msg


# Views drawn once at random (numpy default_rng(13)): permutations of a
# contiguous base, slices, a stride-0 dim, operands broadcast over random
# dims; bit-exact against the oracle.
RANDOM_VIEWS = [  # dtype, base shape, view shape, strides, offset, addend shape, multiplier shape
    ("f32", (3, 2, 1, 100, 257), (1, 2, 100, 3, 257), (25700, 25700, 257, 51400, 1), 0, (1, 2, 1, 3, 1), None),
    ("f32", (128, 32, 16, 7, 3), (7, 128, 3, 32, 16), (3, 10752, 1, 336, 21), 0, None, (1, 128, 3, 1, 1)),
    ("f32", (32, 3, 32, 1, 1), (1, 1, 3, 32, 32), (1, 1, 32, 1, 96), 0, (1, 1, 1, 1, 1), (1, 1, 1, 32, 32)),
    ("f16", (100,), (44,), (1,), 56, (1,), None),
    ("f16", (257, 3, 257, 3), (257, 2, 3, 257), (2313, 1, 771, 3), 1, (257, 2, 3, 257), (1, 2, 1, 257)),
    ("f32", (7, 7), (7, 7), (1, 7), 0, (7, 1), (1, 7)),
    ("f16", (64, 16, 128), (16, 128, 64), (128, 1, 2048), 0, (16, 1, 64), None),
    ("f16", (100, 32, 7), (7, 100, 32), (1, 224, 7), 0, (1, 1, 1), (7, 100, 32)),
    ("f16", (16, 64, 3), (3, 64, 16), (1, 3, 192), 0, None, None),
]


@pytest.mark.parametrize("case", RANDOM_VIEWS)
def test_random_views(sdk, orc, case):
    dt, base, shape, strides, off, ashape, mshape = case
    x = orc.normal(base, 70, 0, 0.0, 1.0, dt)
    A = None if ashape is None else orc.uniform(ashape, 70, 1, -1.0, 1.0, dt)
    M = None if mshape is None else orc.uniform(mshape, 70, 2, -1.0, 1.0, dt)
    view_case(sdk, orc, x, shape, strides, off, A, M, dtype=dt)
