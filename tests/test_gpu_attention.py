"""Scaled dot-product attention on the GPU against the CPU oracle.

The oracle restates the reference's accelerator semantics
(src/platform/cuda/attention_cuda.cu:25-99, pinned to the reference build's
tensor_sdpa_f32 in test_oracle_vs_reference.py). The GPU computes the same
scores but folds them with an online softmax and normalises once at the end,
so outputs are compared against sum_j p_j |v_j| (the scale of any reordered
accumulation of p_j v_j):
  f32: |got - want| <= 1e-5 * sum_j p_j |v_j|   (north-star f32 reduction bound)
  f16: within 1 f16 ulp of the oracle, or |got - want| <= 2e-3 * sum_j p_j |v_j|
       (north-star f16 reduction bound).
Special rows (all masked, +inf or NaN scores) must match exactly."""
import ctypes

import numpy as np
import pytest

from tests.helpers import f16_ulps

pytestmark = pytest.mark.gpu

SHAPES = [  # batch, q heads, kv heads, q len, kv len, head dim, value dim
    (1, 4, 2, 5, 9, 16, 8),
    (2, 2, 1, 33, 33, 64, 64),
    (1, 3, 3, 7, 4, 5, 3),          # dims that are not whole vectors
    (1, 2, 2, 1, 50, 32, 32),       # a decode step
    (1, 8, 2, 128, 200, 128, 128),
    (2, 12, 12, 64, 64, 64, 64),
    (1, 2, 1, 70, 130, 96, 80),
    (1, 1, 1, 3, 700, 256, 512),
    (1, 4, 1, 300, 300, 128, 128),  # MFMA path: ragged query and key tiles, 4 heads per kv head
    (1, 2, 2, 129, 1000, 64, 64),   # MFMA path: kv longer than q (causal offset 871)
    (3, 2, 2, 1, 77, 128, 128),     # MFMA path: one query
    (1, 2, 1, 40, 2048, 128, 128),  # MFMA path, key range split over 8 blocks
    (2, 3, 3, 100, 1500, 64, 64),   # MFMA path, key range split in 6 (f16) / 8 (f32, uneven) parts
    (1, 2, 2, 600, 600, 64, 64),    # MFMA path, causal: long query blocks split, short ones whole
    (1, 64, 8, 130, 150, 64, 64),   # 128-query blocks (>= 64 of them): ragged query and key tiles
    (1, 32, 4, 256, 300, 128, 128), # 128-query blocks at D 128, 8 q-heads per kv head
    (1, 64, 16, 128, 1024, 64, 64), # causal: 128-query blocks, split key ranges; else 64-query two-part blocks
    (2, 64, 8, 257, 100, 64, 64),   # f16 256-query blocks (>= 256 of them), ragged; f32 128
    (1, 128, 32, 300, 90, 128, 128),  # f16 256-query blocks at D 128
]


def inputs(orc, shape, dtype, seed, masked):
    b, h, kh, lq, lk, d, dv = shape
    q = orc.normal((b, h, lq, d), seed, 0, 0.0, 1.0, dtype)
    k = orc.normal((b, kh, lk, d), seed, 1, 0.0, 1.0, dtype)
    v = orc.normal((b, kh, lk, dv), seed, 2, 0.0, 1.0, dtype)
    mask = None
    if masked:
        mask = orc.uniform((lq, lk), seed, 3, -4.0, 0.0, dtype)
        mask[:, lk // 2] = -np.inf
    return q, k, v, mask


def check(got, want, weight, dtype, what):
    g = got.astype(np.float64)
    w = want.astype(np.float64)
    assert np.array_equal(np.isnan(g), np.isnan(w)), f"{what}: NaN positions differ"
    g, w, wt = g[~np.isnan(w)], w[~np.isnan(w)], weight[~np.isnan(w)]
    err = np.abs(g - w)
    if dtype == "f32":
        ok = err <= 1e-5 * wt + 1e-30
    else:
        ok = (f16_ulps(got[~np.isnan(want.astype(np.float64))],
                       want[~np.isnan(want.astype(np.float64))]) <= 1) | (err <= 2e-3 * wt)
    bad = np.flatnonzero(~ok)
    assert bad.size == 0, (f"{what}: {bad.size} of {ok.size} outside the bound; worst "
                           f"{float((err / np.maximum(wt, 1e-30)).max()):.3g} of sum p|v|")


def run_device(sdk, q, k, v, mask, scale, causal, dtype):
    tq, tk, tv = sdk.from_numpy(q), sdk.from_numpy(k), sdk.from_numpy(v)
    tm = None if mask is None else sdk.from_numpy(mask)
    out = sdk.tensor(dtype, q.shape[:3] + (v.shape[3],))
    sdk.call(f"tensor_sdpa_device_{dtype}", tq, tk, tv, tm, scale, int(causal), out)
    return out.download()


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("dtype", ["f16", "f32"])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("masked", [False, True])
def test_device_sdpa(sdk, orc, shape, dtype, causal, masked):
    q, k, v, mask = inputs(orc, shape, dtype, 30, masked)
    scale = 1.0 / np.sqrt(shape[5])
    got = run_device(sdk, q, k, v, mask, scale, causal, dtype)
    want = orc.sdpa(q, k, v, mask, scale, causal)
    weight = orc.sdpa_abs_weight(q, k, v, mask, scale, causal)
    check(got, want, weight, dtype, f"{shape} causal={causal} mask={masked}")


# MFMA-path shapes with several 64-key tiles per row
RAMP_SHAPES = [(1, 2, 1, 64, 2048, 128, 128), (1, 4, 4, 256, 256, 64, 64)]


@pytest.mark.parametrize("shape", RAMP_SHAPES)
@pytest.mark.parametrize("dtype", ["f16", "f32"])
@pytest.mark.parametrize("direction", [1.0, -1.0])
@pytest.mark.parametrize("causal", [False, True])
def test_growing_row_maxima(sdk, orc, shape, dtype, direction, causal):
    """Scores that climb (or fall) steadily along the keys, 60 log2 units
    over the row for f16: the running maximum of the f16 kernel moves on
    some tiles (growth past 2^8 since it last moved) and stays on others
    (probabilities up to 2^8 in the f16 P operand); falling scores keep the
    first tile's maximum throughout. f32 climbs 20 log2 units: one rounding
    of a score s moves exp(s) by |s| ulps, which at 40 nats exceeds the f32
    bound whatever the kernel."""
    b, h, kh, lq, lk, d, dv = shape
    q, k, v, _ = inputs(orc, shape, dtype, 31, False)
    scale = 1.0 / np.sqrt(d)
    climb = 60.0 if dtype == "f16" else 20.0   # log2 units from the first key to the last
    reach = climb / (4.0 * scale * np.log2(np.e))   # q[..., 0] * k[..., -1, 0] * scale
    q[..., 0] = 4.0
    k[..., :, 0] = (direction * reach * np.arange(lk) / lk).astype(k.dtype)
    got = run_device(sdk, q, k, v, None, scale, causal, dtype)
    want = orc.sdpa(q, k, v, None, scale, causal)
    weight = orc.sdpa_abs_weight(q, k, v, None, scale, causal)
    check(got, want, weight, dtype, f"{shape} direction={direction} causal={causal}")


@pytest.mark.parametrize("dtype,scale", [("f16", -0.2), ("f16", 0.0), ("f16", 3.0),
                                         ("f32", -0.2), ("f32", 0.0), ("f32", 0.2)])
@pytest.mark.parametrize("shape", [(1, 4, 1, 300, 300, 128, 128), (1, 2, 1, 40, 2048, 128, 128)])
@pytest.mark.parametrize("causal", [False, True])
def test_flash_scales(sdk, orc, scale, shape, dtype, causal):
    """Scales other than 1/sqrt(d) on the MFMA path, unsplit and split: a
    negative or zero scale takes the f16 kernel's general variant (raw
    products cannot carry the scale into the maximum), a large one makes
    the softmax nearly one-hot. f32 stops at 0.2: its scores' own rounding
    (|q.k| up to ~40 for d = 128, summed in another order than the
    oracle's, ~3e-5 apart) times the scale is the relative error of p, and
    past ~0.3 that alone exceeds the f32 bound."""
    q, k, v, _ = inputs(orc, shape, dtype, 32, False)
    got = run_device(sdk, q, k, v, None, scale, causal, dtype)
    want = orc.sdpa(q, k, v, None, scale, causal)
    weight = orc.sdpa_abs_weight(q, k, v, None, scale, causal)
    check(got, want, weight, dtype, f"{shape} scale={scale} causal={causal}")


def table_slots(sdk):
    sdk.lib.tensor_attention_cuda_backend.restype = ctypes.c_void_p
    return ctypes.cast(sdk.lib.tensor_attention_cuda_backend(), ctypes.POINTER(ctypes.c_void_p))


def run_slot(sdk, dtype, q, k, v, mask, scale, causal):
    slots = table_slots(sdk)
    P, Z = ctypes.c_void_p, ctypes.c_size_t
    fn = ctypes.CFUNCTYPE(ctypes.c_int, P, P, P, P, P, Z, Z, Z, Z, Z, Z, Z, ctypes.c_float,
                          ctypes.c_int)(slots[3] if dtype == "f32" else slots[4])
    b, h, lq, d = q.shape
    kh, lk, dv = k.shape[1], k.shape[2], v.shape[3]
    out = np.zeros((b, h, lq, dv), q.dtype)
    ok = fn(q.ctypes.data, k.ctypes.data, v.ctypes.data,
            None if mask is None else mask.ctypes.data, out.ctypes.data, b, h, kh, lq, lk, d, dv,
            scale, int(causal))
    return ok, out


def test_table_known_answers(sdk):
    """reference tests/test_attention.c:441-496 through the accelerator
    table's host-pointer run slot (what tensor_sdpa_f32 calls)."""
    slots = table_slots(sdk)
    assert ctypes.CFUNCTYPE(ctypes.c_int)(slots[2])() == 1
    q = np.array([1, 0, 0, 1, 1, 0, 0, 1], np.float32).reshape(1, 2, 2, 2)
    k = np.array([1, 0, 0, 1], np.float32).reshape(1, 1, 2, 2)
    v = np.array([1, 0, 0, 2], np.float32).reshape(1, 1, 2, 2)
    near = lambda a, b: np.allclose(a, b, atol=1e-5, rtol=0)
    ok, out = run_slot(sdk, "f32", q, k, v, None, 1.0, False)
    assert ok and near(out.ravel()[:4], [0.73105858, 0.53788284, 0.26894143, 1.4621172])
    assert near(out.ravel()[4:], out.ravel()[:4])
    ok, out = run_slot(sdk, "f32", q, k, v, None, 1.0, True)
    assert ok and near(out.ravel()[:4], [1.0, 0.0, 0.26894143, 1.4621172])
    mask = np.array([-np.inf, 0, 0, 0], np.float32).reshape(2, 2)
    ok, out = run_slot(sdk, "f32", q, k, v, mask, 1.0, False)
    assert ok and near(out.ravel()[:2], [0.0, 2.0])
    ok, out = run_slot(sdk, "f32", q, k, v, np.full((2, 2), -np.inf, np.float32), 1.0, False)
    assert ok and (out == 0).all()


@pytest.mark.parametrize("dtype", ["f16", "f32"])
def test_table_run_matches_oracle(sdk, orc, dtype):
    shape = (1, 4, 2, 37, 53, 64, 64)
    q, k, v, mask = inputs(orc, shape, dtype, 31, True)
    ok, got = run_slot(sdk, dtype, q, k, v, mask, 0.125, True)
    assert ok
    check(got, orc.sdpa(q, k, v, mask, 0.125, True), orc.sdpa_abs_weight(q, k, v, mask, 0.125, True),
          dtype, "table run")


def test_table_rejects_bad_arguments(sdk):
    q = np.ones((1, 3, 2, 4), np.float32)
    k = np.ones((1, 2, 2, 4), np.float32)   # 3 query heads over 2 kv heads
    ok, _ = run_slot(sdk, "f32", q, k, k, None, 1.0, False)
    assert ok == 0
    ok, _ = run_slot(sdk, "f32", q[:, :2], k, k, None, float("inf"), False)
    assert ok == 0


@pytest.mark.parametrize("dtype", ["f16", "f32"])
def test_special_rows(sdk, orc, dtype):
    """Rows whose scores are only -inf and NaN are zero; a row whose max is
    +inf is zero; a NaN score beside finite ones makes the row NaN. Bitwise
    equal to the oracle, NaN positions included."""
    npt = np.float16 if dtype == "f16" else np.float32
    big = 60000.0 if dtype == "f16" else 1e38
    q = np.zeros((1, 1, 4, 8), npt)
    q[0, 0, 1] = big           # +inf scores in f32 accumulation
    q[0, 0, 2] = 1.0
    q[0, 0, 3] = 0.5
    k = np.ones((1, 1, 3, 8), npt)
    k[0, 0, 1, 0] = np.nan
    v = np.arange(6, dtype=npt).reshape(1, 1, 3, 2)
    mask = np.zeros((4, 3), npt)
    mask[0, 0] = mask[0, 2] = -np.inf   # row 0: only the NaN key is left
    got = run_device(sdk, q, k, v, mask, 1.0, False, dtype)
    want = orc.sdpa(q, k, v, mask, 1.0, False)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(np.nan_to_num(got.astype(np.float64)), np.nan_to_num(want.astype(np.float64)))
    assert (got[0, 0, 0] == 0).all() and np.isnan(got[0, 0, 2]).all()
    if dtype == "f32":  # 8 * 1e38 overflows the f32 score: max +inf, zero row
        assert (got[0, 0, 1] == 0).all()


def test_device_sdpa_validation(sdk):
    q = sdk.tensor("f16", (1, 4, 8, 64))
    k = sdk.tensor("f16", (1, 3, 8, 64))
    out = sdk.tensor("f16", (1, 4, 8, 64))
    ok, msg = sdk.try_call("tensor_sdpa_device_f16", q, k, k, None, 1.0, 0, out)
    assert not ok and msg == "SDPA tensor dimensions do not match"
    k2 = sdk.tensor("f16", (1, 2, 8, 64))
    bad_mask = sdk.tensor("f16", (8, 9))
    ok, msg = sdk.try_call("tensor_sdpa_device_f16", q, k2, k2, bad_mask, 1.0, 0, out)
    assert not ok and msg == "SDPA mask shape must be [query_length, key_length]"
    ok, msg = sdk.try_call("tensor_sdpa_device_f16", q, k2, k2, None, 1.0, 2, out)
    assert not ok and "finite scale" in msg
    wide = sdk.tensor("f16", (1, 1, 2, 520))
    ok, msg = sdk.try_call("tensor_sdpa_device_f16", wide, wide, wide, None, 1.0, 0, wide)
    assert not ok and "up to 512" in msg


@pytest.mark.parametrize("dtype", ["f16", "f32"])
def test_split_key_range_special_rows(sdk, orc, dtype):
    """A small grid with a long key range is split over several blocks and
    merged; the special-row rules hold across splits, bitwise vs the oracle:
    row 0 sees one key, in the last split; row 1 has a NaN query (every score
    NaN: nothing visible, zero row); row 2 has a +inf mask entry in one split
    (row max +inf: zero row); row 3 is ordinary."""
    npt = np.float16 if dtype == "f16" else np.float32
    lq, lk, d = 4, 1024, 64
    q = orc.normal((1, 1, lq, d), 33, 0, 0.0, 1.0, dtype)
    k = orc.normal((1, 1, lk, d), 33, 1, 0.0, 1.0, dtype)
    v = orc.normal((1, 1, lk, d), 33, 2, 0.0, 1.0, dtype)
    q[0, 0, 1, 5] = np.nan
    mask = np.zeros((lq, lk), npt)
    mask[0, :] = -np.inf
    mask[0, 900] = 0
    mask[2, 500] = np.inf
    got = run_device(sdk, q, k, v, mask, 0.125, False, dtype)
    want = orc.sdpa(q, k, v, mask, 0.125, False)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert (got[0, 0, 1] == 0).all() and (got[0, 0, 2] == 0).all()
    np.testing.assert_array_equal(got[0, 0, 0], v[0, 0, 900].astype(got.dtype))
    weight = orc.sdpa_abs_weight(q, k, v, mask, 0.125, False)
    check(got[0, 0, 3:], want[0, 0, 3:], weight[0, 0, 3:], dtype, "ordinary row")


# Causal shapes with uneven key ranges that take blocks of 128 queries whose
# 8 waves are 4 query groups x 2 key parts (alternate key tiles: 64 keys
# f16, 32 f32), merged in LDS: f16 where its 256-query blocks would be about
# one round on the GPU, f32 from 256 such blocks. The oracle runs on the
# first and the last kv head's query heads only.
KEY_PART_SHAPES = [
    (1, 128, 16, 512, 512, 64, 64),     # 4 and 8 key tiles per 256 queries
    (2, 64, 16, 512, 512, 128, 128),    # batch 2, D 128
    (1, 128, 32, 500, 500, 64, 64),     # ragged query and key tiles
    (1, 64, 16, 700, 720, 64, 64),      # kv longer than q (causal offset 20), ragged
    (1, 64, 64, 512, 512, 128, 128),    # one q head per kv head
    (1, 16, 4, 2048, 2048, 64, 64),     # one round of 256 blocks: long blocks' key ranges split too
]


def head_subset(q, k, v, got):
    """(q, k, v, got) restricted to the query heads of kv heads 0 and -1."""
    group = q.shape[1] // k.shape[1]
    qs = np.r_[0:group, q.shape[1] - group:q.shape[1]]
    ks = np.r_[0:1, k.shape[1] - 1:k.shape[1]]
    return q[:, qs], k[:, ks], v[:, ks], got[:, qs]


@pytest.mark.parametrize("shape", KEY_PART_SHAPES)
@pytest.mark.parametrize("dtype", ["f16", "f32"])
def test_key_parts(sdk, orc, shape, dtype):
    q, k, v, _ = inputs(orc, shape, dtype, 34, False)
    scale = 1.0 / np.sqrt(shape[5])
    got = run_device(sdk, q, k, v, None, scale, True, dtype)
    q, k, v, got = head_subset(q, k, v, got)
    want = orc.sdpa(q, k, v, None, scale, True)
    weight = orc.sdpa_abs_weight(q, k, v, None, scale, True)
    check(got, want, weight, dtype, f"{shape} causal")


@pytest.mark.parametrize("direction", [1.0, -1.0])
@pytest.mark.parametrize("dtype", ["f16", "f32"])
def test_key_parts_growing_row_maxima(sdk, orc, direction, dtype):
    """Scores climbing (or falling) along the keys (60 log2 units for f16,
    20 for f32, as in test_growing_row_maxima): the two key parts' running
    maxima move at different tiles and are merged with their own weights."""
    shape = (1, 128, 16, 512, 512, 64, 64)
    q, k, v, _ = inputs(orc, shape, dtype, 35, False)
    scale = 1.0 / np.sqrt(shape[5])
    climb = 60.0 if dtype == "f16" else 20.0
    reach = climb / (4.0 * scale * np.log2(np.e))
    q[..., 0] = 4.0
    k[..., :, 0] = (direction * reach * np.arange(shape[4]) / shape[4]).astype(k.dtype)
    got = run_device(sdk, q, k, v, None, scale, True, dtype)
    q, k, v, got = head_subset(q, k, v, got)
    want = orc.sdpa(q, k, v, None, scale, True)
    weight = orc.sdpa_abs_weight(q, k, v, None, scale, True)
    check(got, want, weight, dtype, f"direction={direction}")


@pytest.mark.parametrize("dtype", ["f16", "f32"])
def test_key_parts_special_rows(sdk, orc, dtype):
    """Special rows across the two key parts, bitwise vs the oracle: a NaN
    query (every score NaN: zero row); a NaN key in the second part's first
    tile (rows that see it are NaN); a +inf key component in the second
    part's second tile (rows that see it with a positive query component:
    max +inf, zero row; negative: -inf score, the key drops out)."""
    shape = (1, 128, 16, 512, 512, 64, 64)
    q, k, v, _ = inputs(orc, shape, dtype, 36, False)
    q[0, 0, 1, 5] = np.nan
    k[0, 15, 70, 3] = np.nan
    k[0, 15, 200, 0] = np.inf
    got = run_device(sdk, q, k, v, None, 0.125, True, dtype)
    q, k, v, got = head_subset(q, k, v, got)
    want = orc.sdpa(q, k, v, None, 0.125, True)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    zero = (want == 0).all(axis=-1)
    assert zero[0, 0, 1] and zero[0, -1].any()
    assert (got[zero] == 0).all()
    weight = orc.sdpa_abs_weight(q, k, v, None, 0.125, True)
    live = ~zero & ~np.isnan(want).any(axis=-1)
    assert live[0, -1, :70].all()
    check(got[live], want[live], weight[live], dtype, "ordinary rows")


@pytest.mark.parametrize("dtype", ["f16", "f32"])
@pytest.mark.parametrize("scale", [0.125, -0.125])
def test_key_part_plan_general_variant(sdk, orc, dtype, scale):
    """A mask (or a scale <= 0) on a shape whose plan takes two key parts:
    the general variant runs with one key part on the same 128-query plan."""
    shape = (1, 128, 16, 512, 512, 64, 64)
    q, k, v, mask = inputs(orc, shape, dtype, 37, scale > 0)
    got = run_device(sdk, q, k, v, mask, scale, True, dtype)
    q, k, v, got = head_subset(q, k, v, got)
    want = orc.sdpa(q, k, v, mask, scale, True)
    weight = orc.sdpa_abs_weight(q, k, v, mask, scale, True)
    check(got, want, weight, dtype, f"scale={scale} mask={mask is not None}")


def test_small_grid_key_parts_special_rows(sdk, orc):
    """f16, 64 blocks of 128 queries over 1536 keys: two key parts per query
    group and the key range split over blocks (merged by the combine
    kernel). Special rows bitwise vs the oracle across both merges: a NaN
    query (zero row), a NaN key in the second half of the range (every row
    NaN), and a +inf key component in the first half (rows with a positive
    query component: max +inf, zero row)."""
    shape = (1, 64, 16, 128, 1536, 64, 64)
    q, k, v, _ = inputs(orc, shape, "f16", 38, False)
    q[0, 0, 1, 5] = np.nan
    k[0, 15, 1300, 3] = np.nan
    k[0, 0, 70, 0] = np.inf
    got = run_device(sdk, q, k, v, None, 0.125, False, "f16")
    q, k, v, got = head_subset(q, k, v, got)
    want = orc.sdpa(q, k, v, None, 0.125, False)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    zero = (want == 0).all(axis=-1)
    assert zero[0, 0, 1] and zero[0, 1].any() and np.isnan(want[0, -1]).all()
    assert (got[zero] == 0).all()
    weight = orc.sdpa_abs_weight(q, k, v, None, 0.125, False)
    live = ~zero & ~np.isnan(want).any(axis=-1)
    assert live.any()
    check(got[live], want[live], weight[live], "f16", "ordinary rows")


# f16, non-causal, 64-128 blocks of 128 queries over at most 1024 keys:
# 64-query blocks of 4 waves (2 query groups x 2 key parts, merged in LDS),
# no key-range split; with a mask the general variant runs one key part on
# the same 64-query plan.
SHORT_GRID_SHAPES = [
    (1, 64, 16, 128, 1024, 64, 64),     # 64 blocks of 128 queries
    (1, 12, 12, 1024, 1024, 64, 64),    # 96, one q head per kv head
    (1, 96, 24, 100, 1000, 128, 128),   # D 128, ragged queries and keys
    (2, 32, 8, 200, 512, 64, 64),       # batch 2, 128 blocks, a ragged 64-query block
    (1, 64, 64, 130, 77, 128, 128),     # two key tiles, the second ragged
]


@pytest.mark.parametrize("shape", SHORT_GRID_SHAPES)
@pytest.mark.parametrize("masked", [False, True])
def test_short_small_grid(sdk, orc, shape, masked):
    q, k, v, mask = inputs(orc, shape, "f16", 39, masked)
    scale = 1.0 / np.sqrt(shape[5])
    got = run_device(sdk, q, k, v, mask, scale, False, "f16")
    q, k, v, got = head_subset(q, k, v, got)
    want = orc.sdpa(q, k, v, mask, scale, False)
    weight = orc.sdpa_abs_weight(q, k, v, mask, scale, False)
    check(got, want, weight, "f16", f"{shape} mask={masked}")


def test_short_small_grid_special_rows(sdk, orc):
    """The 64-query two-part plan, special rows bitwise vs the oracle: a NaN
    query (zero row), a NaN key in the second key part's first tile (every
    row of that kv head NaN), a +inf key component in the first part's
    second tile (rows with a positive query component: max +inf, zero
    row)."""
    shape = (1, 64, 16, 128, 1024, 64, 64)
    q, k, v, _ = inputs(orc, shape, "f16", 40, False)
    q[0, 0, 1, 5] = np.nan
    k[0, 15, 70, 3] = np.nan
    k[0, 0, 130, 0] = np.inf
    got = run_device(sdk, q, k, v, None, 0.125, False, "f16")
    q, k, v, got = head_subset(q, k, v, got)
    want = orc.sdpa(q, k, v, None, 0.125, False)
    assert np.array_equal(np.isnan(got), np.isnan(want))
    zero = (want == 0).all(axis=-1)
    assert zero[0, 0, 1] and zero[0, 1].any() and np.isnan(want[0, -1]).all()
    assert (got[zero] == 0).all()
    weight = orc.sdpa_abs_weight(q, k, v, None, 0.125, False)
    live = ~zero & ~np.isnan(want).any(axis=-1)
    assert live.any()
    check(got[live], want[live], weight[live], "f16", "ordinary rows")


# f16, exactly 256 blocks of 128 queries (one per CU): two key parts per
# query group, causal too when the key ranges are even (kv much longer than q).
ROUND_SHAPES = [
    ((1, 32, 8, 1024, 1024, 64, 64), False),
    ((1, 32, 8, 1000, 1000, 128, 128), False),    # ragged query and key tiles
    ((1, 64, 16, 512, 2048, 64, 64), True),       # causal offset 1536
    ((2, 16, 16, 1024, 4096, 64, 64), True),      # causal offset 3072, batch 2
]


@pytest.mark.parametrize("shape,causal", ROUND_SHAPES)
def test_one_round_key_parts(sdk, orc, shape, causal):
    q, k, v, _ = inputs(orc, shape, "f16", 41, False)
    scale = 1.0 / np.sqrt(shape[5])
    got = run_device(sdk, q, k, v, None, scale, causal, "f16")
    q, k, v, got = head_subset(q, k, v, got)
    want = orc.sdpa(q, k, v, None, scale, causal)
    weight = orc.sdpa_abs_weight(q, k, v, None, scale, causal)
    check(got, want, weight, "f16", f"{shape} causal={causal}")


# f16, more than 256 blocks of 128 queries but fewer than 256 of 256: the
# 256-query plan below one round of blocks
@pytest.mark.parametrize("shape,causal", [((1, 48, 12, 1000, 1000, 64, 64), False),
                                          ((1, 64, 8, 520, 2100, 128, 128), True)])
def test_partial_round_256_query_blocks(sdk, orc, shape, causal):
    q, k, v, _ = inputs(orc, shape, "f16", 42, False)
    scale = 1.0 / np.sqrt(shape[5])
    got = run_device(sdk, q, k, v, None, scale, causal, "f16")
    q, k, v, got = head_subset(q, k, v, got)
    want = orc.sdpa(q, k, v, None, scale, causal)
    weight = orc.sdpa_abs_weight(q, k, v, None, scale, causal)
    check(got, want, weight, "f16", f"{shape} causal={causal}")


def sdpa_f64(q, k, v, scale, causal):
    """Float64 numpy restatement of the oracle's rule for finite inputs
    without a mask (oracle/oracle.c sdpa_generic): query i sees key j unless
    causal and j > i + max(kv_len - q_len, 0); softmax over the visible keys;
    returns (out, sum_j p |v|)."""
    b, h, lq, d = q.shape
    kvh, lk = k.shape[1], k.shape[2]
    group = h // kvh
    kk = np.repeat(k.astype(np.float64), group, axis=1)
    vv = np.repeat(v.astype(np.float64), group, axis=1)
    s = np.einsum("bhid,bhjd->bhij", q.astype(np.float64), kk) * scale
    if causal:
        offset = max(lk - lq, 0)
        s = np.where(np.arange(lk)[None, :] > np.arange(lq)[:, None] + offset, -np.inf, s)
    p = np.exp(s - s.max(axis=-1, keepdims=True))
    p /= p.sum(axis=-1, keepdims=True)
    return p @ vv, p @ np.abs(vv)


def test_sdpa_f64_restatement_matches_oracle(orc):
    """The float64 restatement used by the plan sweep against the oracle on
    small causal (kv longer and shorter than q) and full shapes."""
    for shape, causal in (((1, 4, 2, 37, 70, 64, 64), True), ((1, 2, 1, 70, 37, 64, 64), True),
                          ((2, 2, 2, 33, 50, 128, 128), False)):
        q, k, v, _ = inputs(orc, shape, "f32", 43, False)
        scale = 1.0 / np.sqrt(shape[5])
        want, weight = sdpa_f64(q, k, v, scale, causal)
        got = orc.sdpa(q, k, v, None, scale, causal)
        assert np.allclose(got, want, rtol=0, atol=1e-5 * weight.max())


# Random shapes over every block plan (fewer than 64, 64-256 and more than
# 256 blocks of 128 queries; ragged lengths, kv shorter and longer than q,
# 1-8 q heads per kv head), drawn once with numpy's default_rng(2026).
SWEEP_SHAPES = [
    ((1, 1, 1, 548, 1547, 128, 128), True), ((2, 32, 8, 1082, 977, 128, 128), True),
    ((2, 64, 16, 424, 1984, 64, 64), False), ((1, 64, 16, 690, 1244, 128, 128), True),
    ((1, 4, 4, 406, 2057, 128, 128), True), ((1, 2, 2, 716, 1929, 128, 128), True),
    ((1, 128, 16, 892, 892, 64, 64), True), ((1, 16, 4, 471, 527, 64, 64), True),
    ((1, 8, 4, 870, 832, 128, 128), False), ((1, 16, 4, 558, 2303, 128, 128), True),
    ((2, 4, 1, 866, 2479, 64, 64), False), ((2, 64, 16, 490, 1081, 64, 64), False),
    ((1, 32, 4, 89, 2116, 64, 64), True), ((1, 8, 2, 625, 1711, 128, 128), False),
    ((1, 64, 16, 241, 241, 128, 128), True), ((1, 16, 2, 154, 2040, 64, 64), True),
    ((2, 32, 16, 259, 259, 128, 128), False), ((1, 16, 4, 989, 2466, 64, 64), True),
    ((1, 8, 1, 102, 1794, 128, 128), False), ((1, 32, 16, 984, 1903, 128, 128), True),
    ((1, 8, 4, 50, 2780, 128, 128), True), ((2, 64, 16, 989, 989, 128, 128), True),
    ((1, 16, 2, 117, 404, 128, 128), False), ((1, 8, 4, 284, 2881, 64, 64), False),
]


@pytest.mark.parametrize("shape,causal", SWEEP_SHAPES)
@pytest.mark.parametrize("dtype", ["f16", "f32"])
def test_plan_sweep(sdk, orc, shape, causal, dtype):
    q, k, v, _ = inputs(orc, shape, dtype, 44, False)
    scale = 1.0 / np.sqrt(shape[5])
    got = run_device(sdk, q, k, v, None, scale, causal, dtype)
    q, k, v, got = head_subset(q, k, v, got)
    want, weight = sdpa_f64(q, k, v, scale, causal)
    want = want.astype(np.float16 if dtype == "f16" else np.float32)   # the output's rounding
    check(got, want, weight, dtype, f"{shape} causal={causal}")


# Long query ranges with few heads: split key ranges whose items would
# overflow the work table (128 per batch and head) take larger parts until
# they fit (before, such plans fell back to whole query blocks but kept a
# stale part count, so the split kernel ran without a split).
@pytest.mark.parametrize("shape,causal", [
    ((1, 2, 2, 2041, 2301, 64, 64), False), ((1, 2, 1, 1425, 3753, 64, 64), False),
    ((1, 4, 2, 1657, 2158, 128, 128), True), ((1, 1, 1, 2500, 3000, 128, 128), False),
    ((1, 1, 1, 3000, 4000, 64, 64), True)])
@pytest.mark.parametrize("dtype", ["f16", "f32"])
def test_split_work_table_limit(sdk, orc, shape, causal, dtype):
    q, k, v, _ = inputs(orc, shape, dtype, 45, False)
    scale = 1.0 / np.sqrt(shape[5])
    got = run_device(sdk, q, k, v, None, scale, causal, dtype)
    q, k, v, got = head_subset(q, k, v, got)
    want, weight = sdpa_f64(q, k, v, scale, causal)
    want = want.astype(np.float16 if dtype == "f16" else np.float32)
    check(got, want, weight, dtype, f"{shape} causal={causal}")


def sdpa_f64_masked(q, k, v, mask, scale, causal):
    """sdpa_f64 with an optional additive [Lq, Lkv] mask (entries may be
    -inf; every row here keeps a finite score)."""
    b, h, lq, d = q.shape
    kvh, lk = k.shape[1], k.shape[2]
    group = h // kvh
    kk = np.repeat(k.astype(np.float64), group, axis=1)
    vv = np.repeat(v.astype(np.float64), group, axis=1)
    s = np.einsum("bhid,bhjd->bhij", q.astype(np.float64), kk) * scale
    if mask is not None:
        s = s + mask.astype(np.float64)
    if causal:
        offset = max(lk - lq, 0)
        s = np.where(np.arange(lk)[None, :] > np.arange(lq)[:, None] + offset, -np.inf, s)
    p = np.exp(s - s.max(axis=-1, keepdims=True))
    p /= p.sum(axis=-1, keepdims=True)
    return p @ vv, p @ np.abs(vv)


def test_sdpa_f64_masked_matches_oracle(orc):
    for shape, causal in (((1, 2, 1, 37, 70, 32, 16), True), ((1, 2, 2, 40, 33, 64, 64), False)):
        q, k, v, mask = inputs(orc, shape, "f32", 46, True)
        want, weight = sdpa_f64_masked(q, k, v, mask, -0.1, causal)
        got = orc.sdpa(q, k, v, mask, -0.1, causal)
        assert np.allclose(got, want, rtol=0, atol=1e-5 * weight.max())


# Mixed cases drawn once with default_rng(11): masks, scales of zero and
# below (the general variant), head dims off the MFMA path (the row
# kernel), D != Dv, short and long key ranges.
MIXED_CASES = [
    ((1, 4, 1, 1567, 87, 32, 32), True, False, -0.1), ((1, 8, 8, 1733, 743, 64, 64), False, False, -0.1),
    ((1, 1, 1, 1218, 2471, 128, 64), True, False, 0.05), ((1, 2, 2, 1886, 2020, 64, 32), True, False, 0.0),
    ((1, 4, 2, 9, 2989, 128, 128), True, False, 0.0), ((1, 8, 1, 1293, 61, 16, 16), True, True, 0.05),
    ((2, 1, 1, 18, 1399, 128, 128), True, False, 0.0), ((2, 4, 1, 1970, 2220, 32, 32), False, True, 0.176777),
    ((1, 2, 1, 2067, 2181, 128, 128), True, False, 0.0), ((1, 16, 2, 237, 203, 128, 128), True, True, 0.088388),
    ((1, 16, 4, 316, 1990, 128, 128), False, False, 0.05), ((1, 8, 8, 1407, 490, 32, 32), False, True, 0.0),
    ((1, 2, 1, 15, 116, 96, 96), True, False, 0.05), ((1, 8, 2, 775, 276, 128, 128), True, False, 0.088388),
    ((1, 1, 1, 652, 1494, 64, 64), True, False, -0.1), ((1, 16, 4, 1481, 2295, 128, 128), True, False, -0.1),
]


@pytest.mark.parametrize("shape,causal,masked,scale", MIXED_CASES)
@pytest.mark.parametrize("dtype", ["f16", "f32"])
def test_mixed_cases(sdk, orc, shape, causal, masked, scale, dtype):
    q, k, v, mask = inputs(orc, shape, dtype, 47, masked)
    got = run_device(sdk, q, k, v, mask, scale, causal, dtype)
    q, k, v, got = head_subset(q, k, v, got)
    want, weight = sdpa_f64_masked(q, k, v, mask, scale, causal)
    want = want.astype(np.float16 if dtype == "f16" else np.float32)
    check(got, want, weight, dtype, f"{shape} causal={causal} mask={masked} scale={scale}")
