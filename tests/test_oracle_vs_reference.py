"""The oracle restatement against the reference's own portable C path
(oracle/_ref/libref.so, compiled from the reference sources), bit for bit on
seeded inputs: tensor_silu_*, tensor_rms_norm_*, tensor_layer_norm_*,
tensor_residual_add_f16 and the softmax inside tensor_sdpa_f32."""
import numpy as np
import pytest

from tests.helpers import assert_bits_equal

SHAPES = [(1, 1), (3, 7), (16, 64), (5, 1000), (2, 2048)]


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("dtype", ["f16", "f32"])
def test_silu(orc, ref, shape, dtype):
    x = orc.normal(shape, 11, 0, 0.0, 4.0, dtype)
    assert_bits_equal(orc.silu(x), ref.silu(x), "silu")


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("dtype", ["f16", "f32"])
@pytest.mark.parametrize("eps", [0.0, 1e-6, 1e-2])
def test_rms_norm(orc, ref, shape, dtype, eps):
    x = orc.normal(shape, 12, 0, 0.0, 1.0, dtype)
    w = orc.uniform(shape[-1:], 12, 1, 0.5, 1.5, dtype)
    assert_bits_equal(orc.rms_norm(x, w, eps), ref.rms_norm(x, w, eps), "rms_norm")


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("dtype", ["f16", "f32"])
@pytest.mark.parametrize("affine", ["none", "scale", "both"])
def test_layer_norm(orc, ref, shape, dtype, affine):
    x = orc.normal(shape, 13, 0, 0.5, 2.0, dtype)
    scale = orc.uniform(shape[-1:], 13, 1, 0.5, 1.5, dtype) if affine != "none" else None
    bias = orc.uniform(shape[-1:], 13, 2, -1.0, 1.0, dtype) if affine == "both" else None
    assert_bits_equal(orc.layer_norm(x, scale, bias, 1e-5), ref.layer_norm(x, scale, bias, 1e-5),
                      "layer_norm")


@pytest.mark.parametrize("n", [1, 4, 1000, 65536])
def test_residual_add_f16(orc, ref, n):
    a = orc.normal((n,), 14, 0, 0.0, 100.0)
    b = orc.normal((n,), 14, 1, 0.0, 100.0)
    assert_bits_equal(orc.add(a, b), ref.residual_add_f16(a, b), "residual add")


def test_residual_add_f16_all_pairs_sample(orc, ref):
    """Every half against a fixed set of partners, including specials."""
    a = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16)
    for partner in (0x0000, 0x8000, 0x3c00, 0x0001, 0x7bff, 0xfbff, 0x7c00, 0x3555):
        b = np.full(65536, partner, np.uint16).view(np.float16)
        assert_bits_equal(orc.add(a, b), ref.residual_add_f16(a, b), f"partner {partner:#x}")


@pytest.mark.parametrize("q_len,k_len", [(1, 1), (4, 4), (5, 9), (33, 64), (64, 300)])
@pytest.mark.parametrize("causal", [False, True])
def test_softmax_via_sdpa(orc, ref, q_len, k_len, causal):
    s = orc.normal((q_len, k_len), 15, 0, 0.0, 3.0, "f32")
    assert_bits_equal(orc.softmax(s, causal), ref.softmax_rows_f32(s, causal), "softmax")


def test_softmax_special_rows_via_sdpa(orc, ref):
    """+inf rows, -inf (masked) entries, all -inf rows, huge finite values.
    NaN scores are not reachable through the reference's public API; the NaN
    rule is restated from attention.c:346-372 and checked in test_oracle_math."""
    inf = np.inf
    s = np.array([[1, 2, inf, 3], [inf, inf, 0, 1], [-inf, -inf, -inf, -inf],
                  [-inf, 5, -inf, 5], [1e30, -1e30, 0, 1], [-inf, -inf, inf, -inf]], np.float32)
    for causal in (False, True):
        assert_bits_equal(orc.softmax(s, causal), ref.softmax_rows_f32(s, causal), "special rows")


INDEX_TYPES = [np.int16, np.uint16, np.int32, np.uint32, np.int64, np.uint64]


@pytest.mark.parametrize("index_type", INDEX_TYPES)
@pytest.mark.parametrize("dtype", ["f16", "f32"])
@pytest.mark.parametrize("case", ["valid", "negative", "past_end", "last_row", "empty"])
def test_embedding_lookup(orc, ref, index_type, dtype, case):
    """tensor_embedding_lookup_* (src/common/tensor_ops.c:86-161): outputs
    and the accept/reject decision agree for every index dtype."""
    rows, width = 37, 5
    table = orc.normal((rows, width), 16, 0, 0.0, 1.0, dtype)
    ids = (orc.uniform((23,), 16, 1, 0.0, rows - 0.001, "f32")).astype(np.int64)
    if case == "negative":
        if not np.issubdtype(index_type, np.signedinteger):
            pytest.skip("unsigned indices cannot be negative")
        ids[7] = -1
    elif case == "past_end":
        ids[11] = rows
    elif case == "last_row":
        ids[-1] = rows - 1
    elif case == "empty":
        ids = ids[:0]
    ids = ids.astype(index_type)
    ok, got, message = ref.embedding_lookup(table, ids)
    want = orc.embedding_lookup(table, ids)
    assert ok == (want is not None), message
    if ok:
        assert_bits_equal(want, got, "embedding")
        assert_bits_equal(want, table[ids.astype(np.int64)], "embedding vs numpy take")
    else:
        assert message == "embedding index is negative or outside the table"


def test_embedding_lookup_f16_rejects_float_indices(orc, ref):
    """The F16 entry point does not check the index dtype up front: a
    non-integer index buffer fails when its first index is read."""
    table = orc.normal((4, 3), 17, 0, 0.0, 1.0, "f16")
    ids = np.array([1.0, 2.0], np.float32)
    ok, _, message = ref.embedding_lookup(table, ids)
    assert not ok and message == "embedding index is negative or outside the table"
    assert orc.embedding_lookup(table, ids) is None


@pytest.mark.parametrize("shape", [(1, 4, 2, 5, 9, 16, 8), (2, 2, 1, 33, 33, 64, 64),
                                   (1, 3, 3, 7, 4, 5, 3), (1, 2, 2, 1, 50, 32, 32)])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("masked", [False, True])
def test_sdpa_f32_matches_reference_cpu_path(orc, ref, shape, causal, masked):
    """The accelerator-semantics restatement (attention_cuda.cu:25-99) against
    the reference build's tensor_sdpa_f32 (its CPU loop, attention.c:227-410)
    on finite inputs: the two differ only in p / sum versus p * (1 / sum), so
    every output is within a few f32 roundings of sum_j p_j |v_j|."""
    b, h, kh, lq, lk, d, dv = shape
    q = orc.normal((b, h, lq, d), 19, 0, 0.0, 1.0, "f32")
    k = orc.normal((b, kh, lk, d), 19, 1, 0.0, 1.0, "f32")
    v = orc.normal((b, kh, lk, dv), 19, 2, 0.0, 1.0, "f32")
    mask = None
    if masked:
        mask = orc.uniform((lq, lk), 19, 3, -4.0, 0.0, "f32")
        mask[:, 0] = -np.inf  # a masked key in every row
    ok, want, message = ref.sdpa_f32(q, k, v, mask, 0.25, causal)
    assert ok, message
    got = orc.sdpa(q, k, v, mask, 0.25, causal)
    weight = orc.sdpa_abs_weight(q, k, v, mask, 0.25, causal)
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    assert (err <= 1e-6 * weight + 1e-30).all(), float((err / np.maximum(weight, 1e-30)).max())


def test_sdpa_special_rows(orc):
    """Closed forms of the accelerator rules (attention_cuda.cu:44-54): a row
    whose scores are all -inf is zero; a +inf score makes the row's max
    non-finite, so the row is zero (the CPU loop would share the row among the
    +inf keys instead); a NaN score never becomes the max, so a row of only
    NaN scores is zero, while a NaN beside finite scores makes the row NaN."""
    q = np.zeros((1, 1, 3, 4), np.float32)
    q[0, 0, 1] = 1e38           # row 1: scores overflow to +inf
    q[0, 0, 2] = 1.0            # row 2: finite scores
    k = np.ones((1, 1, 2, 4), np.float32)
    k[0, 0, 1, 0] = np.nan       # key 1 scores NaN in every row
    v = np.arange(4, dtype=np.float32).reshape(1, 1, 2, 2)
    mask = np.zeros((3, 2), np.float32)
    mask[0] = -np.inf            # row 0: key 0 masked, key 1 NaN -> no finite max
    out = orc.sdpa(q, k, v, mask, 1.0, False)
    assert (out[0, 0, 0] == 0).all() and (out[0, 0, 1] == 0).all()
    assert np.isnan(out[0, 0, 2]).all()
    k_all_nan = np.full((1, 1, 2, 4), np.nan, np.float32)
    assert (orc.sdpa(q, k_all_nan, v, None, 1.0, False) == 0).all()
