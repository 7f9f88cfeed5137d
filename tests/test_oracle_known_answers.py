"""The oracle against the reference's own known-answer tests:
tests/test_tensor_ops.c, tests/test_tensor_compute.c, tests/test_attention.c
and tests/test_cuda_vision_sequence.cu of the reference (values restated)."""
import math

import numpy as np

F16 = np.float16


def h(bits):
    return np.array(bits, np.uint16).view(F16)


def test_residual_add_f16_bit_exact(orc):
    # test_tensor_ops.c:131-150, test_tensor_device.c:144-176
    got = orc.add(h([0x3c00, 0xc000, 0x4200, 0xc400]), h([0x4000, 0x3800, 0xbc00, 0x4400]))
    assert got.view(np.uint16).tolist() == [0x4200, 0xbe00, 0x4000, 0x0000]


def test_rms_norm_f32(orc):
    # test_tensor_ops.c:84-97
    y = orc.rms_norm(np.array([[3, 4], [0, 2]], np.float32), np.array([2, .5], np.float32), 0.0)
    assert np.allclose(y.ravel(), [1.69705627, 0.56568545, 0.0, 0.70710678], atol=1e-5, rtol=0)
    # test_tensor_compute.c:121-128 (vtable form)
    y = orc.rms_norm(np.array([[1, 2], [3, 4]], np.float32), np.ones(2, np.float32), 1e-5)
    assert np.allclose(y.ravel(), [0.63245, 1.2649, 0.84853, 1.13137], atol=2e-4, rtol=0)


def test_layer_norm_f32(orc):
    # test_tensor_ops.c:99-118
    x = np.array([[1, 2, 3, 4], [2, 2, 2, 2]], np.float32)
    y = orc.layer_norm(x, np.array([1, 2, 1, .5], np.float32), np.array([0, 1, -1, 2], np.float32), 1e-5)
    want = [-1.34164079, 0.10557281, -0.55278640, 2.67082039, 0.0, 1.0, -1.0, 2.0]
    assert np.allclose(y.ravel(), want, atol=1e-5, rtol=0)
    # test_tensor_compute.c:130-139
    y = orc.layer_norm(np.array([[1, 3], [2, 4]], np.float32), np.ones(2, np.float32),
                       np.zeros(2, np.float32), 1e-5)
    assert np.allclose(y.ravel(), [-1, 1, -1, 1], atol=2e-4, rtol=0)


def test_silu_f32(orc):
    # test_tensor_ops.c:120-129
    y = orc.silu(np.array([-2, -1, 0, 1], np.float32))
    assert np.allclose(y, [-0.23840584, -0.26894143, 0.0, 0.73105858], atol=1e-5, rtol=0)


def test_bias_add_f32(orc):
    # test_tensor_compute.c:141-148
    y = orc.bias_add(np.array([[1, 2], [3, 4]], np.float32), np.array([10, 20], np.float32))
    assert y.ravel().tolist() == [11, 22, 13, 24]


def test_gelu_f32_with_clamps(orc):
    # test_tensor_compute.c:150-158
    y = orc.gelu(np.array([0, 1, 10.375, -10.375, 20, -20], np.float32))
    assert np.all(np.isfinite(y))
    assert abs(y[0]) < 2e-4 and abs(y[1] - 0.84119) < 2e-4
    assert abs(y[2] - 10.375) < 2e-4 and abs(y[3]) < 2e-4


def test_rope_f32(orc):
    # test_tensor_compute.c:160-168: seq 2, one head each, dim 2, theta 1e4
    q, k = orc.rope(np.array([1, 0, 1, 0], np.float32), np.array([1, 0, 1, 0], np.float32),
                    1, 1, 2, 10000.0)
    for v in (q, k):
        assert np.allclose(v, [1, 0, math.cos(1.0), math.sin(1.0)], atol=2e-4, rtol=0)


def test_silu_multiply_f32(orc):
    # test_tensor_compute.c:170-175 (first operand is SiLU'd)
    y = orc.silu_multiply(np.array([0, 1], np.float32), np.array([2, 3], np.float32))
    assert np.allclose(y, [0, 2.19318], atol=2e-4, rtol=0)


def test_gelu_multiply_f16(orc):
    # test_tensor_compute.c:177-193 and test_cuda_vision_sequence.cu:95-122
    x = np.array([0, 1, -1, 0.5, 10.375, -10.375], np.float32).astype(F16)
    g = np.array([2, 3, 4, -2, 0.25, 1.5], np.float32).astype(F16)
    y = orc.gelu_multiply(x, g).astype(np.float32)
    for xi, gi, yi in zip(x.astype(np.float32), g.astype(np.float32), y):
        gelu = xi if xi >= 5 else 0.0 if xi <= -5 else \
            0.5 * xi * (1.0 + math.tanh(0.7978845608 * (xi + 0.044715 * xi ** 3)))
        assert abs(yi - gelu * gi) < 2e-3


def test_relu_f16(orc):
    # test_tensor_compute.c:194-199, test_cuda_vision_sequence.cu:123-134
    y = orc.relu(h([0xbc00, 0x0000, 0x4200])).astype(np.float32)
    assert y.tolist() == [0.0, 0.0, 3.0]


def test_residual_add_f32(orc):
    # test_tensor_compute.c:201-207
    assert orc.add(np.array([1, 2, 3], np.float32), np.array([4, 5, 6], np.float32)).tolist() == [5, 7, 9]


def test_argmax_ties_first(orc):
    # test_tensor_compute.c:209-212
    assert orc.argmax(np.array([-2, 5, 5, 1], np.float32)) == 1


def test_softmax_sdpa_known_answers(orc):
    """test_attention.c:441-496: Q rows (1,0),(0,1), K = I, V rows (1,0),(0,2),
    scale 1. Output = softmax(QK^T) V."""
    v = np.array([[1, 0], [0, 2]], np.float64)
    scores = np.array([[1, 0], [0, 1]], np.float32)
    out = orc.softmax(scores).astype(np.float64) @ v
    assert np.allclose(out.ravel(), [0.73105858, 0.53788284, 0.26894143, 1.4621172], atol=1e-5)
    out = orc.softmax(scores, causal=True).astype(np.float64) @ v
    assert np.allclose(out[0], [1.0, 0.0], atol=1e-5)
    assert np.allclose(out[1], [0.26894143, 1.4621172], atol=1e-5)
    # additive mask [-inf, 0; 0, 0] makes row 0 pick key 1: output (0, 2)
    masked = scores + np.array([[-np.inf, 0], [0, 0]], np.float32)
    out = orc.softmax(masked).astype(np.float64) @ v
    assert np.allclose(out[0], [0.0, 2.0], atol=1e-5)
    # all masked -> zeros
    allm = np.full((2, 2), -np.inf, np.float32)
    assert np.all(orc.softmax(allm) == 0.0)


def test_embedding_lookup_f32(orc):
    # test_tensor_ops.c:62-82: ids {2, 0, 2} pick rows 2, 0, 2; id 4 of a
    # 4-row table is rejected
    table = np.array([0, 1, 2, 10, 11, 12, 20, 21, 22, 30, 31, 32], np.float32).reshape(4, 3)
    got = orc.embedding_lookup(table, np.array([2, 0, 2], np.uint32))
    assert got.ravel().tolist() == [20, 21, 22, 0, 1, 2, 20, 21, 22]
    assert orc.embedding_lookup(table, np.array([2, 4, 2], np.uint32)) is None


def test_embedding_compute_slot_f32(orc):
    # test_tensor_compute.c:112-119 (embedding_f32 slot, uint32 ids)
    table = np.arange(8, dtype=np.float32).reshape(4, 2)
    got = orc.embedding_gather_u32(table, np.array([2, 0], np.uint32))
    assert got.ravel().tolist() == [4, 5, 0, 1]


def test_sdpa_accelerator_semantics_known_answers(orc):
    # test_attention.c:441-496: the same values whichever backend runs them
    q = np.array([1, 0, 0, 1, 1, 0, 0, 1], np.float32).reshape(1, 2, 2, 2)
    k = np.array([1, 0, 0, 1], np.float32).reshape(1, 1, 2, 2)
    v = np.array([1, 0, 0, 2], np.float32).reshape(1, 1, 2, 2)
    near = lambda a, b: np.allclose(a, b, atol=1e-5, rtol=0)
    out = orc.sdpa(q, k, v, None, 1.0, False).ravel()
    assert near(out[:4], [0.73105858, 0.53788284, 0.26894143, 1.4621172]) and near(out[4:], out[:4])
    out = orc.sdpa(q, k, v, None, 1.0, True).ravel()
    assert near(out[:4], [1.0, 0.0, 0.26894143, 1.4621172])
    mask = np.array([-np.inf, 0, 0, 0], np.float32).reshape(2, 2)
    out = orc.sdpa(q, k, v, mask, 1.0, False).ravel()
    assert near(out[:2], [0.0, 2.0])
    all_masked = np.full((2, 2), -np.inf, np.float32)
    assert (orc.sdpa(q, k, v, all_masked, 1.0, False) == 0).all()
    # the same through f16 inputs and outputs
    out16 = orc.sdpa(q.astype(F16), k.astype(F16), v.astype(F16), None, 1.0, False).ravel()
    assert np.allclose(out16.astype(np.float32)[:4], [0.73105858, 0.53788284, 0.26894143, 1.4621172],
                       atol=1e-3, rtol=0)
