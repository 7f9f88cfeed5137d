"""BASELINE configs[4]'s decoder-layer non-GEMM chain at its full shape, run
as the bench runs it: fused residual add + RMSNorm on [4096, 2048], RoPE on
q, k [4096, 32, 64] (theta 1e4, positions 0..4095) and SwiGLU on
[4096, 8192], enqueued back to back on device buffers with one
synchronisation at the end, against the CPU oracle on the same seeded inputs
(the bench's seeds). The sum is bit-exact; the normalised rows, the rotations
and SwiGLU follow the f16 transcendental rules (1 ulp; RoPE's cancellation
bound)."""
import pytest

from tests.helpers import assert_bits_equal, assert_f16_ulps, rope_close

pytestmark = pytest.mark.gpu


def test_config5_chain_full_size(sdk, orc):
    tok, hid, inter, heads, dim = 4096, 2048, 8192, 32, 64
    print("configs[4] chain: [4096,2048] residual+RMSNorm, RoPE [4096,32,64], "
          "SwiGLU [4096,8192]", flush=True)
    x = orc.normal((tok, hid), 5, 0, 0.0, 1.0)
    r = orc.normal((tok, hid), 5, 1, 0.0, 1.0)
    w = orc.normal((hid,), 5, 9, 0.0, 1.0)
    q = orc.normal((tok, heads, dim), 5, 2, 0.0, 1.0)
    k = orc.normal((tok, heads, dim), 5, 3, 0.0, 1.0)
    gate = orc.normal((tok, inter), 5, 4, 0.0, 1.0)
    up = orc.normal((tok, inter), 5, 5, 0.0, 1.0)
    tx, tr, tw = sdk.from_numpy(x), sdk.from_numpy(r), sdk.from_numpy(w)
    th, tn = sdk.tensor("f16", x.shape), sdk.tensor("f16", x.shape)
    tq, tk = sdk.from_numpy(q), sdk.from_numpy(k)
    tg, tu, to = sdk.from_numpy(gate), sdk.from_numpy(up), sdk.tensor("f16", gate.shape)
    sdk.synchronize()
    sdk.call("tensor_residual_rms_norm_f16", tx, tr, tw, 1e-6, th, tn)
    sdk.call("tensor_rope_f16", tq, tk, heads, heads, dim, 10000.0, 0)
    sdk.call("tensor_silu_multiply_f16", tg, tu, to)
    sdk.synchronize()
    h_ref, n_ref = orc.residual_rms_norm(x, r, w, 1e-6)
    assert_bits_equal(th.download(), h_ref, "residual sum")
    assert_f16_ulps(tn.download(), n_ref, 1, "RMSNorm of the sum")
    q_ref, k_ref = orc.rope(q, k, heads, heads, dim, 10000.0)
    # the cancellation clause must stay a rare exception at the full shape
    for name, got, want, src in (("q", tq, q_ref, q), ("k", tk, k_ref, k)):
        total, _, cancel, _ = rope_close(got.download(), want, src, f"RoPE {name} [4096,32,64]")
        assert cancel <= total // 10000, f"RoPE {name}: {cancel} of {total} pass only by cancellation"
    assert_f16_ulps(to.download(), orc.silu_multiply(gate, up), 1, "SwiGLU [4096, 8192]")
