"""tensor_sum_max_f32_no_alloc: the allocation-free variant of
tensor_sum_max_f32 (partials in the library's fixed device array instead of
allocated scratch). Through the C ABI it must give exactly the results of
tensor_sum_max_f32 -- the same kernels over the same partial layout -- on two
calls in a row, the second smaller than the first (the array keeps the first
call's partials, which the second must not read), and match the oracle to the
reductions' bar. Host-storage operands and malformed outputs are refused
before any device work."""
import numpy as np
import pytest

from inference_c_amd import SdkError


def _run(sdk, name, tx, with_sum=True, with_max=True):
    ts = sdk.tensor("f64", (1,)) if with_sum else None
    tm = sdk.tensor("f32", (1,)) if with_max else None
    sdk.call(name, tx, ts, tm)
    return (None if ts is None else ts.download()[0]), (None if tm is None else tm.download()[0])


@pytest.mark.gpu
def test_no_alloc_matches_allocating_entry_point(sdk, orc):
    sizes = [(1 << 28) + 12345, 1000003]   # second call smaller: 2049 then 8 partials
    for seed, n in enumerate(sizes):
        print(f"no-alloc sum/max, call {seed + 1}: {n} elements", flush=True)
        tx = sdk.tensor("f32", (n,))
        sdk.call("tensor_fill_uniform", tx, 50 + seed, 0, -1.0, 1.0)
        s_ref, m_ref = _run(sdk, "tensor_sum_max_f32", tx)
        s, m = _run(sdk, "tensor_sum_max_f32_no_alloc", tx)
        assert np.float64(s).tobytes() == np.float64(s_ref).tobytes()
        assert np.float32(m).tobytes() == np.float32(m_ref).tobytes()
        x = tx.download()
        want_s, abs_s, want_m = orc.sum_max(x)
        assert abs(float(s) - want_s) <= 1e-6 * abs_s
        assert m == want_m
        del tx


@pytest.mark.gpu
def test_no_alloc_single_output_and_specials(sdk, orc):
    x = orc.uniform((100000,), 51, 0, -1.0, 1.0)
    tx = sdk.from_numpy(x)
    s, m = _run(sdk, "tensor_sum_max_f32_no_alloc", tx, with_max=False)
    s_ref, _ = _run(sdk, "tensor_sum_max_f32", tx, with_max=False)
    assert m is None and np.float64(s).tobytes() == np.float64(s_ref).tobytes()
    _, m = _run(sdk, "tensor_sum_max_f32_no_alloc", tx, with_sum=False)
    assert m == x.max()
    x[77] = np.nan
    s, m = _run(sdk, "tensor_sum_max_f32_no_alloc", sdk.from_numpy(x))
    assert np.isnan(s) and np.isnan(m)


def test_no_alloc_refuses_host_operands(lib):
    from inference_c_amd import Sdk
    sdk = Sdk()
    tx = sdk.from_numpy(np.ones(16, np.float32), device=False)
    ts, tm = sdk.tensor("f64", (1,), False), sdk.tensor("f32", (1,), False)
    with pytest.raises(SdkError, match="requires device-storage operands"):
        sdk.call("tensor_sum_max_f32_no_alloc", tx, ts, tm)
    with pytest.raises(SdkError, match="non-empty F32 input"):
        sdk.call("tensor_sum_max_f32_no_alloc", tx, tm, ts)
