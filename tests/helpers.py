"""Comparison rules shared by the tests (tolerances from BASELINE.json's
north_star: add/mul bit-exact; transcendentals <= 1 f16 ulp or 1e-6 relative
in f32; reductions 1e-5 relative f32 / 2e-3 f16)."""
import numpy as np


def f16_ordinal(a: np.ndarray) -> np.ndarray:
    """Monotonic integer image of f16 bit patterns (ulp distance = difference)."""
    b = np.ascontiguousarray(a).view(np.uint16).astype(np.int32)
    return np.where(b & 0x8000, 0x8000 - b, b)


def f32_ordinal(a: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(a, np.float32).view(np.uint32).astype(np.int64)
    return np.where(b & 0x80000000, 0x80000000 - b, b)


def f16_ulps(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """ulp distance of two f16 arrays; NaN vs NaN counts 0, NaN vs number huge."""
    d = np.abs(f16_ordinal(a) - f16_ordinal(b))
    an, bn = np.isnan(a.astype(np.float32)), np.isnan(b.astype(np.float32))
    d = np.where(an & bn, 0, d)
    return np.where(an ^ bn, 1 << 20, d)


def f32_ulps(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    d = np.abs(f32_ordinal(a) - f32_ordinal(b))
    an, bn = np.isnan(a), np.isnan(b)
    d = np.where(an & bn, 0, d)
    return np.where(an ^ bn, 1 << 40, d)


def assert_bits_equal(got: np.ndarray, want: np.ndarray, what: str = "") -> None:
    g = np.ascontiguousarray(got)
    w = np.ascontiguousarray(want)
    assert g.shape == w.shape, (what, g.shape, w.shape)
    if g.dtype == np.float16 or g.dtype == np.float32:
        gn, wn = np.isnan(g.astype(np.float32)), np.isnan(w.astype(np.float32))
        assert np.array_equal(gn, wn), f"{what}: NaN positions differ"
        g, w = np.where(gn, 0, g), np.where(wn, 0, w)
        view = np.uint16 if got.dtype == np.float16 else np.uint32
        bad = np.flatnonzero(g.view(view) != w.view(view))
    else:
        bad = np.flatnonzero(g != w)
    assert bad.size == 0, (f"{what}: {bad.size} of {g.size} differ; first at {bad[:5]}: "
                           f"{g.reshape(-1)[bad[:5]]} vs {w.reshape(-1)[bad[:5]]}")


def assert_f16_ulps(got, want, max_ulps=1, what=""):
    d = f16_ulps(got, want)
    worst = int(d.max()) if d.size else 0
    assert worst <= max_ulps, (f"{what}: max {worst} ulp (> {max_ulps}); "
                               f"{int((d > max_ulps).sum())} elements")


def assert_f32_rel(got, want, rel, what="", floor=0.0):
    """|got - want| <= rel * |want| + floor, NaN positions equal."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    gn, wn = np.isnan(got), np.isnan(want)
    assert np.array_equal(gn, wn), f"{what}: NaN positions differ"
    g, w = got[~gn], want[~wn]
    inf = np.isinf(w)
    assert np.array_equal(g[inf], w[inf]), f"{what}: infinities differ"
    err = np.abs(g[~inf] - w[~inf])
    bound = rel * np.abs(w[~inf]) + floor
    bad = np.flatnonzero(err > bound)
    assert bad.size == 0, (f"{what}: {bad.size} elements beyond rel {rel}; worst ratio "
                           f"{float((err / np.maximum(bound, 1e-300)).max()):.3g}")


def arbitrated(got: np.ndarray, ref: np.ndarray, exact: np.ndarray, ulps) -> np.ndarray:
    """Elements that pass the transcendental rule: within one ulp of the
    reference, or no farther from the double-precision evaluation of the
    same formula than the reference is (the reference's own float evaluation
    of 1 + tanh(u) cancels near x = -5)."""
    within = ulps(got, ref) <= 1
    g = got.astype(np.float64)
    r = ref.astype(np.float64)
    with np.errstate(invalid="ignore"):   # Inf - Inf: NaN compares False; `within` decides
        closer = np.abs(g - exact) <= np.abs(r - exact)
    return within | closer


def rope_close(got, want, src, what="RoPE"):
    """RoPE f16 rule: 1 f16 ulp, or -- where l*c - r*s cancels -- the f32
    error of a rotation whose cos/sin are each within an f32 ulp of the
    reference's: 2^-22 (|l| + |r|).

    Returns (elements, within 1 ulp, passing only through the cancellation
    clause, largest ulp distance among those) and prints it, so that a
    widening of the second clause cannot hide behind it."""
    half = src.shape[-1] // 2
    pair = np.abs(src[..., :half].astype(np.float64)) + np.abs(src[..., half:].astype(np.float64))
    pair = np.concatenate([pair, pair], axis=-1)
    d = np.abs(got.astype(np.float64) - want.astype(np.float64))
    ulps = f16_ulps(got, want)
    near = ulps <= 1
    cancel = ~near & (d <= 2.0 ** -22 * pair)
    ok = near | cancel
    worst = int(ulps[cancel].max()) if cancel.any() else 0
    counts = (int(ok.size), int(near.sum()), int(cancel.sum()), worst)
    print(f"{what}: {counts[0]} elements, {counts[1]} within 1 ulp, {counts[2]} only through "
          f"the cancellation clause (largest distance there {worst} ulp)", flush=True)
    assert ok.all(), f"{(~ok).sum()} elements beyond the RoPE bound"
    return counts
