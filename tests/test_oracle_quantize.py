"""The oracle's quantize.rs restatement, pinned by the reference's unit tests (quantize.rs:167-216) and by closed
forms of the rounding rules."""

import numpy as np

import oracle


def test_uniform_is_in_unit_interval_and_row_keyed():
    # quantize.rs:171-181
    draws = np.array([oracle.uniform(7, 0, 3, r) for r in range(10_000)])
    assert ((draws >= 0) & (draws < 1)).all()
    assert abs(draws.mean() - 0.5) < 0.02
    assert oracle.uniform(7, 0, 3, 1 << 32) != oracle.uniform(7, 0, 3, 0)


def test_mix32_is_lowbias32():
    # lowbias32 (hash-prospector): 0 is its fixed point; the mixer is a bijection, so distinct inputs stay distinct
    assert oracle.lib().oracle_mix32(0) == 0
    xs = np.arange(1, 200_001, dtype=np.uint64) * 2654435761 % (1 << 32)
    out = {oracle.lib().oracle_mix32(int(x)) for x in xs[:20_000]}
    assert len(out) == 20_000


def test_stochastic_rounding_is_unbiased():
    # quantize.rs:183-192
    spec = oracle.quant_spec(2.0, 1.0, None, 4, True, 11, 0)
    n = 200_000
    packed = oracle.quantize(spec, np.full(n, 0.3, np.float32), np.full(n, 0.5, np.float32))
    g, _ = oracle.unpack(packed)
    mean = g.sum() / n * spec.grad_scale
    assert abs(mean - 0.3) < 0.01


def test_stochastic_rounding_brackets_the_scaled_value():
    # every g_q is floor or ceil of grad / scale (clamped); every h_q of hess / scale
    rng = np.random.default_rng(3)
    grad = (rng.standard_normal(50_000) * 0.7).astype(np.float32)
    hess = rng.uniform(0, 0.25, 50_000).astype(np.float32)
    spec = oracle.quant_spec(float(np.abs(grad).max()), float(hess.max()), None, 8, True, 5, 2)
    g, h = oracle.unpack(oracle.quantize(spec, grad, hess))
    x = grad.astype(np.float64) * spec.inv_grad_scale
    assert ((g == np.floor(x)) | (g == np.ceil(x)) | (np.abs(g) == spec.grad_max_q)).all()
    assert (np.abs(g) <= spec.grad_max_q).all()
    y = hess.astype(np.float64) * spec.inv_hess_scale
    assert ((h == np.floor(y)) | (h == np.ceil(y))).all()
    assert ((h >= 0) & (h <= spec.hess_max_q)).all()
    # both directions occur, at rates that track the fractional part
    frac = x - np.floor(x)
    up = (g == np.ceil(x)) & (frac > 0)
    assert abs(up.mean() - frac[frac > 0].mean() * (frac > 0).mean()) < 0.01


def test_deterministic_rounding_is_ties_to_even():
    # quantize.rs:119, 133: round_ties_even(grad * inv_scale)
    spec = oracle.quant_spec(4.0, 4.0, None, 8, False, 1, 0)  # grad_scale 1, hess_scale 0.5
    grad = np.array([0.5, 1.5, 2.5, -0.5, -1.5, 3.49, -3.51, 9.0], np.float32)
    hess = np.array([0.25, 0.75, 1.25, 0.0, 2.0, 0.1, 9.0, 1.0], np.float32)
    g, h = oracle.unpack(oracle.quantize(spec, grad, hess))
    assert list(g) == [0, 2, 2, 0, -2, 3, -4, 4]
    assert list(h) == [0, 2, 2, 0, 4, 0, 8, 2]


def test_pack_round_trips_negative_gradients():
    # quantize.rs:194-201
    gs = np.repeat(np.arange(-32, 33), 65)
    hs = np.tile(np.arange(0, 65), 65)
    packed = (hs * 65536 + gs).astype(np.int32)
    g, h = oracle.unpack(packed)
    assert (g == gs).all() and (h == hs).all()
    for gv, hv in [(-32, 64), (5, 0), (-1, 1)]:
        a, b = oracle.lib().oracle_unpack.argtypes[1]._type_(), oracle.lib().oracle_unpack.argtypes[2]._type_()
        oracle.lib().oracle_unpack(hv * 65536 + gv, a, b)
        assert (a.value, b.value) == (gv, hv)


def test_constant_hessian_counts_rows():
    # quantize.rs:203-207
    spec = oracle.quant_spec(1.0, 1.0, 1.0, 4, True, 1, 0)
    _, h = oracle.unpack(oracle.quantize(spec, np.array([-0.7], np.float32), np.array([1.0], np.float32), 5))
    assert h[0] == 1


def test_fixed_point_scale_bounds_magnitude():
    # quantize.rs:209-215
    s = oracle.lib().oracle_fixed_point_scale(3.7)
    assert float(np.float32(3.7) * np.float32(s)) <= 2.0 ** 30
    assert float(np.float32(3.7) * np.float32(s)) > 2.0 ** 29
    assert oracle.lib().oracle_fixed_point_scale(0.0) == 1.0
    assert oracle.lib().oracle_fixed_point_scale(float("inf")) == 1.0
    # a power of two: 2^(30 - ceil(log2 max))
    for m, e in [(1.0, 30), (0.75, 30), (2.0, 29), (1e-3, 39), (1000.0, 20)]:
        assert oracle.lib().oracle_fixed_point_scale(m) == 2.0 ** e


def test_scales_follow_the_maxima():
    # quantize.rs:56-84: grad_scale = max|g| / (bins/2), hess_scale = max h / bins; zero maxima give scale 1
    s = oracle.quant_spec(3.0, 2.0, None, 4, True, 1, 0)
    assert s.grad_scale == 1.5 and s.hess_scale == 0.5 and s.grad_max_q == 2 and s.hess_max_q == 4
    assert s.inv_grad_scale == np.float32(1 / 1.5)
    z = oracle.quant_spec(0.0, 0.0, None, 4, True, 1, 0)
    assert z.grad_scale == 1.0 and z.hess_scale == 1.0
    c = oracle.quant_spec(3.0, 2.0, 1.0, 16, True, 1, 0)
    assert c.hess_scale == 1.0 and c.constant_hessian == 1


def test_in_bag_fraction():
    got = np.mean([oracle.lib().oracle_in_bag(4, 1, r, 0.7) for r in range(20_000)])
    assert abs(got - 0.7) < 0.02


def _lightgbm_fixture():
    import json
    import pathlib

    return json.loads((pathlib.Path(__file__).parent / "golden" / "lightgbm_bins_all_rows.json").read_text())


def _fixture_columns(mix, rows):
    """The numerical columns of gen_lightgbm_bins.py:64-86 built with the mixer `mix`."""
    r = np.arange(rows, dtype=np.uint32)
    mr = mix(r)

    def unit(stream):
        h = mix(mr ^ mix(np.array([stream], np.uint32))[0])
        return (h >> np.uint32(8)).astype(np.float64) / 16777216.0

    a20, a40, a60 = unit(20), unit(40), unit(60)
    u50 = unit(50)
    return {
        "normal": (((unit(10) + unit(11)) + unit(12)) + unit(13) - 2.0) * 1.5,
        "zeros_nan": np.where(a20 < 0.3, 0.0, np.where(a20 < 0.4, np.nan, ((unit(21) + unit(22)) - 1.0) * 3.0)),
        "integers": np.floor(unit(30) * 20.0) - 5.0,
        "mass_points": np.where(a40 < 0.5, 1.0, ((unit(41) * unit(42)) * unit(43)) * 1000.0),
        "negative": -(u50 * u50 * 10.0) - 0.5,
        "tiny": np.where(a60 < 0.2, 1e-36, np.where(a60 < 0.3, -1e-36, unit(61) - 0.5)),
    }


def _lightgbm_range(col):
    """LightGBM 3.3.5 BinMapper's [min:max]: NaN dropped, |v| <= 1e-35 counted as zero, zero inside the range when
    any row is zero."""
    v = col[~np.isnan(col)]
    zero = np.abs(v) <= 1e-35
    nz = v[~zero]
    lo, hi = nz.min(), nz.max()
    if zero.any():
        lo, hi = min(lo, 0.0), max(hi, 0.0)
    return lo, hi


def test_mix32_rebuilds_the_lightgbm_fixture_ranges():
    # gen_lightgbm_bins.py:54-89 builds every feature from mix32; with 150,000 rows LightGBM's bin sample is all of
    # them, so the recorded feature_infos are the exact extremes of the mix32-built columns, to the last bit
    fx = _lightgbm_fixture()
    cols = _fixture_columns(oracle.mix32, fx["rows"])
    for name, col in cols.items():
        lo, hi = fx["feature_infos"][name].strip("[]").split(":")
        assert _lightgbm_range(col) == (float(lo), float(hi)), name


def test_the_lightgbm_ranges_reject_a_wrong_mixer():
    # the same check fails for a mixer one constant or one shift away from lowbias32
    fx = _lightgbm_fixture()

    def near_miss(mul2, shift2):
        def mix(x):
            x = x.astype(np.uint32)
            x ^= x >> np.uint32(16)
            x *= np.uint32(0x7FEB352D)
            x ^= x >> np.uint32(shift2)
            x *= np.uint32(mul2)
            x ^= x >> np.uint32(16)
            return x
        return mix

    for mix in (near_miss(0x846CA68D, 15), near_miss(0x846CA68B, 16)):
        cols = _fixture_columns(mix, fx["rows"])
        lo, hi = fx["feature_infos"]["normal"].strip("[]").split(":")
        assert _lightgbm_range(cols["normal"]) != (float(lo), float(hi))


# 16-bit units (num_grad_quant_bins up to 32766) are an extension of the reference, which takes 2..=64
# (config.rs:416-421): pinned by closed forms only. The units stay within their bounds, the packed word round trips
# them, and the oracle's histogram (64-bit packed blocks of INT32_MAX / max_q rows, cpu.rs:479-525) equals direct
# sums of the unpacked units.
def test_sixteen_bit_units_round_trip_and_sum_exactly():
    import silvic_amd
    from tests.helpers import naive_histogram

    data = silvic_amd.synthetic(2, rows=20_000, cols=24, seed=9)
    rng = np.random.default_rng(4)
    g = rng.standard_normal(data.num_rows).astype(np.float32)
    h = rng.uniform(0.05, 1.0, data.num_rows).astype(np.float32)
    for bins in (256, 4096, 32766):
        spec = oracle.quant_spec(float(np.abs(g).max()), float(h.max()), None, bins, True, 3, 1)
        assert spec.grad_max_q == bins // 2 and spec.hess_max_q == bins
        packed = oracle.quantize(spec, g, h)
        gq, hq = oracle.unpack(packed)
        assert gq.min() >= -bins // 2 and gq.max() <= bins // 2 and hq.min() >= 0 and hq.max() <= bins
        assert np.array_equal(packed, (hq.astype(np.int64) * 65536 + gq).astype(np.int32))
        assert np.abs(gq).max() > bins // 4  # the range is used
        # stochastic rounding brackets the scaled value
        sg = g.astype(np.float64) / spec.grad_scale
        assert (np.abs(gq - sg) < 1.0 + 1e-3).all()
        rows = np.sort(rng.choice(data.num_rows, 7_000, replace=False)).astype(np.uint32)
        got = oracle.histogram(data, packed, max(bins // 2, bins), rows)
        assert np.array_equal(got, naive_histogram(data, rows, gq[rows], hq[rows])), bins


def test_the_rocm_trainer_takes_sixteen_bit_units():
    from silvic_amd import _abi, engine

    for bins in (2, 64, 256, 32766):
        assert engine.resolve_params({"num_grad_quant_bins": bins})["num_grad_quant_bins"] == bins
    for bins in (0, 7, 32768):
        try:
            engine.resolve_params({"num_grad_quant_bins": bins})
        except _abi.SilvicError:
            continue
        raise AssertionError(bins)
