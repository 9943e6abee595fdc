"""CPU tests pinning the numpy oracle (no GPU).

The oracle is checked against (a) the committed torch-CPU fixtures in
tests/golden/ (torch is the library the reference's FP8 path is written in),
(b) brute force over the FP8 code tables and exact integer maths, and
(c) the invariants the reference's own tests assert.  Each check is chosen
so that a plausible slip in the oracle (wrong rounding direction, a dropped
clamp, dtype of the scale arithmetic, op order of the error update) fails.
"""
from pathlib import Path

import numpy as np
import pytest

from oracle import fp8 as ofp8
from oracle import gemm as og
from oracle import quant as oq

GOLD = np.load(Path(__file__).parent / "golden" / "torch_primitives.npz")
GOLD_BS = np.load(Path(__file__).parent / "golden" / "torch_block_scales.npz")


# ---------------------------------------------------------------- fp8 casts
def test_decode_tables_match_torch():
    for fmt, key in ((ofp8.E4M3, "dec_e4m3"), (ofp8.E5M2, "dec_e5m2")):
        mine = ofp8.DECODE[fmt]
        ref = GOLD[key]
        same = (mine == ref) | (np.isnan(mine) & np.isnan(ref))
        assert same.all(), fmt


@pytest.mark.parametrize("fmt", [ofp8.E4M3, ofp8.E5M2])
def test_encode_matches_torch_fixture(fmt):
    x, c = (GOLD["x_e4m3"], GOLD["c_e4m3"]) if fmt == ofp8.E4M3 else (GOLD["x_e5m2"], GOLD["c_e5m2"])
    assert np.array_equal(ofp8.encode(x, fmt), c)


def _brute_nearest_even(x, fmt):
    """Nearest finite code by exhaustive search; ties -> even mantissa."""
    table = ofp8.DECODE[fmt].astype(np.float64)
    codes = np.arange(256)
    ok = np.isfinite(table)
    table, codes = table[ok], codes[ok]
    out = np.empty(x.shape, dtype=np.uint8)
    for i, v in enumerate(x.astype(np.float64)):
        d = np.abs(table - v)
        best = d.min()
        cand = codes[d == best]
        # prefer same sign (signed zero) then even mantissa bit
        sgn = 0x80 if np.signbit(v) else 0
        cand = sorted(cand, key=lambda c: (((c & 0x80) != sgn), c & 1))
        out[i] = cand[0]
    return out


@pytest.mark.parametrize("fmt", [ofp8.E4M3, ofp8.E5M2])
def test_encode_is_nearest_even_by_brute_force(fmt):
    rng = np.random.default_rng(1)
    mx = ofp8.FP8_MAX[fmt]
    fin = np.unique(ofp8.DECODE[fmt][np.isfinite(ofp8.DECODE[fmt])]).astype(np.float64)
    mids = ((fin[:-1] + fin[1:]) / 2).astype(np.float32)
    x = np.concatenate([
        rng.uniform(-mx, mx, 1500).astype(np.float32),
        (rng.standard_normal(1500) * 2.0 ** rng.integers(-20, 4, 1500)).astype(np.float32),
        mids, np.nextafter(mids, np.float32(np.inf)), np.nextafter(mids, np.float32(-np.inf)),
        np.float32([0.0, -0.0, 1e-30, -1e-30, mx, -mx]),
    ]).astype(np.float32)
    assert np.array_equal(ofp8.encode(x, fmt), _brute_nearest_even(x, fmt))


def test_bf16_round_matches_torch():
    import torch

    rng = np.random.default_rng(2)
    x = (rng.standard_normal(200000) * 10.0 ** rng.uniform(-10, 10, 200000)).astype(np.float32)
    assert np.array_equal(ofp8.bf16_round(x), torch.from_numpy(x).bfloat16().float().numpy())


# ------------------------------------------------------------ ceil(log2(q))
def test_ceil_log2_matches_torch_fixture():
    assert np.array_equal(oq.ceil_log2_f32(GOLD["q"]), GOLD["clog2"].astype(np.int64))


def test_ceil_log2_is_exact_away_from_boundaries():
    # for q far from a power of two, ceil(log2(q)) is the exact integer
    rng = np.random.default_rng(3)
    k = rng.integers(-126, 120, 50000)
    m = rng.uniform(1.01, 1.99, 50000)
    q = (m * 2.0 ** k).astype(np.float32)
    assert np.array_equal(oq.ceil_log2_f32(q), k + 1)
    # exact powers of two
    p = (2.0 ** np.arange(-126, 127)).astype(np.float32)
    assert np.array_equal(oq.ceil_log2_f32(p), np.arange(-126, 127))


def test_ceil_log2_boundary_rounds_like_correctly_rounded_log2():
    # q = 2^k (1 + j 2^-23): a correctly rounded fp32 log2 returns exactly k
    # for small j; high-precision log2 + fp32 rounding decides which j.
    ks = np.arange(-126, 121)
    js = np.arange(1, 30)
    bits = ((ks[:, None] + 127) << 23) | js[None, :]
    q = bits.astype(np.uint32).view(np.float32)
    exact = np.log2(1.0 + js.astype(np.longdouble) * np.longdouble(2.0) ** -23)
    rl = (ks[:, None].astype(np.longdouble) + exact[None, :]).astype(np.float32)
    expect = np.where(rl == ks[:, None].astype(np.float32), ks[:, None], ks[:, None] + 1)
    assert np.array_equal(oq.ceil_log2_f32(q.ravel()), expect.ravel())


# ------------------------------------------------------ per-tensor scaling
def test_per_tensor_scale_matches_torch_rdiv_fp32():
    for a, s, inv in zip(GOLD["amax"], GOLD["scale_f32"], GOLD["inv_f32"]):
        t = np.array([a, -a / 2], dtype=np.float32)
        sc = oq.per_tensor_scale(t, "f32")
        assert sc == s and np.float32(1.0) / sc == inv


def test_per_tensor_scale_matches_torch_rdiv_e5m2():
    for a, s in zip(GOLD["amax"][:500], GOLD["scale_f32_e5m2"][:500]):
        assert oq.per_tensor_scale(np.array([a], np.float32), "f32", ofp8.E5M2) == s


def test_per_tensor_scale_bf16_rounds_in_bf16():
    for a, s, inv in zip(GOLD["amax_bf16"], GOLD["scale_bf16"], GOLD["inv_bf16"]):
        sc = oq.per_tensor_scale(np.array([a], np.float32), "bf16")
        assert sc == s and np.float32(1.0) / sc == inv
    # the C1 example: X ~ N(0,1) bf16 with amax 5.25 -> 85.5 (not 85.33)
    assert oq.per_tensor_scale(np.array([5.25], np.float32), "bf16") == np.float32(85.5)


def test_to_fp8_per_tensor_special_cases():
    z = np.zeros((4, 8), np.float32)
    codes, inv, scale = oq.to_fp8_per_tensor(z)
    assert (codes == 0).all() and scale == np.float32(448.0) / np.float32(1e-12) * 0 + oq.per_tensor_scale(z, "f32")
    # the amax element maps exactly to +-448
    x = np.array([[0.5, -3.0, 1.0]], np.float32)
    codes, inv, scale = oq.to_fp8_per_tensor(x)
    assert ofp8.decode(codes, ofp8.E4M3)[0, 1] == -448.0
    # values below half the smallest subnormal flush to (signed) zero
    x = np.array([448.0, 2.0 ** -10, -(2.0 ** -10), 2.0 ** -9], np.float32)
    codes, _, _ = oq.to_fp8_per_tensor(x)
    assert list(codes) == [0x7E, 0x00, 0x80, 0x01]


# ------------------------------------------------------- dual quant (a2)
def test_dual_quant_per_tensor_invariants():
    rng = np.random.default_rng(4)
    W = (rng.standard_normal((64, 96)) * 0.02).astype(np.float32)
    ef = (rng.standard_normal((64, 96)) * 1e-5).astype(np.float32)
    hi, lo, ih, il, ef_new, res = oq.dual_quant_per_tensor(W, ef)
    w = W + ef
    # hi is the plain per-tensor cast of W + EF, lo the cast of the residual
    hi2, ih2, _ = oq.to_fp8_per_tensor(w)
    assert np.array_equal(hi, hi2) and ih == ih2
    lo2, il2, _ = oq.to_fp8_per_tensor(w - ofp8.decode(hi, ofp8.E4M3) * ih)
    assert np.array_equal(lo, lo2) and il == il2
    # error is relative to W (not W + EF) and closes the decomposition
    rec = ofp8.decode(hi, ofp8.E4M3) * ih + ofp8.decode(lo, ofp8.E4M3) * il
    assert np.allclose(rec + ef_new, W, atol=1e-9, rtol=0)
    assert not np.allclose(rec + ef_new, w, atol=1e-9, rtol=0)
    # dual FP8 beats a single FP8 cast by a wide margin
    single = ofp8.decode(hi2, ofp8.E4M3) * ih2
    assert np.abs(W - rec).mean() < np.abs(w - single).mean() / 4
    # zero EF == no EF
    a = oq.dual_quant_per_tensor(W, np.zeros_like(W))
    b = oq.dual_quant_per_tensor(W, None)
    assert all(np.array_equal(x, y) for x, y in zip(a, b))


def test_sr_candidates_per_tensor():
    rng = np.random.default_rng(5)
    x = np.clip(rng.standard_normal(20000).astype(np.float32) * 100, -448, 448)
    lo, hi, frac, exact = oq.sr_candidates_per_tensor(x)
    lo_f, hi_f = ofp8.decode(lo, ofp8.E4M3), ofp8.decode(hi, ofp8.E4M3)
    ok = ~exact & np.isfinite(hi_f)
    # x lies between the two candidates and frac is its relative position
    assert (np.minimum(lo_f, hi_f)[ok] <= x[ok]).all() and (x[ok] <= np.maximum(lo_f, hi_f)[ok]).all()
    e = lo_f + np.sign(hi_f - lo_f) * frac * np.abs(hi_f - lo_f)
    assert np.allclose(e[ok], x[ok], rtol=1e-5, atol=1e-6)


# ------------------------------------------- delayed scaling (PDDS, f4)
def test_delayed_first_call_is_the_plain_dual_quant():
    rng = np.random.default_rng(21)
    W = (rng.standard_normal((24, 40)) * 0.02).astype(np.float32)
    ef = (rng.standard_normal(W.shape) * 1e-4).astype(np.float32)
    st = oq.new_delayed_state()
    hi, lo, ih, il, ef1, val = oq.dual_quant_per_tensor_delayed(W, ef, st, "w")
    hi2, lo2, ih2, il2, ef2, _ = oq.dual_quant_per_tensor(W, ef)
    assert val and np.array_equal(hi, hi2) and np.array_equal(lo, lo2)
    assert ih == ih2 and il == il2 and np.array_equal(ef1, ef2)


def test_delayed_without_memory_is_the_plain_dual_quant_every_step():
    # decay 0 keeps only the current amax; validating every step measures
    # the residual: each step must equal the plain per-tensor dual quant
    rng = np.random.default_rng(22)
    st = oq.new_delayed_state()
    W = (rng.standard_normal((16, 32)) * 0.05).astype(np.float32)
    ef = np.zeros_like(W)
    for _ in range(4):
        hi, lo, ih, il, ef_d, val = oq.dual_quant_per_tensor_delayed(W, ef, st, "w", decay=0.0,
                                                                      interval=1)
        hi2, lo2, ih2, il2, ef_p, _ = oq.dual_quant_per_tensor(W, ef)
        assert val and np.array_equal(hi, hi2) and np.array_equal(lo, lo2)
        assert ih == ih2 and il == il2 and np.array_equal(ef_d, ef_p)
        ef = ef_d
        W = (W * np.float32(1.3) + np.float32(0.01)).astype(np.float32)


def test_delayed_ema_closed_form():
    # amax 2 then 4 with decay 0.5: the delayed amax is exactly 3, and the
    # W_hi scale is torch's reciprocal-then-product of it
    st = oq.new_delayed_state()
    W1 = np.full((4, 8), 2.0, np.float32)
    W2 = np.full((4, 8), -4.0, np.float32)
    oq.dual_quant_per_tensor_delayed(W1, None, st, "w", decay=0.5)
    assert st["amax"]["w.w_hi"] == np.float32(2.0)
    _, _, ih, il, _, val = oq.dual_quant_per_tensor_delayed(W2, None, st, "w", decay=0.5)
    assert not val and st["amax"]["w.w_hi"] == np.float32(3.0)
    scale = np.float32(np.float32(1.0) / np.float32(3.0)) * np.float32(448.0)
    assert ih == np.float32(1.0) / np.float32(scale)
    # W_lo is predicted, not measured: both residuals are 0 (amax clamps to
    # 1e-12, ratio 1e-12 / 2), so the predicted residual amax is 1.5e-12
    # where a measurement would give 1e-12
    pred = np.float32(np.float32(3.0) * np.float32(np.float32(1e-12) / np.float32(2.0)))
    scale_lo = np.float32(np.float32(1.0) / pred) * np.float32(448.0)
    assert il == np.float32(1.0) / np.float32(scale_lo)
    assert il != np.float32(1.0) / (np.float32(np.float32(1.0) / np.float32(1e-12)) * np.float32(448.0))


def test_delayed_prediction_equals_measurement_when_exact():
    # constant W with a power-of-two amax and decay 0: the ratio measured on
    # step 1 predicts step 2's residual amax exactly, so the predicted step
    # must reproduce the measured one bit for bit
    rng = np.random.default_rng(23)
    W = (rng.standard_normal((16, 64)) * 0.1).astype(np.float32)
    W[0, 0] = np.float32(0.5)
    W = np.clip(W, -0.5, 0.5)
    st = oq.new_delayed_state()
    first = oq.dual_quant_per_tensor_delayed(W, None, st, "w", decay=0.0)
    second = oq.dual_quant_per_tensor_delayed(W, None, st, "w", decay=0.0)
    assert first[5] and not second[5]
    for a, b in zip(first[:5], second[:5]):
        assert np.array_equal(np.asarray(a), np.asarray(b))


# ------------------------------------------------- NF-aware scaling (core.py:161-193)
def _stdev_exact_f32(x):
    # statistics.stdev sums the squared deviations exactly (rationals), then
    # rounds once to double and takes a double sqrt: an independent
    # implementation of the sample (unbiased) standard deviation
    import statistics

    return np.float32(statistics.stdev([float(v) for v in np.ravel(x)]))


@pytest.mark.parametrize("n", [2, 3, 17, 1000])
@pytest.mark.parametrize("shift,scale", [(0.0, 1.0), (0.0, 0.02), (100.0, 1e-3), (1.0, 1e-5)])
def test_nf_std_matches_exact_rational_stdev(n, shift, scale):
    rng = np.random.default_rng(n + int(shift))
    x = (rng.standard_normal(n) * scale + shift).astype(np.float32)
    assert oq.nf_std_f32(x) == _stdev_exact_f32(x)


@pytest.mark.parametrize("shape", [(64, 64), (257, 33), (1024, 512)])
def test_nf_std_matches_torch_std_for_zero_mean_data(shape):
    import torch

    g = torch.Generator().manual_seed(shape[0])
    t = torch.randn(shape, generator=g) * 0.02
    assert oq.nf_std_f32(t.numpy()) == np.float32(t.std().item())


def test_nf_std_closed_forms_and_degenerate_sizes():
    import warnings

    import torch

    # unbiased: var([1, 2, 3, 4]) = 5/3 (the population variance is 5/4)
    assert oq.nf_std_f32(np.array([1, 2, 3, 4], np.float32)) == np.float32(np.sqrt(5.0 / 3.0))
    assert oq.nf_std_f32(np.full(10, 0.3, np.float32)) == 0.0
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        for v in ([0.5], []):
            assert np.isnan(torch.tensor(v, dtype=torch.float32).std().item())
            assert np.isnan(oq.nf_std_f32(np.array(v, np.float32)))


@pytest.mark.parametrize("sigma", [3.0, 2.5, 1.1, 3.3])
def test_nf_target_rule(sigma):
    import torch

    rng = np.random.default_rng(5)
    # the product is torch's fp32 tensor * Python float (the factor rounded
    # to fp32 first), which for some spreads differs from rounding the
    # double product once
    seen_double_differs = False
    for i in range(40):
        x = (rng.standard_normal((16, 24)) * (0.01 + 0.001 * i)).astype(np.float32)
        std = oq.nf_std_f32(x)
        want = np.float32((sigma * torch.tensor(std, dtype=torch.float32)).item())
        assert oq.nf_target(x, sigma) == want
        seen_double_differs |= bool(want != np.float32(sigma * np.float64(std)))
    assert seen_double_differs == (sigma in (1.1, 3.3))
    # std < 1e-6 (including a constant or zero tensor) falls back to the
    # clamped amax; one element gives NaN
    assert oq.nf_target(np.full((4, 4), -0.5, np.float32), sigma) == np.float32(0.5)
    tiny = (np.float32(0.25) + rng.standard_normal(256).astype(np.float32) * np.float32(1e-7))
    assert oq.nf_std_f32(tiny) < np.float32(1e-6)
    assert oq.nf_target(tiny, sigma) == np.float32(np.max(np.abs(tiny)))
    assert oq.nf_target(np.zeros((3, 3), np.float32), sigma) == np.float32(1e-12)
    assert np.isnan(oq.nf_target(np.array([[0.3]], np.float32), sigma))


def test_nf_aware_quantisation_properties():
    # the reference's own checks (tests/test_tensor_cores.py:27-68 upstream):
    # bounded round-trip error and MSE on Gaussian data, finite near-constant
    rng = np.random.default_rng(42)
    x = rng.standard_normal((1024, 1024)).astype(np.float32)
    codes, inv, scale = oq.to_fp8_nf_aware(x)
    recon = ofp8.decode(codes, "e4m3") * inv
    assert np.abs(x - recon).mean() / np.abs(x).mean() < 0.15
    assert np.square(x - recon).mean() / np.square(x).mean() < 0.01
    # 3 sigma sits below the amax: the scale is larger than the amax rule's
    # and everything beyond 3 sigma saturates at +-448
    assert scale > oq.per_tensor_scale(x, "f32")
    beyond = np.abs(x) * scale > 448
    assert beyond.any() and np.all((codes[beyond] & 0x7F) == 0x7E)
    c, inv_c, _ = oq.to_fp8_nf_aware(np.full((64, 64), 0.5, np.float32))
    assert np.isfinite(inv_c) and np.all((c & 0x7F) == 0x7E)


def test_nf_dual_quant_composition():
    rng = np.random.default_rng(6)
    W = (rng.standard_normal((48, 80)) * 0.02).astype(np.float32)
    W[3, 5] = 0.5  # an outlier far beyond 3 sigma
    ef = (rng.standard_normal(W.shape) * 1e-4).astype(np.float32)
    hi, lo, ih, il, ef_new, res = oq.dual_quant_per_tensor(W, ef, sigma_factor=3.0)
    w = W + ef
    hi2, ih2, _ = oq.to_fp8_nf_aware(w, 3.0)
    assert np.array_equal(hi, hi2) and ih == ih2
    # the clipped outlier's excess moves into the residual, which W_lo
    # quantises with its own amax rule
    assert np.abs(res).max() == np.abs(res[3, 5]) and res[3, 5] > 0.4
    lo2, il2, _ = oq.to_fp8_per_tensor(res, "f32")
    assert np.array_equal(lo, lo2) and il == il2
    # the delayed NF branch: the first call and every memoryless step equal
    # the plain NF dual quantisation
    st = oq.new_delayed_state()
    for step in range(3):
        d = oq.dual_quant_per_tensor_delayed(W, ef, st, "w", decay=0.0, interval=1,
                                             sigma_factor=3.0)
        p = oq.dual_quant_per_tensor(W, ef, sigma_factor=3.0)
        assert d[5] and all(np.array_equal(np.asarray(a), np.asarray(b))
                            for a, b in zip(d[:5], p[:5])), f"step {step}"
        assert st["amax"]["w.w_hi"] == oq.nf_target(W + ef, 3.0)
        ef = d[4]


# ------------------------------------------------------- block quant (a4)
# ---------------------------------------------------- compute_block_scales
def test_block_scales_bf16_log2_rounding_over_every_bf16_quotient():
    """torch's bf16 ``exp2(ceil(log2(q)))`` for all 32639 positive finite
    bf16 q: the oracle's fp32 log2 rounded to bf16 reproduces it (a log2
    kept in fp32 would not: just above an integer it differs)."""
    q = GOLD_BS["q_bf16"]
    mine = oq.compute_block_scales(q.reshape(-1, 1), 1, 1.0, "bf16").ravel()
    keep = q >= np.float32(1.0018652574217413e-12)  # above the clamp
    assert np.array_equal(mine[keep], GOLD_BS["pow2_bf16"][keep])
    # the fp32 rule disagrees with the bf16 one on many of these
    f32 = np.exp2(np.ceil(np.log2(q[keep].astype(np.float64)))).astype(np.float32)
    assert np.sum(f32 != GOLD_BS["pow2_bf16"][keep]) > 1000


@pytest.mark.parametrize("dt", ["f32", "bf16"])
@pytest.mark.parametrize("bs", [16, 32, 64, 128])
@pytest.mark.parametrize("fm", [448.0, 57344.0])
def test_block_scales_match_torch_formula(dt, bs, fm):
    """The reference's compute_block_scales op sequence on torch CPU (zero,
    below-clamp, NaN and inf blocks included) equals the oracle."""
    x = GOLD_BS[f"x_{dt}"]
    ref = GOLD_BS[f"s_{dt}_{bs}_{int(fm)}"]
    mine = oq.compute_block_scales(x, bs, fm, dt)
    assert mine.shape == ref.shape == (x.shape[0], x.shape[1] // bs)
    assert np.array_equal(mine, ref, equal_nan=True)
    # powers of two (or 0 / inf / NaN) that bring each block under fp8_max:
    # within fp32's log2 rounding margin, or under 2x fp8_max in bf16, whose
    # 8-bit log2 can round a quotient just above 2^k down to k (the
    # reference's own test allows that factor, tests/test_core.py:101-108)
    fin = np.isfinite(ref) & (ref > 0)
    m, e = np.frexp(ref[fin])
    assert np.all(m == 0.5)
    amax = np.abs(x.reshape(x.shape[0], -1, bs)).max(-1)[fin]
    bound = fm * (1 + 2 ** -17) if dt == "f32" else 2 * fm
    assert np.all(amax / ref[fin] <= bound)

@pytest.mark.parametrize("bs", [32, 64, 128])
def test_block_quantize_exponent_and_codes(bs):
    import torch

    rng = np.random.default_rng(6 + bs)
    x = (rng.standard_normal((16, 4 * bs)) * 2.0 ** rng.integers(-20, 20, (16, 1))).astype(np.float32)
    codes, exps = oq.block_quantize(x, bs)
    assert exps.shape == (4, 16) and exps.dtype == np.int8
    # exponent: torch's ceil(log2(amax / 448)) on the block amax
    amax = torch.from_numpy(np.abs(x).reshape(16, 4, bs).max(-1)).clamp(min=1e-12)
    e_t = torch.clamp(torch.ceil(torch.log2(amax / 448.0)), min=-126).to(torch.int8).numpy()
    assert np.array_equal(exps.T, e_t)
    # codes: brute-force nearest-even of x / 2^e
    scaled = x.reshape(16, 4, bs) / (2.0 ** exps.T.astype(np.float64))[..., None]
    assert np.array_equal(codes.ravel(), _brute_nearest_even(np.clip(scaled, -448, 448).astype(np.float32).ravel(), ofp8.E4M3))


def test_block_quantize_zero_and_e5m2():
    codes, exps = oq.block_quantize(np.zeros((3, 64), np.float32), 32)
    assert (codes == 0).all() and (exps == -48).all()  # ceil(log2(1e-12/448)) = -48
    x = np.full((2, 32), 2.0 ** 20, np.float32)  # amax/57344 = 18.3 -> e = 5
    c, e = oq.block_quantize(x, 32, ofp8.E5M2)
    assert (e == 5).all()
    assert np.all(ofp8.decode(c, ofp8.E5M2) * 2.0 ** e.T.repeat(32, 1).astype(np.float64) == 2.0 ** 20)


# ----------------------------------------------- block dual quant (a3)
@pytest.mark.parametrize("bs", [32, 64, 128])
def test_block_dual_equals_separate_block_quantize(bs):
    # the reference's bitwise fused-vs-separate test (test_fused_dual_quant.py:79-155)
    rng = np.random.default_rng(7)
    w = rng.standard_normal((32, 2 * bs)).astype(np.float32)
    ef = (rng.standard_normal(w.shape) * 1e-3).astype(np.float32)
    hi, lo, eh, el, ef_new = oq.block_dual_quantize(w, bs, ef)
    wc = w + ef
    hi2, eh2 = oq.block_quantize(wc, bs)
    assert np.array_equal(hi, hi2) and np.array_equal(eh, eh2)
    res = wc - oq.block_dequantize(hi2, eh2, bs)
    lo2, el2 = oq.block_quantize(res, bs)
    assert np.array_equal(lo, lo2) and np.array_equal(el, el2)
    expect = w - (oq.block_dequantize(hi, eh, bs) + oq.block_dequantize(lo, el, bs))
    assert np.allclose(ef_new, expect, atol=1e-5, rtol=1e-5)


def test_block_dual_zero_residual_sentinel():
    w = np.zeros((4, 64), np.float32)
    w[1] = 1.0  # exactly representable: residual is zero
    hi, lo, eh, el, _ = oq.block_dual_quantize(w, 32)
    assert (el == -128).all() and (lo == 0).all()
    assert ((el >= -126) | (el == -128)).all()


@pytest.mark.parametrize("bs", [32, 64, 128])
def test_block_requant_t_exact_when_representable_and_bounded(bs):
    rng = np.random.default_rng(bs)
    # small integers are exact in E4M3 under both blockings: re-blocking
    # returns the transposed values exactly, with zero residual blocks
    v = rng.integers(-15, 16, size=(2 * bs, 3 * bs)).astype(np.float32)
    hi, lo, eh, el, _ = oq.block_dual_quantize(v, bs)
    ht, lt, eht, elt = oq.block_requant_t(hi, lo, eh, el, bs)
    assert ht.shape == (3 * bs, 2 * bs) and eht.shape == (2, 3 * bs)
    assert np.array_equal(oq.block_dequantize(ht, eht, bs), v.T) and (elt == -128).all()
    # general weights: the result approximates deq(W)^T to within a second
    # dual-FP8 rounding, |err| <= 2^-7 of the block's maximum
    w = (rng.standard_normal((4 * bs, 2 * bs)) * 0.02).astype(np.float32)
    hi, lo, eh, el, _ = oq.block_dual_quantize(w, bs)
    v = (oq.block_dequantize(hi, eh, bs) + oq.block_dequantize(lo, el, bs)).T
    ht, lt, eht, elt = oq.block_requant_t(hi, lo, eh, el, bs)
    got = oq.block_dequantize(ht, eht, bs) + np.where(
        np.repeat(elt.T, bs, axis=1) == -128, 0.0, oq.block_dequantize(lt, elt, bs))
    amax = np.repeat(np.abs(v).reshape(v.shape[0], -1, bs).max(-1), bs, axis=1)
    assert np.all(np.abs(got - v) <= amax * 2.0 ** -7)
    assert not np.array_equal(ht, hi.T)  # the blocking changed the codes
    # W_hi alone (ABD)
    ht2, _, eht2, _ = oq.block_requant_t(hi, None, eh, None, bs)
    assert np.array_equal(ht2, oq.block_dual_quantize(
        np.ascontiguousarray(oq.block_dequantize(hi, eh, bs).T), bs)[0])


# ----------------------------------- fp32 (non-power-of-two) block scales
@pytest.mark.parametrize("bs", [32, 64, 128])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("fmt", [ofp8.E4M3, ofp8.E5M2])
def test_block_quantize_f32s_is_per_tensor_rule_per_block(bs, dtype, fmt):
    # each (row, K-block) must equal to_fp8_per_tensor (pinned against torch
    # above) run on that block alone
    rng = np.random.default_rng(11 + bs)
    x = (rng.standard_normal((5, 3 * bs)) * 2.0 ** rng.integers(-12, 12, (5, 3, 1)).repeat(bs, -1)
         .reshape(5, 3 * bs)).astype(np.float32)
    if dtype == "bf16":
        x = ofp8.bf16_round(x)
    x[2, :bs] = 0.0  # an all-zero block: amax clamps to 1e-12
    codes, inv = oq.block_quantize_f32s(x, bs, dtype, fmt)
    assert inv.shape == (3, 5) and inv.dtype == np.float32
    for r in range(5):
        for b in range(3):
            c, i, _ = oq.to_fp8_per_tensor(x[r, b * bs:(b + 1) * bs], dtype, fmt)
            assert np.array_equal(codes[r, b * bs:(b + 1) * bs], c), (r, b)
            assert inv[b, r] == i, (r, b)
    # and the scales are not the power-of-two exponents of the reference format
    assert not np.all(np.log2(inv) == np.round(np.log2(inv)))


@pytest.mark.parametrize("bs", [32, 128])
def test_block_dual_f32s_is_per_tensor_dual_per_block(bs):
    # codes and multipliers of every block equal the per-tensor dual quant
    # (nn/__init__.py:343-383, pinned above) of that block; the error update
    # follows the block path's (w - deq_hi) - deq_lo order
    rng = np.random.default_rng(12)
    w = rng.standard_normal((6, 2 * bs)).astype(np.float32)
    ef = (rng.standard_normal(w.shape) * 1e-3).astype(np.float32)
    w[3, :bs] = 0.5  # exact in E4M3: zero residual block
    ef[3, :bs] = 0.0
    hi, lo, ih, il, ef_new = oq.block_dual_quantize_f32s(w, bs, ef)
    for r in range(6):
        for b in range(2):
            sl = slice(b * bs, (b + 1) * bs)
            h2, l2, ih2, il2, ef2, _ = oq.dual_quant_per_tensor(w[r, sl], ef[r, sl])
            assert np.array_equal(hi[r, sl], h2) and np.array_equal(lo[r, sl], l2), (r, b)
            assert ih[b, r] == ih2 and il[b, r] == il2, (r, b)
            # same quantity, other rounding order: within an ulp of |w|
            assert np.allclose(ef_new[r, sl], ef2, rtol=0, atol=2.0 ** -22), (r, b)
    assert (lo[3, :bs] == 0).all()
    deq = oq.block_dequantize_f32s(hi, ih, bs) + oq.block_dequantize_f32s(lo, il, bs)
    assert np.abs(ef_new - (w - deq)).max() <= 2.0 ** -22


def test_block_gemm_f32s_reduces_to_exponent_gemm():
    # with power-of-two multipliers the fp32-scale GEMM is the reference
    # format's block GEMM (kernels.py:1939-2028)
    rng = np.random.default_rng(13)
    bs = 32
    a, ea = oq.block_quantize(rng.standard_normal((8, 4 * bs)).astype(np.float32), bs)
    w = rng.standard_normal((6, 4 * bs)).astype(np.float32)
    hi, lo, eh, el, _ = oq.block_dual_quantize(w, bs)
    assert (el != -128).all()
    got = og.block_dual_gemm_f32s_nt(a, np.exp2(ea.astype(np.float32)), hi, lo,
                                     np.exp2(eh.astype(np.float32)), np.exp2(el.astype(np.float32)), bs)
    ref = og.block_dual_gemm_nt(a, ea, hi, lo, eh, el, bs)
    assert np.allclose(got, ref, rtol=1e-12, atol=0)


# ------------------------------------------------------- GEMM oracle
def test_dual_gemm_oracle_closed_forms():
    rng = np.random.default_rng(8)
    a = rng.integers(0, 256, (8, 32)).astype(np.uint8)
    a[(a & 0x7F) == 0x7F] = 0  # no NaN codes
    hi = rng.integers(0, 256, (5, 32)).astype(np.uint8)
    hi[(hi & 0x7F) == 0x7F] = 1
    lo = np.zeros_like(hi)
    out = og.dual_gemm_nt(a, ofp8.E4M3, hi, lo, 0.5, 2.0, 3.0)
    A = ofp8.decode(a, ofp8.E4M3).astype(np.float64)
    B = ofp8.decode(hi, ofp8.E4M3).astype(np.float64)
    brute = np.array([[sum(A[i, k] * B[j, k] for k in range(32)) for j in range(5)] for i in range(8)])
    assert np.allclose(out, brute, rtol=1e-12, atol=0)
    # linear in each scale
    assert np.allclose(og.dual_gemm_nt(a, ofp8.E4M3, lo, hi, 0.5, 2.0, 3.0), 1.5 * brute)


def test_torch_ref_step_matches_numpy_oracle():
    """oracle/torch_ref.py (the torch restatement used for the training-loss
    parity test) against the numpy oracle on CPU: codes, EF, forward, and
    the three backward products."""
    import torch

    from oracle import torch_ref as tr

    g = torch.Generator().manual_seed(5)
    x = torch.randn(48, 64, generator=g).bfloat16()
    W = torch.randn(32, 64, generator=g) * 0.05
    b = torch.randn(32, generator=g)
    ef = {}
    xr = x.clone().requires_grad_(True)
    Wr = W.clone().requires_grad_(True)
    out = tr.RefTCFP12Function.apply(xr, Wr, b, ef, "", True)
    gout = torch.randn(48, 32, generator=g)
    out.backward(gout)
    hi, lo, ih, il, ef_new, _ = oq.dual_quant_per_tensor(W.numpy(), np.zeros((32, 64), np.float32))
    assert np.array_equal(ef[""].numpy(), ef_new)
    aq, ai, _ = oq.to_fp8_per_tensor(x.float().numpy(), "bf16")
    ref = og.dual_gemm_nt(aq, ofp8.E4M3, hi, lo, ai, ih, il) + b.double().numpy()
    assert og.rel_fro(out.detach().numpy(), ref) < 1e-6
    gq, gi, _ = oq.to_fp8_per_tensor(gout.numpy(), "f32", ofp8.E5M2)
    G = ofp8.decode(gq, ofp8.E5M2).astype(np.float64) * gi
    Wd = ofp8.decode(hi, ofp8.E4M3).astype(np.float64) * ih + ofp8.decode(lo, ofp8.E4M3).astype(np.float64) * il
    assert og.rel_fro(xr.grad.float().numpy(), G @ Wd) < 1e-2  # dX returned in bf16
    A = ofp8.decode(aq, ofp8.E4M3).astype(np.float64) * ai
    assert og.rel_fro(Wr.grad.numpy(), G.T @ A) < 1e-6


def test_torch_ref_block_step_matches_numpy_oracle():
    """oracle/torch_ref.py's block-scaled restatement (the TinyGPT loss
    parity reference) against the numpy oracle on CPU: codes, exponents,
    the sentinel, EF, forward and the three backward products."""
    import torch

    from oracle import torch_ref as tr

    g = torch.Generator().manual_seed(6)
    x = torch.randn(2, 48, 128, generator=g)
    W = torch.randn(64, 128, generator=g) * 0.05
    W[:, :64] = torch.round(W[:, :64] * 64) / 64  # exactly representable: zero residual blocks
    b = torch.randn(64, generator=g)
    ef = {}
    xr = x.clone().requires_grad_(True)
    Wr = W.clone().requires_grad_(True)
    out = tr.RefBlockTCFP12Function.apply(xr, Wr, b, ef, "", True, 64)
    gout = torch.randn(2, 48, 64, generator=g)
    out.backward(gout)
    hi, lo, e_hi, e_lo, ef_new = oq.block_dual_quantize(W.numpy(), 64, np.zeros((64, 128), np.float32))
    assert (e_lo == -128).any() and (e_lo != -128).any()
    assert np.array_equal(ef[""].numpy(), ef_new)
    # (+ the zero error buffer: -0.0 + 0.0 is +0.0, as in the kernels)
    q_hi, s_hi = tr.block_quant(W + torch.zeros_like(W), 64, 448.0, torch.float8_e4m3fn)
    assert np.array_equal(q_hi.view(torch.uint8).numpy(), hi)
    assert np.array_equal(s_hi.numpy(), e_hi)
    aq, ae = oq.block_quantize(x.reshape(-1, 128).numpy(), 64)
    ref = og.block_dual_gemm_nt(aq, ae, hi, lo, e_hi, e_lo, 64) + b.double().numpy()
    assert og.rel_fro(out.detach().reshape(-1, 64).numpy(), ref) < 1e-6
    gq, ge = oq.block_quantize(gout.reshape(-1, 64).numpy(), 64, ofp8.E5M2)
    dx = og.block_dgrad(gq, ge, hi, lo, e_hi, e_lo, 64)
    assert og.rel_fro(xr.grad.reshape(-1, 128).numpy(), dx) < 1e-6
    A = og.block_deq64(aq, ae, 64)
    dw = gout.reshape(-1, 64).double().numpy().T @ A
    assert og.rel_fro(Wr.grad.numpy(), dw) < 1e-6


# ------------------------------------------------------------ column sums
def _big_and_ones(rows, cols, ones):
    """2^24 at row 0 of every column; column i has +1 at the rows ones[i]."""
    x = np.zeros((rows, cols), np.float32)
    x[0] = 2.0**24
    for c, rs in enumerate(ones):
        x[list(rs), c] = 1.0
    return x


def test_column_sums_within_group_tree():
    """Adding +1 to 2^24 is lost, +2 is kept: which ones survive tells the
    order.  Halving folds pair rows l, l + 32 first, then l, l + 16, ...:
    ones at rows 1 and 33 meet each other first (kept, +2) while ones at 32
    and 48 each meet the 2^24 chain alone (lost).  Row-sequential and
    adjacent-pair orders give the opposite answers."""
    x = _big_and_ones(64, 5, [(32, 48), (1, 33), range(1, 64), (2, 3), (16, 48)])
    got = oq.column_sums(x).astype(np.float64) - 2.0**24
    # (2, 3): fold 1 is the last, both lost; (16, 48): paired at fold 32 (+2)
    assert got.tolist() == [0.0, 2.0, 62.0, 0.0, 2.0]


def test_column_sums_finalising_order():
    """Group sums: 2^24 in group 0, ones in groups (16, 24) meet in lane 0's
    second pair (kept), ones in groups (8, 16) meet 2^24 in the first pair
    and ones in groups (1, 9) sit in lane 1, added to lane 0's total last."""
    g = 40
    x = np.zeros((64 * g, 3), np.float32)
    x[0] = 2.0**24
    for c, gs in enumerate([(16, 24), (8, 16), (1, 9)]):
        for q in gs:
            x[64 * q, c] = 1.0
    got = oq.column_sums(x).astype(np.float64) - 2.0**24
    assert got.tolist() == [2.0, 0.0, 2.0]


@pytest.mark.parametrize("shape", [(1, 8), (63, 16), (64, 8), (65, 24), (1000, 24), (4096, 8)])
def test_column_sums_close_to_exact_and_exact_on_integers(shape):
    rng = np.random.default_rng(shape[0])
    x = rng.standard_normal(shape).astype(np.float32)
    ref = x.astype(np.float64).sum(0)
    bound = np.abs(x).astype(np.float64).sum(0) * 2.0**-24 * (np.log2(shape[0]) + 10)
    assert np.all(np.abs(oq.column_sums(x) - ref) <= bound)
    xi = rng.integers(-1000, 1000, shape).astype(np.float32)  # every partial exact
    assert np.array_equal(oq.column_sums(xi), xi.astype(np.float64).sum(0).astype(np.float32))


def test_lo_threshold_exps_rule():
    """Closed cases of the reference's W_lo sparsity rule
    (tcfp/kernels.py:766-776): a tile of 64 rows is dropped for a K-block
    only when its largest scale is <= the threshold; the sentinel counts as
    scale 0; a threshold below every scale drops nothing."""
    from oracle import gemm as og

    e = np.full((2, 130), -10, dtype=np.int8)
    e[0, 70] = -5          # tile 1 (rows 64..127) of block 0 holds one larger scale
    e[1, :64] = -128       # tile 0 of block 1: all sentinel
    out = og.lo_threshold_exps(e, 2.0 ** -8)
    assert (out[0, :64] == -128).all()            # tile 0, block 0: max 2^-10 <= 2^-8
    assert (out[0, 64:128] == e[0, 64:128]).all() # kept: 2^-5 > 2^-8
    assert (out[0, 128:] == -128).all()           # the partial last tile
    assert (out[1] == -128).all()
    assert np.array_equal(og.lo_threshold_exps(e, 2.0 ** -20), e)
    assert (og.lo_threshold_exps(e, 1.0) == -128).all()
    # equality counts as dropped (max(scale) <= threshold)
    assert (og.lo_threshold_exps(np.full((1, 64), -3, np.int8), 0.125) == -128).all()
