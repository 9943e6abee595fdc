"""GPU parity of the quantisation kernels against the numpy oracle.

Codes, exponents, scales and error buffers must be bit-identical
(integer/byte work); stochastic rounding is checked statistically, as the
reference does (tests/test_fused_dual_quant.py:467-526 upstream).
"""
import numpy as np
import pytest
import torch

from oracle import fp8 as ofp8
from oracle import quant as oq
from tcfp_amd import _hip
from tcfp_amd import kernels as K
from tcfp_amd.core import to_fp8_e4m3, to_fp8_e5m2

pytestmark = pytest.mark.gpu


def u8(t):
    return t.view(torch.uint8).cpu().numpy()


def i8(t):
    return t.cpu().numpy()


# ------------------------------------------------------------ self tests
@pytest.mark.parametrize("fmt,top", [(0, 0x43E00000), (1, 0x47600000)])
def test_hw_fp8_convert_matches_software_exhaustively(dev, fmt, top):
    # every float32 in [0, FP8_MAX] and its negation through both encoders,
    # and all 256 codes through both decoders
    bad = torch.zeros(1, dtype=torch.int64, device=dev)
    _hip.check(_hip.lib().tcfp_selftest_fp8_cvt(0, top, fmt, bad.data_ptr(),
                                                 _hip.stream_of(dev)), "selftest")
    torch.cuda.synchronize()
    assert bad.item() == 0


@pytest.mark.parametrize("u", [0.0, 0.25, 0.5, 0.70710678, 1.0 - 2.0 ** -16])
def test_sr_block_hardware_converts_match_software(dev, u):
    # the block SR rule on hardware converts (scalar and the packed four-value
    # form the kernels use) == on software converts, for every float32 in
    # [0, 448] and its negation, at the draw u truncated to k * 2^-16
    bad = torch.zeros(1, dtype=torch.int64, device=dev)
    _hip.check(_hip.lib().tcfp_selftest_sr_block(0, 0x43E00000, u, bad.data_ptr(),
                                                 _hip.stream_of(dev)), "selftest")
    torch.cuda.synchronize()
    assert bad.item() == 0


def test_philox_known_answers(dev):
    # Random123 known-answer vectors for philox4x32-10
    cases = [
        ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
        ((0xFFFFFFFF,) * 4, (0xFFFFFFFF,) * 2, (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
        ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
         (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
    ]
    for ctr, key, want in cases:
        out = torch.zeros(4, dtype=torch.int32, device=dev)
        _hip.check(_hip.lib().tcfp_selftest_philox(*ctr, *key, 1, out.data_ptr(),
                                                    _hip.stream_of(dev)), "philox")
        got = tuple(int(v) & 0xFFFFFFFF for v in out.cpu().tolist())
        assert got == want


# ------------------------------------------------------- per-tensor (a1/a8)
SHAPES = [(1, 1), (3, 5), (64, 128), (257, 1000), (8192, 1024)]


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("fp8", [torch.float8_e4m3fn, torch.float8_e5m2])
def test_per_tensor_quant_bitexact(dev, shape, dtype, fp8):
    g = torch.Generator().manual_seed(shape[0] * 131 + shape[1] + (dtype == torch.bfloat16) * 7
                                      + (fp8 == torch.float8_e5m2) * 13)
    x = (torch.randn(shape, generator=g) * 3.0).to(dtype)
    fmt = ofp8.E4M3 if fp8 == torch.float8_e4m3fn else ofp8.E5M2
    codes, inv, scale = oq.to_fp8_per_tensor(x.float().numpy(),
                                             "bf16" if dtype == torch.bfloat16 else "f32", fmt)
    q, inv_d, qt, s_d = K.quantize_per_tensor(x.to(dev), fp8, transpose=True, return_scale=True)
    assert q.dtype == fp8 and tuple(q.shape) == shape
    assert np.array_equal(u8(q), codes)
    assert np.array_equal(u8(qt), codes.T)
    assert inv_d.item() == float(inv) and s_d.item() == float(scale)
    # core API: same result without the transposed copy
    q2, inv2 = (to_fp8_e4m3 if fmt == ofp8.E4M3 else to_fp8_e5m2)(x.to(dev))
    assert np.array_equal(u8(q2), codes) and inv2.shape == (1,)


def test_per_tensor_quant_special_inputs(dev):
    x = torch.zeros(16, 32)
    x[3, 7] = 1e-30  # tiny amax -> scale 448/1e-30
    q, inv = to_fp8_e4m3(x.to(dev))
    codes, inv_o, _ = oq.to_fp8_per_tensor(x.numpy())
    assert np.array_equal(u8(q), codes) and inv.item() == float(inv_o)
    z = torch.zeros(5, 8, device=dev)
    q, inv = to_fp8_e4m3(z)
    assert (u8(q) == 0).all() and inv.item() == float(np.float32(1) / oq.per_tensor_scale(np.zeros(1, np.float32), "f32"))
    big = torch.tensor([[3.0e38, -1.0, 2.0 ** -140]], device=dev)
    q, inv = to_fp8_e4m3(big)
    codes, inv_o, _ = oq.to_fp8_per_tensor(big.cpu().numpy())
    assert np.array_equal(u8(q), codes) and inv.item() == float(inv_o)


def test_per_tensor_explicit_scale(dev):
    x = torch.randn(33, 65)
    s = torch.tensor([7.5])
    q, inv = to_fp8_e4m3(x.to(dev), scale=s.to(dev))
    codes, inv_o, _ = oq.to_fp8_per_tensor(x.numpy(), scale=np.float32(7.5))
    assert np.array_equal(u8(q), codes) and inv.item() == float(inv_o)


def test_per_tensor_empty(dev):
    q, inv = to_fp8_e4m3(torch.empty(0, 16, device=dev))
    assert q.shape == (0, 16)


def test_per_tensor_quant_beyond_int32_elements(dev):
    # 2^31 + 32768 bf16 elements (4.3 GB): element offsets past 2^31 must
    # be addressed with 64-bit arithmetic in the amax, flat and transposing
    # passes.  The tensor's maximum sits in its last element, so a wrapped
    # index would lose it; codes are checked against the oracle on rows at
    # the start, across the 2^31 boundary and at the end.
    rows, cols = 65537, 32768
    print(f"per-tensor quant {rows}x{cols} bf16", flush=True)
    g = torch.Generator(device=dev).manual_seed(21)
    x = torch.randn(rows, cols, generator=g, device=dev, dtype=torch.bfloat16)
    x[-1, -1] = 1000.0
    q, inv, qt, s = K.quantize_per_tensor(x, transpose=True, return_scale=True)
    scale = oq.per_tensor_scale(np.array([1000.0], np.float32), "bf16")
    assert s.item() == float(scale) and inv.item() == float(np.float32(1) / scale)
    for r0 in (0, 40000, rows - 2):
        xs = x[r0:r0 + 2].float().cpu().numpy()
        codes, _, _ = oq.to_fp8_per_tensor(xs, "bf16", scale=scale)
        assert np.array_equal(u8(q[r0:r0 + 2]), codes), r0
        assert np.array_equal(u8(qt[:, r0:r0 + 2]), codes.T), r0
    # the flat pass (no transposed copy) writes the same codes
    q2, inv2 = K.quantize_per_tensor(x)
    assert torch.equal(q2.view(torch.uint8), q.view(torch.uint8)) and torch.equal(inv2, inv)
    del x, q, qt, q2
    torch.cuda.empty_cache()


def test_per_tensor_transposed_copy_of_tall_ragged_tensor(dev):
    # cols % 8 != 0 takes the flat pass and the 64 x 64 byte transpose;
    # 4194400 rows are more 64-row tiles than a grid's y dimension holds
    rows, cols = 4194400, 5
    g = torch.Generator().manual_seed(23)
    x = torch.randn(rows, cols, generator=g).bfloat16()
    codes, inv_o, _ = oq.to_fp8_per_tensor(x.float().numpy(), "bf16")
    q, inv, qt = K.quantize_per_tensor(x.to(dev), transpose=True)
    assert np.array_equal(u8(q), codes) and inv.item() == float(inv_o)
    assert np.array_equal(u8(qt), codes.T)


def test_workspace_contents_do_not_matter(dev):
    """The partial-maximum slots of the reduction workspace are scratch:
    whatever they hold before a call (here all-ones bytes) changes no output.
    (The grid-barrier counters after them must stay zero at rest.)"""
    ws = _hip.workspace(dev)
    x = torch.randn(300, 200, generator=torch.Generator().manual_seed(5)).to(dev)
    w = torch.randn(64, 64, generator=torch.Generator().manual_seed(6)).to(dev)
    ref_q = to_fp8_e4m3(x)
    ref_d = K.dual_quantize_per_tensor(w, torch.zeros(64, 64, device=dev))
    ws[:8192].fill_(255)
    q = to_fp8_e4m3(x)
    d = K.dual_quantize_per_tensor(w, torch.zeros(64, 64, device=dev))
    assert torch.equal(q[0].view(torch.uint8), ref_q[0].view(torch.uint8))
    assert torch.equal(q[1], ref_q[1])
    for a, b in zip(d, ref_d):
        assert torch.equal(a.view(torch.uint8) if a.dtype.itemsize == 1 else a,
                           b.view(torch.uint8) if b.dtype.itemsize == 1 else b)


# ---------------------------------------------------- dual quant (a2)
@pytest.mark.parametrize("shape", [(64, 128), (100, 200), (4096, 1024), (1024, 4096)])
@pytest.mark.parametrize("wdtype", [torch.float32, torch.bfloat16])
def test_dual_quant_per_tensor_ef_steps_bitexact(dev, shape, wdtype):
    g = torch.Generator().manual_seed(11)
    W = (torch.randn(shape, generator=g) * 0.02).to(wdtype)
    ef_o = np.zeros(shape, np.float32)
    ef_d = torch.zeros(shape, device=dev)
    Wd = W.to(dev)
    for step in range(3):
        hi, lo, ih, il, ef_new, _ = oq.dual_quant_per_tensor(W.float().numpy(), ef_o)
        h, l, ihd, ild, ht, lt = K.dual_quantize_per_tensor(Wd, ef_d, transposed=True)
        assert np.array_equal(u8(h), hi), f"step {step} hi"
        assert np.array_equal(u8(l), lo), f"step {step} lo"
        assert np.array_equal(u8(ht), hi.T) and np.array_equal(u8(lt), lo.T)
        assert ihd.item() == float(ih) and ild.item() == float(il)
        assert np.array_equal(ef_d.cpu().numpy(), ef_new), f"step {step} ef"
        ef_o = ef_new
        # the "optimizer" moves W a little between steps
        W = (W.float() + 1e-4 * torch.randn(shape, generator=g)).to(wdtype)
        Wd = W.to(dev)


def _cand_case(name, shape, g):
    w = torch.randn(shape, generator=g) * 0.02
    if name == "overflow":       # every |v| near the max: all are candidates
        w = torch.sign(w) * (1.0 + 1e-3 * torch.rand(shape, generator=g))
    elif name == "exact":        # E4M3-representable: every residual is zero
        codes = torch.randint(0, 126, shape, generator=g, dtype=torch.uint8)
        w = codes.view(torch.float8_e4m3fn).float() * 2.0 ** -7
    elif name == "outlier":      # one value far above the rest
        w[3, 5] = 1e4
    elif name == "nan":
        w[7, 11] = float("nan")
    elif name == "inf":
        w[2, 9] = float("inf")
    elif name == "zerohead":     # a zero first quarter (zero-initialised rows)
        w[: shape[0] // 4] = 0.0
    return w


@pytest.mark.parametrize("name", ["normal", "overflow", "exact", "outlier", "nan", "inf",
                                  "zerohead"])
@pytest.mark.parametrize("shape,wdtype", [((4096, 2048), torch.float32),
                                          ((2049, 4097), torch.float32),
                                          ((4096, 2048), torch.bfloat16)])
def test_dual_quant_candidate_pass_matches_full_pass(dev, name, shape, wdtype):
    """The candidate residual pass (tensors of 2^23+ elements) against the
    full residual pass on the same inputs, bit for bit: codes, both inverse
    scales, the transposed codes and the EF update, on data where the
    candidates decide (normal) and where the full pass must run (a region
    overflows, every residual is zero, one outlier, NaN, inf); and against
    the oracle on the finite cases."""
    g = torch.Generator().manual_seed(len(name) + shape[1])
    w = _cand_case(name, shape, g).to(wdtype).to(dev)
    ef0 = (torch.randn(shape, generator=g) * 1e-4).to(dev)
    outs = []
    try:
        for on in (True, False):
            K.set_dual_quant_candidates(on)
            ef = ef0.clone()
            res = K.dual_quantize_per_tensor(w, ef, transposed=True)
            outs.append([r.view(torch.uint8) if r.dtype.itemsize == 1 else r for r in res] + [ef])
    finally:
        K.set_dual_quant_candidates(True)
    for x, y in zip(*outs):
        assert torch.equal(x.nan_to_num(), y.nan_to_num()) and torch.equal(x.isnan(), y.isnan())
    if name in ("nan", "inf"):
        return
    hi, lo, ih, il, ef_new, _ = oq.dual_quant_per_tensor(w.float().cpu().numpy(),
                                                         ef0.cpu().numpy())
    h, l, ihd, ild, ht, lt, efd = outs[0]
    assert np.array_equal(h.cpu().numpy(), hi) and np.array_equal(l.cpu().numpy(), lo)
    assert ihd.item() == float(ih) and ild.item() == float(il)
    assert np.array_equal(efd.cpu().numpy(), ef_new)


@pytest.mark.parametrize("wdtype", [torch.float32, torch.bfloat16])
def test_dual_quant_candidate_pass_without_ef(dev, wdtype):
    """The candidate residual pass with no error-feedback buffer (2^23+
    elements): the full pass's codes and scales, and the oracle's."""
    g = torch.Generator().manual_seed(17)
    w = (torch.randn(4096, 2048, generator=g) * 0.02).to(wdtype).to(dev)
    outs = []
    try:
        for on in (True, False):
            K.set_dual_quant_candidates(on)
            outs.append([r.view(torch.uint8) if r.dtype.itemsize == 1 else r
                         for r in K.dual_quantize_per_tensor(w, None)])
    finally:
        K.set_dual_quant_candidates(True)
    for x, y in zip(*outs):
        assert torch.equal(x, y)
    hi, lo, ih, il, _, _ = oq.dual_quant_per_tensor(w.float().cpu().numpy(), None)
    h, l, ihd, ild = outs[0]
    assert np.array_equal(h.cpu().numpy(), hi) and np.array_equal(l.cpu().numpy(), lo)
    assert ihd.item() == float(ih) and ild.item() == float(il)


@pytest.mark.parametrize("wdtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("transposed", [False, True])
def test_dual_quant_no_update_leaves_ef(dev, wdtype, transposed):
    W = (torch.randn(64, 64, device=dev) * 0.02).to(wdtype)
    ef = torch.randn(64, 64, device=dev) * 1e-4
    before = ef.clone()
    a = K.dual_quantize_per_tensor(W, ef, update_ef=False, transposed=transposed)
    assert torch.equal(ef, before)
    b = K.dual_quantize_per_tensor(W, before.clone(), update_ef=True, transposed=transposed)
    assert all(torch.equal(x.view(torch.uint8) if x.dtype.itemsize == 1 else x,
                           y.view(torch.uint8) if y.dtype.itemsize == 1 else y)
               for x, y in zip(a, b))


@pytest.mark.parametrize("wdtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("transposed", [False, True])
def test_dual_quant_no_ef_matches_zero_ef(dev, wdtype, transposed):
    W = torch.randn(96, 160, device=dev).to(wdtype)
    a = K.dual_quantize_per_tensor(W, None, transposed=transposed)
    b = K.dual_quantize_per_tensor(W, torch.zeros(96, 160, device=dev), transposed=transposed)
    for x, y in zip(a, b):
        assert torch.equal(x.view(torch.uint8) if x.dtype.itemsize == 1 else x,
                           y.view(torch.uint8) if y.dtype.itemsize == 1 else y)


@pytest.mark.parametrize("wdtype", [torch.float32, torch.bfloat16])
def test_dual_quant_sr_candidates_and_unbiased(dev, wdtype):
    g = torch.Generator().manual_seed(3)
    W = torch.randn(128, 256, generator=g).to(wdtype)
    hi_o, lo_rtn, ih_o, il_o, _, res = oq.dual_quant_per_tensor(W.float().numpy(), None)
    scale_lo = oq.per_tensor_scale(res, "f32")
    x = np.clip(res * scale_lo, -448, 448).astype(np.float32)
    lo_c, hi_c, frac, exact = oq.sr_candidates_per_tensor(x)
    acc = np.zeros(x.shape, np.float64)
    n = 200
    for i in range(n):
        h, l, ih, il = K.dual_quantize_per_tensor(W.to(dev), None, stochastic_lo=True, seed=1000 + i)
        assert np.array_equal(u8(h), hi_o) and il.item() == float(il_o)
        c = u8(l)
        assert np.all((c == lo_c) | (c == hi_c)), "SR picked a code outside the candidate pair"
        assert np.all(c[exact] == lo_c[exact])
        acc += (c == hi_c) & (hi_c != lo_c)
    p = acc / n
    m = ~exact & (hi_c != lo_c) & np.isfinite(frac)
    # empirical up-rounding rate tracks frac (binomial noise, n = 200)
    assert abs(float((p[m] - frac[m]).mean())) < 0.01
    assert float(np.abs(p[m] - frac[m]).max()) < 0.2


@pytest.mark.parametrize("wdtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("update", [True, False])
@pytest.mark.parametrize("transposed", [False, True])
def test_dual_quant_sr_with_error_feedback(dev, wdtype, update, transposed):
    """Stochastic W_lo with an error-feedback buffer: the reference's
    Function allows both (nn/__init__.py:363-383; its layer never enables
    both).  W_hi, the scales and the candidate pair follow W + ef, and the
    new error is W - (deq(hi) + deq(lo)) of the codes drawn."""
    g = torch.Generator().manual_seed(5)
    W = torch.randn(128, 256, generator=g).to(wdtype)
    ef0 = torch.randn(128, 256, generator=g) * 1e-3
    Wf = W.float().numpy()
    hi_o, _, ih_o, il_o, _, res = oq.dual_quant_per_tensor(Wf, ef0.numpy())
    scale_lo = oq.per_tensor_scale(res, "f32")
    x = np.clip(res * scale_lo, -448, 448).astype(np.float32)
    lo_c, hi_c, frac, exact = oq.sr_candidates_per_tensor(x)
    ef = ef0.clone().to(dev)
    out = K.dual_quantize_per_tensor(W.to(dev), ef, update_ef=update, stochastic_lo=True,
                                     seed=77, transposed=transposed)
    h, l, ih, il = out[:4]
    assert np.array_equal(u8(h), hi_o)
    assert ih.item() == float(ih_o) and il.item() == float(il_o)
    c = u8(l)
    assert np.all((c == lo_c) | (c == hi_c)), "SR picked a code outside the candidate pair"
    assert np.all(c[exact] == lo_c[exact])
    assert 0 < int((c != lo_c).sum()) < c.size
    if transposed:
        assert np.array_equal(u8(out[4]), hi_o.T) and np.array_equal(u8(out[5]), c.T)
    if update:
        deq_hi = ofp8.decode(hi_o, ofp8.E4M3).astype(np.float32) * np.float32(ih_o)
        deq_lo = ofp8.decode(c, ofp8.E4M3).astype(np.float32) * np.float32(il_o)
        assert np.array_equal(ef.cpu().numpy(), Wf - (deq_hi + deq_lo))
    else:
        assert torch.equal(ef.cpu(), ef0)


# ------------------------------------------------------ block quant (a4)
@pytest.mark.parametrize("bs", [32, 64, 128])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("fp8", [torch.float8_e4m3fn, torch.float8_e5m2])
@pytest.mark.parametrize("m", [1, 37, 512])
def test_block_quantize_bitexact(dev, bs, dtype, fp8, m):
    g = torch.Generator().manual_seed(bs * 7 + m)
    k = 4 * bs
    x = (torch.randn(m, k, generator=g) * 2.0 ** torch.randint(-20, 20, (m, 1), generator=g)).to(dtype)
    fmt = ofp8.E4M3 if fp8 == torch.float8_e4m3fn else ofp8.E5M2
    codes, exps = oq.block_quantize(x.float().numpy(), bs, fmt)
    q, e = K.block_quantize_fp8(x.to(dev), bs, fp8)
    assert tuple(e.shape) == (k // bs, m) and e.dtype == torch.int8
    assert np.array_equal(i8(e), exps)
    assert np.array_equal(u8(q), codes)


def test_block_quantize_zero_and_boundary(dev):
    x = torch.zeros(4, 64)
    x[1, :32] = 448.0 * 2.0 ** -10 * (1 + 2.0 ** -23)  # amax/448 just above 2^-10
    x[2, 32:] = 448.0 * 2.0 ** -10
    codes, exps = oq.block_quantize(x.numpy(), 32)
    q, e = K.block_quantize_fp8(x.to(dev), 32)
    assert np.array_equal(i8(e), exps) and np.array_equal(u8(q), codes)


@pytest.mark.parametrize("bs", [32, 64, 128])
def test_block_dequantize(dev, bs):
    x = torch.randn(40, 2 * bs)
    q, e = K.block_quantize_fp8(x.to(dev), bs)
    d = K.block_dequantize_fp8(q, e, bs).cpu().numpy()
    assert np.array_equal(d, oq.block_dequantize(u8(q), i8(e), bs))


# ------------------------------------------------- block dual quant (a3)
@pytest.mark.parametrize("bs", [32, 64, 128])
@pytest.mark.parametrize("wdtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [(64, 256), (200, 512), (4096, 1024)])
def test_block_dual_quantize_ef_bitexact(dev, bs, wdtype, shape):
    g = torch.Generator().manual_seed(bs + shape[0])
    W = torch.randn(shape, generator=g).to(wdtype)
    ef_o = (np.random.default_rng(bs).standard_normal(shape) * 1e-3).astype(np.float32)
    ef_d = torch.from_numpy(ef_o.copy()).to(dev)
    for step in range(2):
        hi, lo, eh, el, ef_new = oq.block_dual_quantize(W.float().numpy(), bs, ef_o)
        h, l, sh, sl = K.fused_dual_quantize_fp8(W.to(dev), bs, error_buf=ef_d)
        assert np.array_equal(u8(h), hi) and np.array_equal(u8(l), lo)
        assert np.array_equal(i8(sh), eh) and np.array_equal(i8(sl), el)
        assert np.array_equal(ef_d.cpu().numpy(), ef_new), f"step {step}"
        ef_o = ef_new
    # update_ef=False: the same codes from W + ef, the buffer untouched
    hi, lo, eh, el, _ = oq.block_dual_quantize(W.float().numpy(), bs, ef_o)
    h, l, sh, sl = K.fused_dual_quantize_fp8(W.to(dev), bs, error_buf=ef_d, update_ef=False)
    assert np.array_equal(u8(h), hi) and np.array_equal(u8(l), lo)
    assert np.array_equal(i8(sh), eh) and np.array_equal(i8(sl), el)
    assert np.array_equal(ef_d.cpu().numpy(), ef_o)


def test_block_dual_quantize_sentinel_and_no_ef(dev):
    W = torch.zeros(8, 64)
    W[2] = 1.0
    W[5, :32] = torch.randn(32)
    hi, lo, eh, el, _ = oq.block_dual_quantize(W.numpy(), 32)
    h, l, sh, sl = K.fused_dual_quantize_fp8(W.to(dev), 32)
    assert np.array_equal(i8(sl), el) and (i8(sl)[:, 2] == -128).all()
    assert np.array_equal(u8(h), hi) and np.array_equal(u8(l), lo)


@pytest.mark.parametrize("bs", [32, 64, 128])
@pytest.mark.parametrize("wdt", [torch.float32, torch.bfloat16])
def test_block_dual_quantize_sr(dev, bs, wdt):
    # fp32 weights run 8 elements per lane (one Philox call), bf16 weights 16
    # (two calls); the segment spans 2..16 lanes across the block sizes
    g = torch.Generator().manual_seed(9)
    W = torch.randn(64, 256, generator=g).to(wdt)
    Wf = W.float().numpy()
    nb = 256 // bs
    hi, lo_rtn, eh, el, _ = oq.block_dual_quantize(Wf, bs)
    wb = Wf.reshape(64, nb, bs)
    deq_hi = oq.block_dequantize(hi, eh, bs).reshape(64, nb, bs)
    r = (wb - deq_hi).astype(np.float32)
    x = np.clip(r * (2.0 ** -el.T.astype(np.float64))[..., None], -448, 448).astype(np.float32).reshape(64, 256)
    rtn, other, frac, exact = oq.sr_candidates_block(x)
    assert np.array_equal(rtn, lo_rtn)
    acc = np.zeros(x.shape)
    n = 200
    for i in range(n):
        h, l, sh, sl = K.fused_dual_quantize_fp8(W.to(dev), bs, stochastic_lo=True, seed=77 + i)
        assert np.array_equal(u8(h), hi) and np.array_equal(i8(sl), el)
        c = u8(l)
        assert np.all((c == rtn) | (c == other))
        assert np.all(c[exact] == rtn[exact])
        acc += (c == other) & (other != rtn)
    m = ~exact & (other != rtn)
    assert m.sum() > 0
    # unbiased (E[deq(lo)] = residual): the count of round-ups over all
    # inexact elements matches the sum of their probabilities within 5
    # binomial standard deviations (bf16 weights leave few inexact residuals,
    # so the bound scales with how many there are), and no element strays far
    f = frac[m].astype(np.float64)
    z = (acc[m].sum() - n * f.sum()) / np.sqrt(max(n * (f * (1 - f)).sum(), 1e-12))
    assert abs(z) < 5, (int(m.sum()), z)
    assert float(np.abs(acc[m] / n - f).max()) < 0.2


# ------------------- block quantisers on inputs of 64 MB and more (work order)
@pytest.mark.parametrize("shape,dtype,bs,fp8", [
    ((4100, 4160), torch.float32, 64, torch.float8_e4m3fn),
    ((8192, 4096), torch.bfloat16, 32, torch.float8_e5m2)])
def test_block_quantize_large_input_bitexact(dev, shape, dtype, bs, fp8):
    """From 64 MB of input the block quantisers run K-blocks fastest in
    XCD-contiguous runs (4100 x 4160 fp32: an odd workgroup count and a
    partial row group; bf16 at block 32: 64-byte row pieces).  Codes and
    exponents stay the oracle's bit for bit."""
    g = torch.Generator().manual_seed(shape[0] + bs)
    x = (torch.randn(shape, generator=g) *
         2.0 ** torch.randint(-8, 8, (shape[0], 1), generator=g)).to(dtype)
    assert x.numel() * x.element_size() >= 64 << 20
    fmt = ofp8.E4M3 if fp8 == torch.float8_e4m3fn else ofp8.E5M2
    codes, exps = oq.block_quantize(x.float().numpy(), bs, fmt)
    q, e = K.block_quantize_fp8(x.to(dev), bs, fp8)
    assert np.array_equal(i8(e), exps)
    assert np.array_equal(u8(q), codes)


def test_block_dual_quantize_large_input_ef_bitexact(dev):
    """Block-64 dual quantisation with EF of a 64 MB weight (the K-fastest
    order): codes, exponents and the new EF equal the oracle's."""
    g = torch.Generator().manual_seed(5)
    W = torch.randn(4096, 4096, generator=g) * 0.02
    ef_o = (np.random.default_rng(5).standard_normal((4096, 4096)) * 1e-4).astype(np.float32)
    ef_d = torch.from_numpy(ef_o.copy()).to(dev)
    hi, lo, eh, el, ef_new = oq.block_dual_quantize(W.numpy(), 64, ef_o)
    h, l, sh, sl = K.fused_dual_quantize_fp8(W.to(dev), 64, error_buf=ef_d)
    assert np.array_equal(u8(h), hi) and np.array_equal(u8(l), lo)
    assert np.array_equal(i8(sh), eh) and np.array_equal(i8(sl), el)
    assert np.array_equal(ef_d.cpu().numpy(), ef_new)


@pytest.mark.parametrize("bs", [32, 64, 128])
@pytest.mark.parametrize("wdtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("fmt", ["exponent", "fp32"])
def test_block_dual_quantize_large_input_no_update(dev, bs, wdtype, fmt):
    """update_ef=False on a 64 MB weight (the K-fastest order), with either
    scale format: the codes and scales of the updating call, the buffer
    untouched.  With fp32 multipliers, SRR keeps W_hi and both scale arrays
    of the round-to-nearest call and changes only some W_lo codes."""
    print(f"block dq large no-update bs={bs} {wdtype} {fmt}", flush=True)
    rows = 4096 if wdtype == torch.float32 else 8192
    g = torch.Generator().manual_seed(bs)
    W = (torch.randn(rows, 4096, generator=g) * 0.02).to(wdtype).to(dev)
    ef = torch.randn(rows, 4096, generator=g).mul_(1e-4).to(dev)
    keep = ef.clone()
    a = K.fused_dual_quantize_fp8(W, bs, error_buf=ef, update_ef=False, scale_format=fmt)
    assert torch.equal(ef, keep)
    b = K.fused_dual_quantize_fp8(W, bs, error_buf=keep, update_ef=True, scale_format=fmt)
    assert not torch.equal(ef, keep)
    for x, y in zip(a, b):
        assert torch.equal(x.view(torch.uint8), y.view(torch.uint8))
    if fmt == "fp32":
        rne = K.fused_dual_quantize_fp8(W, bs, scale_format=fmt)
        sr = K.fused_dual_quantize_fp8(W, bs, stochastic_lo=True, seed=9, scale_format=fmt)
        for i in (0, 2, 3):
            assert torch.equal(sr[i].view(torch.uint8), rne[i].view(torch.uint8)), i
        moved = (sr[1].view(torch.uint8) != rne[1].view(torch.uint8)).float().mean().item()
        assert 0.0 < moved < 0.75, moved


def test_block_dual_quantize_large_input_sr(dev):
    """SRR on a 64 MB weight (the K-fastest order): W_hi and both exponent
    arrays equal the oracle's, and every W_lo code is one of the two
    stochastic-rounding candidates (the nearest where the residual is exact)."""
    g = torch.Generator().manual_seed(6)
    W = torch.randn(4096, 4096, generator=g) * 0.02
    Wf = W.numpy()
    bs, nb = 64, 4096 // 64
    hi, lo_rtn, eh, el, _ = oq.block_dual_quantize(Wf, bs)
    h, l, sh, sl = K.fused_dual_quantize_fp8(W.to(dev), bs, stochastic_lo=True, seed=11)
    assert np.array_equal(u8(h), hi)
    assert np.array_equal(i8(sh), eh) and np.array_equal(i8(sl), el)
    deq_hi = oq.block_dequantize(hi, eh, bs).reshape(4096, nb, bs)
    r = (Wf.reshape(4096, nb, bs) - deq_hi).astype(np.float32)
    x = np.clip(r * (2.0 ** -el.T.astype(np.float64))[..., None], -448, 448)
    rtn, other, frac, exact = oq.sr_candidates_block(x.astype(np.float32).reshape(4096, 4096))
    c = u8(l)
    assert np.all((c == rtn) | (c == other))
    assert np.all(c[exact] == rtn[exact])
    assert ((c == other) & (other != rtn)).any()


# ------------------------------------------------ quant + column sums (bias grad)
@pytest.mark.parametrize("shape", [(8192, 1024), (300, 200), (7, 4096), (1000, 24), (0, 64)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_quantize_colsum_codes_and_sums(dev, shape, dtype):
    g = torch.Generator().manual_seed(shape[0] + shape[1])
    x = (torch.randn(shape, generator=g) * 1e-3).to(dtype)
    q, inv, qt, cs = K.quantize_per_tensor_colsum(x.to(dev), torch.float8_e5m2, transpose=True)
    if shape[0] == 0:
        assert torch.equal(cs.cpu(), torch.zeros(shape[1]))
        return
    codes, inv_o, _ = oq.to_fp8_per_tensor(x.float().numpy(), "bf16" if dtype == torch.bfloat16
                                           else "f32", ofp8.E5M2)
    assert np.array_equal(u8(q), codes) and np.array_equal(u8(qt), codes.T)
    assert inv.item() == float(inv_o)
    ref = x.double().sum(0).numpy()
    np.testing.assert_allclose(cs.cpu().numpy(), ref, rtol=1e-5, atol=1e-6 * float(np.abs(x.float().numpy()).sum(0).max()))
    # bit for bit in the fixed order (restated in oracle.quant.column_sums)
    assert np.array_equal(cs.cpu().numpy(), oq.column_sums(x.float().numpy()))


# ---------------------------------------- delayed scaling (PDDS) dual quant
@pytest.mark.parametrize("wdt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("transposed", [False, True])
@pytest.mark.parametrize("shape", [(256, 512), (300, 200), (64, 4096), (33, 1000)])
def test_delayed_dual_quant_matches_oracle_over_steps(dev, wdt, transposed, shape):
    from tcfp_amd.core import ErrorFeedbackState

    state = ErrorFeedbackState(ema_decay=0.9, residual_validation_interval=3)
    ost = oq.new_delayed_state()
    g = torch.Generator().manual_seed(sum(shape))
    W = torch.randn(shape, generator=g) * 0.02
    ef_dev = torch.zeros(shape, device=dev)
    ef_np = np.zeros(shape, np.float32)
    for step in range(7):
        Wd = W.to(wdt)
        res = K.dual_quantize_per_tensor_delayed(Wd.to(dev), ef_dev, state, "lin",
                                                 transposed=transposed)
        hi, lo, ih, il, ef_new, val = oq.dual_quant_per_tensor_delayed(
            Wd.float().numpy(), ef_np, ost, "lin", decay=0.9, interval=3)
        tag = f"step {step} validated={val}"
        assert np.array_equal(u8(res[0]), hi), tag
        assert np.array_equal(u8(res[1]), lo), tag
        assert res[2].item() == float(ih) and res[3].item() == float(il), tag
        assert np.array_equal(ef_dev.cpu().numpy().view(np.uint32), ef_new.view(np.uint32)), tag
        assert state._delayed_amax["lin.w_hi"].item() == float(ost["amax"]["lin.w_hi"]), tag
        assert state._residual_ratio["lin.ratio"].item() == float(ost["ratio"]["lin.ratio"]), tag
        if transposed:
            assert np.array_equal(u8(res[4]), hi.T) and np.array_equal(u8(res[5]), lo.T), tag
        ef_np = ef_new
        W = W + torch.randn(shape, generator=g) * 0.004


# ------------------------------------------------------------ edge cases
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_nan_propagates_like_torch(dev, dtype):
    # the reference's amax is NaN-propagating (|t|.max() keeps NaN, clamp
    # keeps NaN), so one NaN makes the scale and every code NaN
    x = torch.randn(64, 96).to(dtype)
    x[7, 11] = float("nan")
    q, inv = to_fp8_e4m3(x.to(dev))
    assert torch.isnan(inv).all()
    codes = u8(q)
    assert np.all((codes & 0x7F) == 0x7F)
    h, l, ih, il = K.dual_quantize_per_tensor(x.float().to(dev))
    assert torch.isnan(ih).all() and np.all((u8(h) & 0x7F) == 0x7F)


def test_per_tensor_dual_quant_empty_and_one_element(dev):
    h, l, ih, il = K.dual_quantize_per_tensor(torch.empty(0, 8, device=dev))
    assert h.shape == (0, 8) and l.shape == (0, 8)
    w = torch.tensor([[0.3]], device=dev)
    h, l, ih, il = K.dual_quantize_per_tensor(w)
    hi, lo, ih2, il2, _, _ = oq.dual_quant_per_tensor(np.array([[0.3]], np.float32))
    assert np.array_equal(u8(h), hi) and np.array_equal(u8(l), lo)
    assert ih.item() == float(ih2) and il.item() == float(il2)


@pytest.mark.parametrize("case", ["mlp", "mixed", "big", "fallback"])
def test_quantize_batch_equals_single_calls(dev, case):
    """tcfp_quantize_batch (three launches for every tensor of the batch)
    against the single-tensor entry points on the same inputs, bit for bit:
    codes, transposed codes, inverse scales and updated EF buffers.  Cases:
    the C4 MLP's two weights and input; fp32 / bf16 weights with and
    without EF, update off, ragged rows, E5M2 activations; a 2^23-element
    weight (the single call takes the candidate pass); a last dimension not
    divisible by 8 (the batch hands it to the single calls)."""
    g = torch.Generator().manual_seed(len(case))
    if case == "mlp":
        shapes = [((4096, 1024), torch.float32, True, True, False),
                  ((1024, 4096), torch.float32, True, True, True)]
        acts = [((8192, 1024), torch.bfloat16, torch.float8_e4m3fn, True)]
    elif case == "mixed":
        shapes = [((300, 200), torch.bfloat16, True, False, True),
                  ((384, 96), torch.float32, False, False, False),
                  ((130, 1000), torch.float32, True, True, True)]
        acts = [((333, 136), torch.float32, torch.float8_e5m2, True)]
    elif case == "big":
        shapes = [((4096, 2048), torch.float32, True, True, True)]
        acts = [((2048, 512), torch.float32, torch.float8_e5m2, False)]
    else:
        shapes = [((64, 100), torch.float32, True, True, False)]
        acts = [((32, 36), torch.float32, torch.float8_e4m3fn, True)]
    dual, efs_a, efs_b = [], [], []
    for shape, wdt, has_ef, upd, tr in shapes:
        w = (torch.randn(shape, generator=g) * 0.02).to(wdt).to(dev)
        e = (torch.randn(shape, generator=g) * 1e-4).to(dev) if has_ef else None
        efs_a.append(e.clone() if e is not None else None)
        efs_b.append(e.clone() if e is not None else None)
        dual.append((w, tr, upd))
    act = [((torch.randn(s, generator=g) * 3).to(dt).to(dev), f, tr) for s, dt, f, tr in acts]
    print(f"[batch] {case}", flush=True)
    rd, ra = K.quantize_batch(dual=[(w, e, u, t) for (w, t, u), e in zip(dual, efs_a)], act=act)
    for (w, t, u), e, r in zip(dual, efs_b, rd):
        ref = K.dual_quantize_per_tensor(w, e, update_ef=u, transposed=t)
        assert len(r) == len(ref)
        for x, y in zip(r, ref):
            x = x.view(torch.uint8) if x.dtype.itemsize == 1 else x
            y = y.view(torch.uint8) if y.dtype.itemsize == 1 else y
            assert torch.equal(x, y), (case, tuple(w.shape))
    for ea, eb in zip(efs_a, efs_b):
        if ea is not None:
            assert torch.equal(ea, eb)
    for (x, f, t), r in zip(act, ra):
        ref = K.quantize_per_tensor(x, f, transpose=t)
        for p, q in zip(r, ref):
            p = p.view(torch.uint8) if p.dtype.itemsize == 1 else p
            q = q.view(torch.uint8) if q.dtype.itemsize == 1 else q
            assert torch.equal(p, q), (case, tuple(x.shape))
