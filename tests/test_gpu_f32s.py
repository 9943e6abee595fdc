"""GPU parity of the fp32 (non-power-of-two) block-scale path.

The reference quantises blocks only with power-of-two int8 exponents; the
fp32 variant applies ``to_fp8_e4m3``'s per-tensor rule to every block
(scale = FP8_MAX / amax, not a power of two) and the block GEMMs take the
fp32 dequantisation multipliers.  Quantisation is held bit-exact to the
oracle (codes, multipliers, error buffer); the GEMMs to relative Frobenius
error EXACT = 1e-4 against the float64 dequant matmul of the same operands
(the contract is 1e-2; an indexing or scaling slip gives errors of order 1).
"""
import numpy as np
import pytest
import torch

from oracle import fp8 as ofp8
from oracle import gemm as og
from oracle import quant as oq
from tcfp_amd import kernels as K

pytestmark = pytest.mark.gpu
EXACT = 1e-4


def u8(t):
    return t.view(torch.uint8).cpu().numpy()


def npy(t):
    return t.cpu().numpy()


def _input(shape, seed, bs, dtype):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(shape, generator=g)
    # per-block magnitudes over many binades, one all-zero block
    x *= torch.exp2(torch.randint(-14, 14, (shape[0], shape[1] // bs, 1), generator=g).float()
                    ).repeat_interleave(bs, -1).reshape(shape)
    x[min(1, shape[0] - 1), :bs] = 0.0
    return x.to(dtype)


@pytest.mark.parametrize("bs", [32, 64, 128])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("fp8", [torch.float8_e4m3fn, torch.float8_e5m2])
@pytest.mark.parametrize("shape", [(300, 384), (64, 128), (7, 1024)])
def test_block_quantize_f32s_bit_exact(dev, bs, dtype, fp8, shape):
    if shape[1] % bs:
        pytest.skip("K not a multiple of the block")
    x = _input(shape, sum(shape) + bs, bs, dtype)
    q, inv = K.block_quantize_fp8(x.to(dev), bs, fp8, scale_format="fp32")
    assert inv.dtype == torch.float32 and tuple(inv.shape) == (shape[1] // bs, shape[0])
    fmt = ofp8.E5M2 if fp8 == torch.float8_e5m2 else ofp8.E4M3
    codes, inv_ref = oq.block_quantize_f32s(x.float().numpy(), bs,
                                            "bf16" if dtype == torch.bfloat16 else "f32", fmt)
    assert np.array_equal(u8(q), codes)
    assert np.array_equal(npy(inv).view(np.uint32), inv_ref.view(np.uint32))
    deq = K.block_dequantize_fp8(q, inv, bs)
    assert np.array_equal(npy(deq), oq.block_dequantize_f32s(codes, inv_ref, bs, fmt))


@pytest.mark.parametrize("bs", [32, 64, 128])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_block_dual_quantize_f32s_with_ef_bit_exact(dev, bs, dtype):
    N, K_ = 200, 4 * bs
    g = torch.Generator().manual_seed(bs)
    W = (torch.randn(N, K_, generator=g) * 0.02).to(dtype)
    W[5, :bs] = 0.25  # exact in E4M3: zero residual block (no sentinel here)
    ef = torch.randn(N, K_, generator=g) * 1e-4
    ef[5, :bs] = 0.0
    ef_dev = ef.to(dev)
    h, l, sh, sl = K.fused_dual_quantize_fp8(W.to(dev), bs, error_buf=ef_dev, scale_format="fp32")
    hi, lo, ih, il, ef_new = oq.block_dual_quantize_f32s(W.float().numpy(), bs, ef.numpy())
    assert np.array_equal(u8(h), hi) and np.array_equal(u8(l), lo)
    assert np.array_equal(npy(sh), ih) and np.array_equal(npy(sl), il)
    assert np.array_equal(npy(ef_dev).view(np.uint32), ef_new.view(np.uint32))
    assert (lo[5, :bs] == 0).all()
    # no EF: the plain dual
    h2, l2, sh2, sl2 = K.fused_dual_quantize_fp8(W.to(dev), bs, scale_format="fp32")
    hi2, lo2, ih2, il2, _ = oq.block_dual_quantize_f32s(W.float().numpy(), bs)
    assert np.array_equal(u8(h2), hi2) and np.array_equal(u8(l2), lo2)
    assert np.array_equal(npy(sh2), ih2) and np.array_equal(npy(sl2), il2)


def test_block_dual_quantize_f32s_stochastic_lo(dev):
    bs = 64
    W = torch.randn(64, 256, generator=torch.Generator().manual_seed(3)) * 0.05
    hi, lo_rtn, ih, il, _ = oq.block_dual_quantize_f32s(W.numpy(), bs)
    # the scaled residual the SR draw rounds
    wb = W.numpy().reshape(64, 4, bs)
    r = (wb - oq.block_dequantize_f32s(hi, ih, bs).reshape(64, 4, bs)).astype(np.float32)
    amax = np.abs(r).max(-1)
    scale = oq.block_scale_f32(amax)
    x = np.clip(r * scale[..., None], -448, 448).astype(np.float32).reshape(64, 256)
    rtn, other, frac, exact = oq.sr_candidates_block(x)
    assert np.array_equal(rtn, lo_rtn)
    hits = np.zeros(x.shape)
    n = 64
    for i in range(n):
        h, l, sh, sl = K.fused_dual_quantize_fp8(W.to(dev), bs, stochastic_lo=True, seed=5 + i,
                                                 scale_format="fp32")
        assert np.array_equal(u8(h), hi) and np.array_equal(npy(sl), il)
        c = u8(l)
        assert np.all((c == rtn) | (c == other)) and np.all(c[exact] == rtn[exact])
        hits += (c == other) & (other != rtn)
    m = ~exact & (other != rtn)
    assert abs(float((hits[m] / n - frac[m]).mean())) < 0.02


def _operands(M, N, K_, bs, dev, seed, act_fp8=torch.float8_e4m3fn):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, K_, generator=g)
    x[: max(1, M // 7)] *= 300.0
    w = torch.randn(N, K_, generator=g) * 0.02
    w[:, :bs] *= 1e-3
    a, sa = K.block_quantize_fp8(x.to(dev), bs, act_fp8, scale_format="fp32")
    h, l, sh, sl = K.fused_dual_quantize_fp8(w.to(dev), bs, scale_format="fp32")
    return a, sa, h, l, sh, sl


F32S_SHAPES = [(64, 128, 64), (256, 512, 256), (300, 256, 1000), (48, 128, 112),
               (1024, 1024, 1024), (36, 384, 72), (520, 640, 136), (128, 192, 64)]


@pytest.mark.parametrize("bs", [32, 64, 128])
@pytest.mark.parametrize("M,K_,N", F32S_SHAPES)
def test_block_dual_gemm_f32s_matches_oracle(dev, bs, M, K_, N):
    if K_ % bs:
        pytest.skip("K not a multiple of the block")
    a, sa, h, l, sh, sl = _operands(M, N, K_, bs, dev, M + N + bs)
    out = K.fused_block_scaled_dual_gemm_forward(a, h, l, sa, sh, sl, bs)
    assert out.dtype == torch.float32 and out.shape == (M, N)
    ref = og.block_dual_gemm_f32s_nt(u8(a), npy(sa), u8(h), u8(l), npy(sh), npy(sl), bs)
    err = og.rel_fro(npy(out), ref)
    print(f"f32s dual bs={bs} M={M} K={K_} N={N} rel_fro={err:.2e}", flush=True)
    assert err < EXACT


@pytest.mark.parametrize("bs", [32, 64, 128])
@pytest.mark.parametrize("fp8", [torch.float8_e4m3fn, torch.float8_e5m2])
@pytest.mark.parametrize("M,K_,N", [(256, 256, 256), (300, 384, 1000), (64, 128, 48)])
def test_block_scaled_single_gemm_f32s(dev, bs, fp8, M, K_, N):
    g = torch.Generator().manual_seed(M + bs)
    a, sa = K.block_quantize_fp8(torch.randn(M, K_, generator=g).to(dev), bs, fp8,
                                 scale_format="fp32")
    b, sb = K.block_quantize_fp8(torch.randn(N, K_, generator=g).to(dev), bs,
                                 scale_format="fp32")
    out = K.block_scaled_gemm(a, b, sa, sb, bs)
    afmt = ofp8.E5M2 if fp8 == torch.float8_e5m2 else ofp8.E4M3
    ref = og.block_dual_gemm_f32s_nt(u8(a), npy(sa), u8(b), None, npy(sb), None, bs, afmt)
    err = og.rel_fro(npy(out), ref)
    print(f"f32s single bs={bs} {fp8} M={M} K={K_} N={N} rel_fro={err:.2e}", flush=True)
    assert err < EXACT


def test_block_dual_gemm_f32s_bf16_out_and_bias(dev):
    M, N, K_, bs = 384, 512, 512, 32
    a, sa, h, l, sh, sl = _operands(M, N, K_, bs, dev, 7)
    bias = torch.randn(N, generator=torch.Generator().manual_seed(1)).to(dev)
    ref = og.block_dual_gemm_f32s_nt(u8(a), npy(sa), u8(h), u8(l), npy(sh), npy(sl), bs)
    ref = ref + npy(bias).astype(np.float64)
    out = K.fused_block_scaled_dual_gemm_forward(a, h, l, sa, sh, sl, bs, bias=bias)
    assert og.rel_fro(npy(out), ref) < EXACT
    ob = K.fused_block_scaled_dual_gemm_forward(a, h, l, sa, sh, sl, bs, bias=bias,
                                                out_dtype=torch.bfloat16)
    assert ob.dtype == torch.bfloat16
    assert og.rel_fro(ob.float().cpu().numpy(), ref) < 1e-2


def test_block_gemm_f32s_rejects_mixed_and_ragged(dev):
    a, sa, h, l, sh, sl = _operands(64, 64, 128, 32, dev, 1)
    _, _, eh, el = K.fused_dual_quantize_fp8(torch.randn(64, 128).to(dev), 32)
    with pytest.raises(TypeError):
        K.fused_block_scaled_dual_gemm_forward(a, h, l, sa, eh, el, 32)
    # the fp32-scale kernel loads multipliers in groups of four rows
    a6, sa6 = K.block_quantize_fp8(torch.randn(66, 128).to(dev), 32, scale_format="fp32")
    with pytest.raises(RuntimeError):
        K.fused_block_scaled_dual_gemm_forward(a6, h, l, sa6, sh, sl, 32)


@pytest.mark.parametrize("bs", [32, 64, 128])
def test_c3_4096_cubed_fp32_scales_against_torch_fp32(dev, bs):
    """The C3 configuration at full size: 4096^3 with fp32 448/amax block
    scales, against torch's fp32 matmul of the dequantised operands."""
    M = N = K_ = 4096
    g = torch.Generator(device=dev).manual_seed(bs)
    x = torch.randn(M, K_, device=dev, generator=g, dtype=torch.bfloat16)
    w = torch.randn(N, K_, device=dev, generator=g, dtype=torch.bfloat16)
    a, sa = K.block_quantize_fp8(x, bs, scale_format="fp32")
    h, l, sh, sl = K.fused_dual_quantize_fp8(w, bs, scale_format="fp32")
    out = K.fused_block_scaled_dual_gemm_forward(a, h, l, sa, sh, sl, bs)
    A = K.block_dequantize_fp8(a, sa, bs)
    W = K.block_dequantize_fp8(h, sh, bs) + K.block_dequantize_fp8(l, sl, bs)
    ref = A @ W.t()
    err = (torch.linalg.norm(out - ref) / torch.linalg.norm(ref)).item()
    print(f"C3 f32s bs={bs} rel_fro vs fp32 matmul {err:.2e}", flush=True)
    assert err < EXACT
