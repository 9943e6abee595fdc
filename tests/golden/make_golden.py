"""Writes tests/golden/torch_primitives.npz: outputs of the torch CPU
primitives that the reference's FP8 path is composed of.

The reference (bwiemz/tcfp) defines its quantisation as torch ops:
``scaled.to(torch.float8_e4m3fn)`` / ``float8_e5m2`` (tcfp/core.py:104,156),
``FP8_MAX / amax`` i.e. ``Tensor.__rtruediv__`` (core.py:101,153),
``torch.ones(1) / scale`` (core.py:105) and ``torch.ceil(torch.log2(.))``
(core.py:250, kernels.py:257).  These fixtures record what torch 2.10 (CPU)
returns for seeded inputs, so the numpy oracle is checked against torch
itself rather than against a retyped formula.

    python tests/golden/make_golden.py
"""
from pathlib import Path

import numpy as np
import torch

OUT = Path(__file__).with_name("torch_primitives.npz")
OUT_BLOCK_SCALES = Path(__file__).with_name("torch_block_scales.npz")


def main() -> None:
    rng = np.random.default_rng(20261201)
    # FP8 decode tables
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    dec_e4m3 = codes.view(torch.float8_e4m3fn).float().numpy()
    dec_e5m2 = codes.view(torch.float8_e5m2).float().numpy()
    # cast samples: random magnitudes over the whole range, plus exact
    # midpoints between adjacent codes (the round-to-even cases)
    x = np.concatenate([
        rng.standard_normal(6000).astype(np.float32) * 2.0 ** rng.integers(-12, 9, 6000),
        rng.uniform(-448, 448, 2000).astype(np.float32),
    ]).astype(np.float32)
    fin = dec_e4m3[np.isfinite(dec_e4m3)]
    fin = np.unique(fin)
    mids_e4m3 = ((fin[:-1].astype(np.float64) + fin[1:]) / 2).astype(np.float32)
    x_e4m3 = np.concatenate([x, mids_e4m3]).astype(np.float32)
    x_e4m3 = np.clip(x_e4m3, -448, 448)
    c_e4m3 = torch.from_numpy(x_e4m3).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    fin5 = np.unique(dec_e5m2[np.isfinite(dec_e5m2)])
    mids_e5m2 = ((fin5[:-1].astype(np.float64) + fin5[1:]) / 2).astype(np.float32)
    x_e5m2 = np.concatenate([x * 64, mids_e5m2]).astype(np.float32)
    x_e5m2 = np.clip(x_e5m2, -57344, 57344)
    c_e5m2 = torch.from_numpy(x_e5m2).to(torch.float8_e5m2).view(torch.uint8).numpy()
    # ceil(log2(q)) at every mantissa offset j < 40 above a power of two
    ks = np.arange(-126, 121)
    js = np.arange(0, 40)
    bits = ((ks[:, None] + 127) << 23) | js[None, :]
    q = bits.astype(np.uint32).view(np.float32).ravel()
    q = np.concatenate([q, (rng.uniform(1, 2, 4000) * 2.0 ** rng.integers(-60, 60, 4000)).astype(np.float32)])
    clog2 = torch.ceil(torch.log2(torch.from_numpy(q))).numpy().astype(np.int32)
    # per-tensor scale: 448 / amax and 1 / scale, fp32 and bf16 amax
    amax = (rng.uniform(1, 2, 3000) * 2.0 ** rng.integers(-30, 30, 3000)).astype(np.float32)
    amax = np.concatenate([amax, np.float32([0.0, 1e-12, 1e-13, 448.0, 1.0])])
    a32 = torch.from_numpy(amax).clamp(min=1e-12)
    s32 = (448.0 / a32).to(torch.float32)
    inv32 = torch.ones(1) / s32
    s32_e5 = (57344.0 / a32).to(torch.float32)
    ab = torch.from_numpy(amax).bfloat16().clamp(min=1e-12)
    sb = (448.0 / ab).to(torch.float32)
    invb = torch.ones(1) / sb
    np.savez_compressed(
        OUT,
        dec_e4m3=dec_e4m3, dec_e5m2=dec_e5m2,
        x_e4m3=x_e4m3, c_e4m3=c_e4m3, x_e5m2=x_e5m2, c_e5m2=c_e5m2,
        q=q, clog2=clog2,
        amax=amax, amax_bf16=ab.float().numpy(),
        scale_f32=s32.numpy(), inv_f32=inv32.numpy(), scale_f32_e5m2=s32_e5.numpy(),
        scale_bf16=sb.numpy(), inv_bf16=invb.numpy(),
        torch_version=np.array(torch.__version__),
    )
    print("wrote", OUT, OUT.stat().st_size, "bytes")


def _block_scales_formula(t: torch.Tensor, bs: int, fp8_max: float) -> torch.Tensor:
    """The op sequence of the reference's compute_block_scales
    (tcfp/core.py:243-251), evaluated by torch on the CPU."""
    *lead, d = t.shape
    amax = t.reshape(*lead, d // bs, bs).abs().amax(dim=-1).clamp(min=1e-12)
    return torch.exp2(torch.ceil(torch.log2(amax / fp8_max)))


def block_scales() -> None:
    """torch CPU outputs of the block-scale rule: every positive finite bf16
    quotient through bf16 log2 / ceil / exp2, and seeded fp32 / bf16 tensors
    (with zero, tiny, NaN and inf blocks) at block sizes 16..128."""
    rng = np.random.default_rng(20261202)
    bits = np.arange(1, 0x7F80, dtype=np.uint32)
    q = (bits << 16).view(np.float32)
    qb = torch.from_numpy(q.copy()).bfloat16()
    pow2_bf16 = torch.exp2(torch.ceil(torch.log2(qb))).float().numpy()
    out = {"q_bf16": q, "pow2_bf16": pow2_bf16}
    for dt in ("f32", "bf16"):
        x = (rng.standard_normal((48, 256)) * 2.0 ** rng.integers(-60, 60, (48, 1))).astype(np.float32)
        x[0] = 0.0
        x[1] = 1e-20
        x[2, 5] = np.nan
        x[3, 7] = np.inf
        t = torch.from_numpy(x)
        if dt == "bf16":
            t = t.bfloat16()
        out[f"x_{dt}"] = t.float().numpy()
        for bs in (16, 32, 64, 128):
            for fm in (448.0, 57344.0):
                out[f"s_{dt}_{bs}_{int(fm)}"] = _block_scales_formula(t, bs, fm).float().numpy()
    np.savez_compressed(OUT_BLOCK_SCALES, **out, torch_version=np.array(torch.__version__))
    print("wrote", OUT_BLOCK_SCALES, OUT_BLOCK_SCALES.stat().st_size, "bytes")


if __name__ == "__main__":
    main()
    block_scales()
