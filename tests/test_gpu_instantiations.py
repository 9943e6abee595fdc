"""Every GEMM kernel instantiation the C ABI can reach, held to a float64
matmul of the same decoded operands.

``tcfp_dual_gemm`` (per-tensor scales), ``tcfp_block_dual_gemm`` (int8
block exponents on the MFMA's E8M0 scale operands) and
``tcfp_block_dual_gemm_f32s`` (fp32 block multipliers) take any of the four
FP8 operand-format pairs (``a_fmt`` / ``b_fmt``), a dual (``b_lo``) or a
single (``b_lo == NULL``) product and fp32 or bf16 output; the dispatcher
then picks a tile path from the shape and the tile policy.  The reference
reaches every format pair: its cuBLASLt wrapper maps both FP8 dtypes of
either operand (``tcfp/csrc/fused_dual_gemm.cu:81-98``) and
``fp8_matmul`` hands both to ``torch._scaled_mm`` (``tcfp/core.py:
527-575``).  Each case below runs one instantiation -- asserted by the
kernel name the profiler records -- on random codes and checks it against
torch's float64 matmul of the decoded operands with the scales applied:
relative Frobenius error <= 1e-4 with fp32 output (fp32 accumulation;
an indexing or scaling slip gives errors of order 1), <= 3e-3 with bf16
output (one round-to-nearest-even to 8 significant bits: RMS 2^-9 / sqrt 3
= 1.1e-3).
"""

import pytest
import torch

from tcfp_amd import _hip
from tcfp_amd import kernels as K

pytestmark = pytest.mark.gpu

FMT = {0: torch.float8_e4m3fn, 1: torch.float8_e5m2}
OUT = {"f32": (0, torch.float32, "float"), "bf16": (1, torch.bfloat16, "unsigned short")}

# tile path -> (tile policy, (M, N, K), kernel-name fragment after the
# "<AF, BF, SPLIT, OutT, " prefix, or None for the persistent kernel)
SMALL = (256, 256, 512)      # a small-tile grid that fits one round
MANY = (2048, 2304, 256)     # more small tiles than CUs
BIG = (2048, 4608, 256)      # more full 256 x 128 tiles than CUs
PATHS = {
    "deep": ("auto", SMALL, "4, 128, 64, {S}, 4, "),
    "small8": ("small8", SMALL, "8, 128, 64, {S}, 4, "),
    "small2": ("small", MANY, "4, 128, 64, {S}, 2, "),
    "large": ("large_nonpersistent", SMALL, "8, 256, 128, {S}, 2, "),
    "persist": ("auto", BIG, None),
    "small": ("auto", SMALL, "4, 128, 64, {S}, 2, "),  # block scales: two stages
    # block-scaled single GEMM, fp32 output: the persistent kernel with the
    # two weight slots on adjacent 64-row blocks, or 128-row blocks where
    # there are at least as many 256 x 256 tiles as CUs
    "persist_spl": ("auto", BIG, None),
    "persist_spl128": ("auto", (4096, 4096, 256), None),
    # per-tensor dual, bf16 output: the persistent tile with four waves
    "persist4": ("large4", BIG, None),
}
# (scale kind, dual) -> the tile paths the dispatcher has for it
SCALE_PATHS = {
    ("pt", True): ["deep", "small8", "small2", "large", "persist", "persist4"],
    ("pt", False): ["deep", "small8", "small2", "large"],
    ("e8m0", True): ["small", "large", "persist"],
    ("e8m0", False): ["small", "persist_spl", "persist_spl128"],
    ("f32s", True): ["small"],
    ("f32s", False): ["small"],
}

def _cases():
    out = []
    for (kind, dual), paths in SCALE_PATHS.items():
        for path in paths:
            for od in OUT:
                if path.startswith("persist_spl") and od != "f32":
                    continue
                if path == "persist4" and od != "bf16":
                    continue
                for af in (0, 1):
                    for bf in (0, 1):
                        bss = (32, 64, 128) if kind == "f32s" else ((64,) if kind == "e8m0" else (0,))
                        for bs in bss:
                            out.append(pytest.param(
                                kind, bs, dual, path, od, af, bf,
                                id=f"{kind}{bs or ''}-{'dual' if dual else 'single'}-{path}-{od}-a{af}b{bf}"))
    return out

def _kernel_names(fn):
    from torch.profiler import ProfilerActivity, profile

    with profile(activities=[ProfilerActivity.CUDA]) as prof:
        fn()
        torch.cuda.synchronize()
    return [e.name for e in prof.events()]

def _codes(shape, fmt, scale, seed, dev):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * scale).to(FMT[fmt]).to(dev)

def _expand(s, bs, rows, k):
    """[k / bs, rows] per-block factors -> [rows, k]."""
    return s.t().repeat_interleave(bs, dim=1)[:rows, :k]

@pytest.mark.parametrize("kind,bs,dual,path,od,af,bf", _cases())
def test_gemm_instantiation_against_float64(dev, kind, bs, dual, path, od, af, bf):
    policy, (m, n, k), frag = PATHS[path]
    print(f"instantiation {kind} bs={bs} dual={dual} {path} {od} a{af} b{bf} {m}x{n}x{k}",
          flush=True)
    seed = 1000 * af + 100 * bf + 7 * bs + (3 if dual else 0) + m % 97
    a = _codes((m, k), af, 2.0, seed, dev)
    b_hi = _codes((n, k), bf, 2.0, seed + 1, dev)
    b_lo = _codes((n, k), bf, 0.05, seed + 2, dev) if dual else None
    bias = (torch.randn(n, generator=torch.Generator().manual_seed(seed + 3)) * 0.5).to(dev)
    out_code, out_dtype, out_name = OUT[od]
    out = torch.empty(m, n, dtype=out_dtype, device=dev)
    lib, st = _hip.lib(), _hip.stream_of(dev)
    P = _hip.ptr  # noqa: N806
    f64 = lambda t: t.to(torch.float64)  # noqa: E731
    gen = torch.Generator().manual_seed(seed + 4)
    if kind == "pt":
        s_a = torch.tensor([0.75], device=dev)
        s_hi = torch.tensor([0.5], device=dev)
        s_lo = torch.tensor([2.0 ** -5], device=dev)

        def run():
            return lib.tcfp_dual_gemm(P(a), af, k, P(b_hi), P(b_lo), bf, k, m, n, k, P(s_a),
                                      P(s_hi), P(s_lo), P(bias), P(out), out_code, n, st)

        ref = 0.75 * 0.5 * (f64(a) @ f64(b_hi).t())
        if dual:
            ref += 0.75 * 2.0 ** -5 * (f64(a) @ f64(b_lo).t())
        scale_id = 0
    else:
        nkb = k // bs
        if kind == "e8m0":
            e_a = torch.randint(-3, 4, (nkb, m), generator=gen, dtype=torch.int8).to(dev)
            e_hi = torch.randint(-3, 4, (nkb, n), generator=gen, dtype=torch.int8).to(dev)
            e_lo = torch.randint(-9, -4, (nkb, n), generator=gen, dtype=torch.int8).to(dev)
            fa, fh, fl = (torch.pow(2.0, f64(e)) for e in (e_a, e_hi, e_lo))

            def run():
                return lib.tcfp_block_dual_gemm(P(a), af, k, P(e_a), P(b_hi), P(b_lo), bf, k,
                                                P(e_hi), P(e_lo) if dual else None, m, n, k, bs,
                                                P(bias), P(out), out_code, n, st)

            scale_id = 1
        else:
            s_a = (torch.rand(nkb, m, generator=gen) * 1.5 + 0.5).to(dev)
            s_hi = (torch.rand(nkb, n, generator=gen) * 1.5 + 0.5).to(dev)
            s_lo = (torch.rand(nkb, n, generator=gen) * 0.01).to(dev)
            fa, fh, fl = f64(s_a), f64(s_hi), f64(s_lo)

            def run():
                return lib.tcfp_block_dual_gemm_f32s(P(a), af, k, P(s_a), P(b_hi), P(b_lo), bf,
                                                     k, P(s_hi), P(s_lo) if dual else None, m, n,
                                                     k, bs, P(bias), P(out), out_code, n, st)

            scale_id = 2
        a_s = f64(a) * _expand(fa, bs, m, k)
        ref = a_s @ (f64(b_hi) * _expand(fh, bs, n, k)).t()
        if dual:
            ref += a_s @ (f64(b_lo) * _expand(fl, bs, n, k)).t()
    ref += f64(bias)[None, :]

    split = "false" if dual else "true"
    if path == "persist_spl":
        want = f"gemm_nt_persist_kernel<{af}, {bf}, float, 0, 1, 6, 64, true>"
    elif path == "persist4":
        want = f"gemm_nt_persist_kernel<{af}, {bf}, unsigned short, 0, 0, 4, 128, false>"
    elif path == "persist_spl128":
        want = f"gemm_nt_persist_kernel<{af}, {bf}, float, 0, 1, 8, 128, true>"
    elif frag is None:
        want = f"gemm_nt_persist_kernel<{af}, {bf}, {out_name}, 0, {scale_id}, 8, 128, false>"
    else:
        want = f"gemm_nt_dma_kernel<{af}, {bf}, {split}, {out_name}, " + frag.format(S=scale_id)
        if kind == "f32s":
            want += f"{bs.bit_length() - 1}, 0>"
    try:
        K.set_gemm_tile_policy(policy)
        rc = []
        names = _kernel_names(lambda: rc.append(run()))
    finally:
        K.set_gemm_tile_policy("auto")
    assert rc == [0], rc
    assert any(want in x for x in names), (want, [x for x in names if "gemm" in x])
    err = (torch.linalg.norm(f64(out) - ref) / torch.linalg.norm(ref)).item()
    print(f"  {want}: rel_fro {err:.2e}", flush=True)
    assert err < (1e-4 if od == "f32" else 3e-3)
