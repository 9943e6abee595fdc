"""The no-allocation dual quantisation entry point against the workspace one.

``tcfp_dual_quantize_per_tensor_noalloc`` keeps its reduction partials in a
library-owned static device array instead of a caller workspace.  Both entry
points are called through the C ABI (ctypes) on the same seeded inputs, twice
in a row -- the second call on a smaller weight, so the shared array still
holds the first call's partials -- and every output (codes, transposed
codes, inverse scales, updated error buffer) must agree bit for bit.
"""
import pytest
import torch

from tcfp_amd import _hip

pytestmark = pytest.mark.gpu

E4M3 = torch.float8_e4m3fn


def _outputs(n, k, dev):
    return {
        "hi": torch.empty((n, k), dtype=E4M3, device=dev),
        "lo": torch.empty((n, k), dtype=E4M3, device=dev),
        "inv_hi": torch.empty(1, dtype=torch.float32, device=dev),
        "inv_lo": torch.empty(1, dtype=torch.float32, device=dev),
        "hi_t": torch.empty((k, n), dtype=E4M3, device=dev),
        "lo_t": torch.empty((k, n), dtype=E4M3, device=dev),
    }


def _call(noalloc, w, ef, o, stream, ws=None, srr=False):
    lib = _hip.lib()
    n, k = w.shape
    dt = _hip.DTYPE_BF16 if w.dtype == torch.bfloat16 else _hip.DTYPE_F32
    common = (
        w.data_ptr(), dt, n, k, ef.data_ptr() if ef is not None else None, 1, int(srr),
        1234, 0, o["hi"].data_ptr(), o["lo"].data_ptr(), o["inv_hi"].data_ptr(),
        o["inv_lo"].data_ptr(), o["hi_t"].data_ptr(), o["lo_t"].data_ptr(),
    )
    if noalloc:
        rc = lib.tcfp_dual_quantize_per_tensor_noalloc(*common, stream)
    else:
        rc = lib.tcfp_dual_quantize_per_tensor(*common, ws.data_ptr(), stream)
    assert rc == 0, lib.tcfp_status_string(rc)


@pytest.mark.parametrize("wdtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("mode", ["ef", "srr"])
def test_noalloc_dual_quant_matches_workspace_entry_point(wdtype, mode):
    dev = torch.device("cuda", 0)
    stream = torch.cuda.current_stream(dev).cuda_stream
    ws = torch.empty(int(_hip.lib().tcfp_workspace_bytes()), dtype=torch.uint8, device=dev)
    g = torch.Generator().manual_seed(7)
    # the first shape has 2^23 elements, so the candidate residual pass runs
    # (its counts and partials also live in the static array); the second
    # call is smaller, and its amax is far below the first's: a stale
    # partial of the first call would change its scales
    for shape, mag in (((4096, 2048), 1.0), ((300, 208), 0.01)):
        print(f"[noalloc] shape={shape} dtype={wdtype} mode={mode}", flush=True)
        W = (torch.randn(shape, generator=g) * mag).to(wdtype).to(dev)
        ef0 = (torch.randn(shape, generator=g) * 1e-3 * mag).to(dev)
        ef_a = ef0.clone() if mode == "ef" else None
        ef_b = ef0.clone() if mode == "ef" else None
        a = _outputs(*shape, dev)
        b = _outputs(*shape, dev)
        _call(False, W, ef_a, a, stream, ws=ws, srr=mode == "srr")
        _call(True, W, ef_b, b, stream, srr=mode == "srr")
        torch.cuda.synchronize()
        for key in a:
            x, y = a[key], b[key]
            if x.dtype == E4M3:
                x, y = x.view(torch.uint8), y.view(torch.uint8)
            assert torch.equal(x, y), (shape, key)
        if ef_a is not None:
            assert torch.equal(ef_a, ef_b), shape
        # the scales follow this call's amax (a stale partial of the larger
        # first call would be ~100x off); bf16 rounding of the scale allowed
        amax = (W.float() + (ef0 if mode == "ef" else 0)).abs().max().clamp(min=1e-12)
        assert float(b["inv_hi"]) == pytest.approx(float(amax) / 448.0, rel=2e-2)


def test_noalloc_call_allocates_no_device_memory():
    """After a warm-up call, further calls leave the device's free memory
    (hipMemGetInfo, through torch.cuda.mem_get_info) unchanged: the entry
    point allocates nothing, on the candidate path (2^23 elements) and the
    plain one."""
    dev = torch.device("cuda", 0)
    stream = torch.cuda.current_stream(dev).cuda_stream
    g = torch.Generator().manual_seed(11)
    for shape in ((4096, 2048), (512, 384)):
        print(f"[noalloc] allocation check shape={shape}", flush=True)
        W = torch.randn(shape, generator=g).to(dev)
        ef = torch.zeros(shape, device=dev)
        o = _outputs(*shape, dev)
        _call(True, W, ef, o, stream)
        torch.cuda.synchronize()
        free0 = torch.cuda.mem_get_info(dev)[0]
        for _ in range(3):
            _call(True, W, ef, o, stream)
        torch.cuda.synchronize()
        assert torch.cuda.mem_get_info(dev)[0] == free0, shape


def test_noalloc_rejects_a_bad_shape_before_launching():
    lib = _hip.lib()
    dev = torch.device("cuda", 0)
    stream = torch.cuda.current_stream(dev).cuda_stream
    rc = lib.tcfp_dual_quantize_per_tensor_noalloc(
        None, 0, -1, 4, None, 0, 0, 0, 0, None, None, None, None, None, None, stream)
    assert rc == 1  # TCFP_ERR_SHAPE, before anything is launched
