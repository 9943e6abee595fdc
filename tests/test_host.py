"""CPU tests of the host side: the C-ABI library loads and exports every
symbol include/tcfp_hip.h declares, the Python boundary validates like the
reference, and the module/state-machine logic behaves like tcfp.nn.
No kernel is launched here."""
import re
from pathlib import Path

import pytest
import torch
import torch.nn as nn

from tcfp_amd import _hip
from tcfp_amd import kernels as K
from tcfp_amd.core import ErrorFeedbackState, FP8Config, to_fp8_e4m3
from tcfp_amd.nn import TCFPLinear, convert_to_tcfp

HEADER = Path(__file__).resolve().parent.parent / "include" / "tcfp_hip.h"


def _declared():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(tcfp_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _hip.load_library()
    declared = _declared()
    assert declared, "no declarations parsed"
    missing = [s for s in declared if not hasattr(lib, s)]
    assert not missing, missing
    # and the ctypes table binds exactly the declared set
    assert sorted(_hip.exported_symbols()) == declared


def test_status_strings_and_workspace_size():
    lib = _hip.load_library()
    assert lib.tcfp_status_string(0) == b"ok"
    assert b"mutually exclusive" in lib.tcfp_status_string(6)
    assert lib.tcfp_workspace_bytes() >= 32


def test_argument_validation_without_launch():
    lib = _hip.load_library()
    # bad shapes/dtypes are rejected before any HIP call
    assert lib.tcfp_block_quantize(None, 0, 4, 48, 32, 0, None, None, None) == 1
    assert lib.tcfp_block_quantize(None, 7, 4, 64, 32, 0, None, None, None) == 2
    assert lib.tcfp_dual_gemm(None, 0, 32, None, None, 0, 32, 4, 4, 24, None, None, None, None,
                              None, 0, 4, None) == 1  # K % 16
    assert lib.tcfp_block_dual_quantize(None, 0, 4, 64, 32, 1, 1, 1, 0, 0, None, None, None,
                                        None, None) == 6  # SR + EF


def test_grid_limit_is_a_shape_error_without_launch():
    """1-D grids past HIP's 2^32-thread limit (gridDim.x * 256 threads) are
    rejected with TCFP_ERR_SHAPE before any launch (the pointers are dummies
    that are never dereferenced)."""
    lib = _hip.load_library()
    p = 4096  # any 16-byte-aligned non-null address
    limit = (2**32 - 1) // 256  # largest 256-thread grid HIP accepts
    # re-blocking: ceil(d_out / 128) * ceil(d_in / 64) workgroups
    d_out, d_in = 128 * 4096, 64 * 4096
    assert (d_out // 128) * (d_in // 64) == limit + 1
    assert lib.tcfp_block_requant_t(p, None, p, None, d_out, d_in, 64, p, p, p, p, None) == 1
    # byte transpose: ceil(rows / 64) * ceil(cols / 64) workgroups
    rows, cols = 64 * 4096, 64 * 4097
    assert (rows // 64) * (cols // 64) > limit
    assert lib.tcfp_transpose_u8(p, rows, cols, p, None) == 1


def test_cpu_tensors_fail_loudly():
    with pytest.raises(RuntimeError, match="only on the GPU"):
        to_fp8_e4m3(torch.randn(4, 4))
    with pytest.raises(RuntimeError, match="only on the GPU"):
        K.block_quantize_fp8(torch.randn(4, 64), 32)


def test_fused_dual_quantize_validation_messages():
    w = torch.randn(8, 64)
    with pytest.raises(AssertionError, match="contiguous"):
        K.fused_dual_quantize_fp8(w.t(), block_size=32)
    with pytest.raises(AssertionError, match="divisible"):
        K.fused_dual_quantize_fp8(torch.randn(8, 48), block_size=32)
    with pytest.raises(ValueError, match="mutually exclusive"):
        K.fused_dual_quantize_fp8(w, 32, error_buf=torch.zeros(8, 64), stochastic_lo=True)
    with pytest.raises(AssertionError, match="float32"):
        K.fused_dual_quantize_fp8(w, 32, error_buf=torch.zeros(8, 64, dtype=torch.float64))
    with pytest.raises(AssertionError, match="shape"):
        K.fused_dual_quantize_fp8(w, 32, error_buf=torch.zeros(8, 32))


def test_error_feedback_state():
    st = ErrorFeedbackState()
    w = torch.randn(4, 8)
    b = st.get_error("a", w)
    assert b.dtype == torch.float32 and b.shape == w.shape and (b == 0).all()
    assert st.get_error("a", w) is b
    st.update_error("a", torch.ones(4, 8, requires_grad=True))
    assert not st._buffers["a"].requires_grad
    assert st.get_error("a", torch.randn(2, 2)).shape == (2, 2)  # shape change re-inits
    st.reset()
    assert st._buffers == {}


def test_fp8_config_validation():
    with pytest.raises(ValueError):
        FP8Config(block_size=24)


def test_tcfplinear_validation_messages():
    with pytest.raises(ValueError, match="32, 64, or 128"):
        TCFPLinear(64, 64, use_tensor_cores=True, scale_block_size=16)
    with pytest.raises(ValueError, match="in_features.*divisible"):
        TCFPLinear(48, 64, use_tensor_cores=True, scale_block_size=32)
    with pytest.raises(ValueError, match="out_features.*divisible"):
        TCFPLinear(64, 48, use_tensor_cores=True, scale_block_size=32)
    with pytest.raises(NotImplementedError):
        TCFPLinear(64, 64)  # fake-quantise path is out of scope


def test_tcfplinear_state_and_srr_disables_ef():
    lin = TCFPLinear(32, 16, use_tensor_cores=True)
    assert lin._error_state is not None and lin.weight.shape == (16, 32)
    assert TCFPLinear(32, 16, use_tensor_cores=True, srr=True)._error_state is None
    assert TCFPLinear(32, 16, use_tensor_cores=True, error_feedback=False)._error_state is None
    assert "use_tensor_cores=True" in repr(lin)


def test_convert_to_tcfp_structure():
    model = nn.Sequential(
        nn.Linear(64, 128), nn.GELU(), nn.Linear(128, 64),
        nn.Sequential(nn.Linear(64, 40)),  # 40 % 16 != 0 -> stays nn.Linear
    )
    model.head = nn.Linear(64, 64)
    w0 = model[0].weight
    convert_to_tcfp(model, use_tensor_cores=True, scale_block_size=64)
    assert isinstance(model[0], TCFPLinear) and model[0].weight is w0
    assert model[0]._param_name == "0" and model[2]._param_name == "2"
    assert model[0].scale_block_size == 64
    assert type(model[3][0]) is nn.Linear
    assert type(model.head) is nn.Linear  # skip pattern
    # scale block dropped per layer when it does not divide
    m2 = convert_to_tcfp(nn.Sequential(nn.Linear(96, 64)), use_tensor_cores=True,
                         scale_block_size=64)
    assert m2[0].scale_block_size is None


def test_ef_guard_version_logic_cpu():
    # the guard reads weight._version; in-place optimizer steps bump it
    lin = TCFPLinear(32, 16, use_tensor_cores=True)
    v0 = lin.weight._version
    with torch.no_grad():
        lin.weight.add_(1.0)
    assert lin.weight._version != v0


def test_ef_state_roundtrip_reference_format(tmp_path):
    """ef_state.pt has the reference's structure (checkpointing.py:200-224)
    and restores buffers, EMA dicts, step counts and decay by layer key."""
    from tcfp_amd.ef_state import ef_state_dict, load_ef_state, save_ef_state

    def model():
        m = nn.Sequential(nn.Linear(64, 128), nn.GELU(), nn.Linear(128, 64))
        return convert_to_tcfp(m, use_tensor_cores=True)

    a = model()
    g = torch.Generator().manual_seed(0)
    for key, lin in (("0", a[0]), ("2", a[2])):
        ef = lin._error_state
        ef._buffers[key] = torch.randn(lin.weight.shape, generator=g)
        ef._amax_ema[key] = torch.rand(1, generator=g)
        ef._step_count[key] = 7
        ef._ema_decay = 0.99
    snap = ef_state_dict(a)
    assert set(snap) == {"0", "2"}
    assert set(snap["0"]) == {"_buffers", "_amax_ema", "_delayed_amax", "_residual_ratio",
                              "_step_count", "_ema_decay"}
    save_ef_state(a, tmp_path / "ef_state.pt")
    b = model()
    assert load_ef_state(b, tmp_path / "ef_state.pt") == 2
    for key, la, lb in (("0", a[0], b[0]), ("2", a[2], b[2])):
        ea, eb = la._error_state, lb._error_state
        assert torch.equal(ea._buffers[key], eb._buffers[key])
        assert torch.equal(ea._amax_ema[key], eb._amax_ema[key])
        assert eb._step_count[key] == 7 and eb._ema_decay == 0.99
    # unknown keys are skipped, as in the reference
    from tcfp_amd.ef_state import load_ef_state_dict
    assert load_ef_state_dict(b, {"nope": snap["0"]}) == 0


def test_reference_gate_functions_without_gpu():
    # the reference's dispatch gates (tcfp/nn/__init__.py:40-66) exist and
    # report the backend unusable here; the ext entry points fail loudly
    import torch

    from tcfp_amd import cuda_ext, kernels

    assert kernels.is_triton_available() is False
    assert cuda_ext.is_cuda_ext_available() is False
    z = torch.zeros(16, 16)
    s = torch.ones(1)
    with pytest.raises(RuntimeError):
        cuda_ext.cuda_ext_dual_gemm_forward(z, z, z, s, s, s)
    with pytest.raises(RuntimeError):
        cuda_ext.cuda_ext_dual_gemm_backward_dx(z, z, z, s, s, s)


def test_error_feedback_state_delayed_methods_follow_the_oracle():
    # the torch-op state transitions (reference tcfp/core.py:341-403) give
    # the same EMA values as the oracle's restatement used for the kernels
    import numpy as np

    from oracle import quant as oq

    st = ErrorFeedbackState(ema_decay=0.9, residual_validation_interval=3)
    ost = oq.new_delayed_state()
    g = torch.Generator().manual_seed(5)
    W = torch.randn(16, 32, generator=g) * 0.05
    for step in range(5):
        cur = W.abs().max().clamp(min=1e-12)
        delayed = st.get_delayed_amax("w.w_hi", cur)
        validate = st.should_validate_residual("w")
        if validate:
            st.update_residual_ratio("w", delayed, torch.tensor(0.01 * (step + 1)))
        pred = st.predict_residual_amax("w", delayed)
        # oracle: the same sequence of amax / measured residual values
        key = "w.w_hi"
        ost["amax"][key] = np.float32(cur) if key not in ost["amax"] else oq._ema_f32(
            ost["amax"][key], np.float32(cur), 0.9)
        assert float(delayed) == float(ost["amax"][key]), step
        if validate:
            r = np.float32(np.float32(0.01 * (step + 1)) / np.float32(delayed))
            rk = "w.ratio"
            ost["ratio"][rk] = r if rk not in ost["ratio"] else oq._ema_f32(ost["ratio"][rk], r, 0.9)
        assert float(pred) == float(max(np.float32(np.float32(delayed) * ost["ratio"]["w.ratio"]),
                                        np.float32(1e-12))), step
        assert validate == (step == 0 or (step + 1) % 3 == 0)
        W = W * 1.1


def test_fuse_tcfp_mlp_structure_and_cpu_fallback():
    from tcfp_amd.nn import TCFPMLP, fuse_tcfp_mlp

    torch.manual_seed(0)
    seq = nn.Sequential(nn.Linear(64, 256), nn.GELU(), nn.Linear(256, 64))
    keys = list(seq.state_dict())
    conv = convert_to_tcfp(seq, use_tensor_cores=True)
    fused = fuse_tcfp_mlp(conv)
    assert isinstance(fused, TCFPMLP) and list(fused.state_dict()) == keys
    assert fused[0] is conv[0] and fused[2] is conv[2]  # the same modules, shared parameters
    # a CPU input is not fusable: the plain sequence runs and raises as
    # TCFPLinear does without a GPU
    assert not fused._fusable(torch.randn(16, 64))
    with pytest.raises(RuntimeError):
        fused(torch.randn(16, 64))
    # nested blocks are replaced in place; other sequences are left alone
    model = nn.Module()
    model.mlp = nn.Sequential(nn.Linear(64, 128), nn.GELU(), nn.Linear(128, 64))
    model.other = nn.Sequential(nn.Linear(64, 64), nn.GELU(approximate="tanh"), nn.Linear(64, 64))
    out = fuse_tcfp_mlp(convert_to_tcfp(model, use_tensor_cores=True, skip_patterns=("none",)))
    assert out is model and isinstance(model.mlp, TCFPMLP) and type(model.other) is nn.Sequential


def test_set_block_dgrad_modes():
    import tcfp_amd.nn as tnn

    assert tnn._BLOCK_DGRAD == "exact"  # the reference's numerics by default
    try:
        tnn.set_block_dgrad("fp8")
        assert tnn._BLOCK_DGRAD == "fp8"
        with pytest.raises(ValueError, match="exact"):
            tnn.set_block_dgrad("tf32")
        assert tnn._BLOCK_DGRAD == "fp8"
    finally:
        tnn.set_block_dgrad("exact")
    assert tnn._BLOCK_DGRAD == "exact"


# names a user of the reference imports (tcfp/__init__.py:12-34; tcfp/core.py
# public functions; the operator layer of tcfp/kernels.py and tcfp/cuda_ext.py
# that tcfp/nn/__init__.py:40-66 binds; the tcfp.nn surface)
_REFERENCE_NAMES = {
    "tcfp": ["ErrorFeedbackState", "FP8Config", "TCFPMode", "ensure_column_major",
             "fp8_matmul", "to_fp8_e4m3", "to_fp8_e4m3_nf_aware", "to_fp8_e4m3_sr",
             "to_fp8_e5m2", "__version__"],
    "tcfp.core": ["FP8_E4M3_MAX", "FP8_E4M3_MIN", "FP8_E4M3_SMALLEST_NORMAL", "FP8_E5M2_MAX",
                  "FP8_E5M2_MIN", "DEFAULT_BLOCK_SIZE", "VALID_BLOCK_SIZES",
                  "SCALE_EXPONENT_BIAS", "TCFPMode", "FP8Config", "to_fp8_e4m3",
                  "to_fp8_e4m3_sr", "to_fp8_e5m2", "to_fp8_e4m3_nf_aware",
                  "ensure_column_major", "compute_block_scales", "ErrorFeedbackState",
                  "stochastic_round_to_fp8_e4m3", "apply_block_scales",
                  "reverse_block_scales", "fp8_matmul", "fp8_matmul_nn", "bits_per_value"],
    "tcfp.kernels": ["is_triton_available", "fused_dual_gemm_forward",
                     "fused_dual_gemm_backward_dx", "block_quantize_fp8",
                     "block_dequantize_fp8", "fused_dual_quantize_fp8", "block_scaled_gemm",
                     "fused_block_scaled_dual_gemm_forward", "fused_act_quant_dual_gemm_forward",
                     "fused_wtquant_block_scaled_dual_gemm_forward",
                     "fused_block_scaled_backward_dx",
                     "fused_block_scaled_dual_gemm_backward_dx"],
    "tcfp.cuda_ext": ["is_cuda_ext_available", "cuda_ext_dual_gemm_forward",
                      "cuda_ext_dual_gemm_backward_dx"],
    "tcfp.nn": ["TCFPLinear", "convert_to_tcfp", "_TCFP12TensorCoreFunction",
                "_TCFP12BlockScaledFunction"],
}


def test_reference_import_names_resolve_to_this_build():
    import importlib
    import sys

    import tcfp_amd

    for mod_name, names in _REFERENCE_NAMES.items():
        mod = importlib.import_module(mod_name)
        # the same module objects, not copies
        assert mod is sys.modules[mod_name.replace("tcfp", "tcfp_amd", 1)], mod_name
        missing = [n for n in names if not hasattr(mod, n)]
        assert not missing, (mod_name, missing)
    import tcfp

    assert tcfp is tcfp_amd
    from tcfp.nn import TCFPLinear as A

    assert A is TCFPLinear
    ns = {}
    exec("from tcfp import *", ns)
    assert set(tcfp.__all__) <= set(ns)


def test_core_host_helpers_match_reference_behaviour():
    from tcfp.core import (
        FP8Config,
        TCFPMode,
        apply_block_scales,
        bits_per_value,
        reverse_block_scales,
    )

    assert bits_per_value(TCFPMode.TCFP12) == 12.5
    assert bits_per_value(TCFPMode.TCFP12, 64) == 12.25
    cfg = FP8Config()
    assert cfg.block_size == 32 and cfg.e4m3_for_weights and cfg.e5m2_for_grads
    # block scaling helpers are plain broadcast arithmetic (CPU tensors here)
    x = torch.randn(4, 64)
    s = torch.tensor([[2.0, 0.5]] * 4)
    y = apply_block_scales(x, s, 32)
    assert torch.equal(y[:, :32], x[:, :32] / 2.0) and torch.equal(y[:, 32:], x[:, 32:] / 0.5)
    assert torch.equal(reverse_block_scales(y, s, 32), x)
    with pytest.raises(AssertionError, match="divisible"):
        from tcfp.core import compute_block_scales

        compute_block_scales(torch.randn(4, 48), 32)


def test_quantize_batch_validation_without_launch():
    """tcfp_quantize_batch: the job struct's layout (tcfp_quant_job, 104
    bytes on x86-64), its workspace size, and the argument checks that
    return before anything is launched (pointers are dummies)."""
    import ctypes

    lib = _hip.load_library()
    assert ctypes.sizeof(_hip.QuantJob) == 104
    assert _hip.QuantJob.rows.offset == 24 and _hip.QuantJob.inv_lo.offset == 96
    one = lib.tcfp_quantize_batch_workspace_bytes(1)
    assert one >= lib.tcfp_workspace_bytes()
    assert lib.tcfp_quantize_batch_workspace_bytes(4) == 4 * one
    assert lib.tcfp_quantize_batch_workspace_bytes(0) == 0
    assert lib.tcfp_quantize_batch_workspace_bytes(5) == 0
    p = 4096
    jobs = (_hip.QuantJob * 1)()
    assert lib.tcfp_quantize_batch(0, jobs, p, one, None) == 1
    assert lib.tcfp_quantize_batch(5, jobs, p, one, None) == 1
    jobs[0] = _hip.QuantJob(_hip.JOB_DUAL, p, 0, 4, 16, None, 0, 0, p, None, p, p, None, p)
    assert lib.tcfp_quantize_batch(1, jobs, None, 0, None) == 5  # no workspace
    assert lib.tcfp_quantize_batch(1, jobs, p, one - 1, None) == 5  # too small
    jobs[0] = _hip.QuantJob(7, p, 0, 4, 16, None, 0, 0, p, None, p, p, None, p)
    assert lib.tcfp_quantize_batch(1, jobs, p, one, None) == 1  # kind
    jobs[0] = _hip.QuantJob(_hip.JOB_DUAL, p, 0, 4, 12, None, 0, 0, p, None, p, p, None, p)
    assert lib.tcfp_quantize_batch(1, jobs, p, one, None) == 1  # cols % 8
    jobs[0] = _hip.QuantJob(_hip.JOB_ACT, p, 0, 4, 16, None, 0, 5, p, None, p, None, None, None)
    assert lib.tcfp_quantize_batch(1, jobs, p, one, None) == 2  # fp8 format


def test_single_pass_wgrad_arguments_without_launch():
    """The split_lo argument of tcfp_block_grad_prep and
    tcfp_block_wgrad_presplit: 0 or 1 only, and the single pass (0) only
    for token counts that are a multiple of 64 -- checked before anything
    is launched (dummy pointers); the single pass's workspace is no larger
    than the split's."""
    lib = _hip.load_library()
    p = 4096
    # (g, m, n, block, g_deq, g_split_t, split_lo, bias_grad, g_fp8, g_exps, ws, ws_bytes, stream)
    assert lib.tcfp_block_grad_prep(p, 128, 256, 64, None, p, 2, None, None, None, None, 0,
                                    None) == 1
    # (g_split_t, split_lo, m, n_out, x, x_fmt, e_x, k_in, block, dw, ws, ws_bytes, stream)
    ws1 = lib.tcfp_block_wgrad_presplit_workspace_bytes(128, 256, 512, 1)
    ws0 = lib.tcfp_block_wgrad_presplit_workspace_bytes(128, 256, 512, 0)
    assert 0 < ws0 <= ws1
    assert lib.tcfp_block_wgrad_presplit(p, 2, 128, 256, p, 0, p, 512, 64, p, p, ws1, None) == 1
    assert lib.tcfp_block_wgrad_presplit(p, 0, 100, 256, p, 0, p, 512, 64, p, p, ws1, None) == 1
    assert lib.tcfp_block_wgrad_presplit(p, 0, 128, 256, p, 0, p, 512, 64, p, p, 0, None) == 5
