"""CPU oracle for the TCFP-12 dual-FP8 hot path (TEST INFRASTRUCTURE ONLY).

This package is a numpy restatement of the reference algorithm
(bwiemz/tcfp, read-only under /root/reference).  It exists so the HIP
kernels in ``tcfp_amd`` can be checked bit-for-bit on the same seeded
inputs.  Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import it, and only as the checker or as the
timed CPU baseline -- never as a product code path.

Every function cites the reference file:line it restates.  Pinning status
(what independent check each function is held to):

=====================================  ==========================================
function                               pinned by
=====================================  ==========================================
fp8.encode / fp8.decode                OCP FP8 spec (brute-force nearest-even over
                                       the 256-entry code table) and torch's CPU
                                       ``.to(float8_*)`` cast
fp8.bf16_round                         torch CPU ``.to(bfloat16)``
quant.ceil_log2_f32                    exact integer maths + torch CPU
                                       ``torch.ceil(torch.log2(.))`` over every
                                       boundary mantissa
quant.to_fp8_per_tensor (a1, a8)       torch CPU ops of ``core.py:99-106``
                                       (``Tensor.__rtruediv__``, IEEE division),
                                       closed-form special cases
quant.dual_quant_per_tensor (a2)       invariants: hi == a1(w), lo == a1(residual),
                                       EF identity, zero-EF == no-EF, EF shrinks
                                       error vs single FP8
quant.block_quantize (a4)              closed form exponent rule + brute-force
                                       nearest code + torch CPU
                                       ``compute_block_scales`` (core.py:221-252)
quant.block_dual_quantize (a3)         fused == separate block_quantize (the
                                       reference's own bitwise test,
                                       test_fused_dual_quant.py:79-155) + EF formula
quant.sr_candidates (a5)               deterministic candidate set; the random
                                       draw itself is statistical only (parity
                                       unpinned bitwise by design: the reference
                                       draws from torch.rand / tl.rand)
gemm.* (a6,a7,a9,a10,a12,a13)          float64 textbook matmul of the same
                                       dequantised FP8 operands
torch_ref.RefTCFP12Function (a1,a2,    the numpy functions above on CPU (codes,
a6-a9 as one training step)            EF, forward, dX, dW) -- used to hold the
                                       HIP path's training loss to the
                                       reference algorithm's
=====================================  ==========================================
"""
