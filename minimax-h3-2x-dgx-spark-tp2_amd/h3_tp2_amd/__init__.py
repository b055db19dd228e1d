"""h3_tp2_amd: the online-FP8 linear path of the MiniMax H3 DiT on MI355X (gfx950).

Three hand-written HIP kernels behind a C ABI (include/h3fp8.h, libh3fp8.so next to this file):
  1. per-token dynamic amax + OCP e4m3fn quant            (ops.quant_rows)
  2. scaled FP8 MFMA GEMM, bf16/fp16 out, fused row-amax   (ops.gemm, ops.scaled_mm, ops.gemm_quant)
  3. gate/up GEMM + SwiGLU + per-token requant            (ops.gemm_swiglu, ops.gemm_swiglu_quant)
and, mirroring the reference plugin's hook surface (h3_tp2.fp8_gemm / fp8_quant_fuse / fp8_swiglu / fp8_consumers /
fp8_cutlass), the modules fp8_gemm, fp8_quant_fuse, fp8_swiglu, fp8_consumers and fp8_hip.
"""
from ._lib import ABI_VERSION, H3Fp8Error, load  # noqa: F401

__all__ = ["ABI_VERSION", "H3Fp8Error", "load"]
