"""inferflux_amd: MI355X (gfx950) quantized GEMV/GEMM path for InferFlux.

The kernels and the C ABI live in libifx_qgemm.so (include/ifx_qgemm.h);
`ops` wraps them for torch device tensors, `fused_quant_gemm` mirrors the
reference's FusedQuantGemm host interface.
"""
from . import ops  # noqa: F401
