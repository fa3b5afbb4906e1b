"""CPU oracle for the quantized GEMV/GEMM path (test infrastructure only)."""
