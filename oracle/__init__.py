"""CPU oracle for the affine-quantized matmul path (test infrastructure only)."""
