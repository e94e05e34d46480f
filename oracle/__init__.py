"""CPU oracle of the quantized matmul path. TEST INFRASTRUCTURE ONLY (see oracle.h)."""
