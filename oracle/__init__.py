"""CPU oracle for the fused residual-add + RMSNorm path (test infrastructure only)."""
