"""CPU oracle for the FPV2 hot path (test infrastructure only)."""
