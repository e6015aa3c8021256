"""CPU oracle for the dilution-attention hot path (test infrastructure only)."""
