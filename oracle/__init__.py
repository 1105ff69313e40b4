"""CPU oracle of the VQ2 decode hot path (test infrastructure only)."""
