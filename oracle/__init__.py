"""CPU oracle for the H3 DiT hot path (test infrastructure only; see h3_oracle)."""
