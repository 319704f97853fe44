"""CPU oracle for the triangle hot path (test infrastructure only; see triangle_oracle)."""
