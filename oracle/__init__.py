"""CPU oracle for tbf16's hot path (test infrastructure only; see tbf16_oracle)."""
