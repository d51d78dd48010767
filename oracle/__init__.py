"""CPU oracle for the quantized decode path (test infrastructure only; see marin_oracle.c)."""
