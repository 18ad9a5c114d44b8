"""CPU oracle (test infrastructure only; see gs_oracle.h)."""
