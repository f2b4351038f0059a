"""CPU parity oracle (test infrastructure only; see si_oracle.h)."""
