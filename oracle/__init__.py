"""CPU oracle of moex's attention hot path: test infrastructure only (see moex_oracle.c)."""
