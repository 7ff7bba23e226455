"""CPU oracle of the DSALT hot path (test infrastructure only; see dsalt_oracle.py)."""
