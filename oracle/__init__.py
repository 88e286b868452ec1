"""CPU oracle package -- test infrastructure only (see poly_oracle.py)."""
