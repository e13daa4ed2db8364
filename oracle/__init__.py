"""CPU oracle of the reference encoder numerics -- test infrastructure only (see oracle.py)."""
