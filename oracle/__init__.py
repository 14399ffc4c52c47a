"""CPU oracle of the Q4_K weight path: test infrastructure only (see oracle.py)."""
