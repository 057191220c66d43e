"""CPU oracle of the reference arithmetic: test infrastructure only (see oracle.py)."""
