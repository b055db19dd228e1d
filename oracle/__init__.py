"""CPU oracle of the online-FP8 linear path (test infrastructure only; see oracle.py)."""
