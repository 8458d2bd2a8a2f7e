"""CPU oracle of the ipu-stack hot path (test infrastructure only; see oracle.py)."""
