"""CPU oracle of the sparse-convolution hot path (test infrastructure only; see oracle.py)."""
