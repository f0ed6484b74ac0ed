"""CPU oracle of the sampler — test infrastructure only (see oracle.py)."""
