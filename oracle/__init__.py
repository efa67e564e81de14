"""CPU oracle of the fused attention path -- test infrastructure only (see oracle.py)."""
