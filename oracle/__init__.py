"""CPU oracle of the motion decoder — test infrastructure only (see mdec.py)."""
