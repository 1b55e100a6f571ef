"""CPU oracle of the INT8 deployment hot path -- test infrastructure only (see oracle.py)."""
