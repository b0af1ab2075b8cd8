"""CPU oracle of the attention hot path. TEST INFRASTRUCTURE ONLY (see oracle.py)."""
