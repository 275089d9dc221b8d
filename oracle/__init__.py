"""CPU oracle of ANNC's hot path -- test infrastructure only (see ora.py)."""
