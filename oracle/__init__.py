"""CPU oracle of the retrieval path — test infrastructure only (see orc.py)."""
