"""CPU oracle of the int4 clock path -- test infrastructure only (see i4ref.py)."""
