"""CPU oracle of the GDN recurrence (test infrastructure only; see gdn_oracle.py)."""
