"""CPU oracle (test infrastructure only): see ``oracle/ref_mla.py``."""
