"""CPU restatement of Hearth's decode path — test infrastructure only (see oracle.py)."""
