"""CPU oracle for the gated DeltaNet op: test infrastructure only (see gdn_oracle.py's header)."""
