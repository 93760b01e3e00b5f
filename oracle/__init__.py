"""CPU oracle for the MLA decode path (test infrastructure only; see
oracle/mla_oracle.py)."""
