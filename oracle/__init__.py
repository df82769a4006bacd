"""CPU oracle for the DSA path -- test infrastructure only (see dsa_oracle.py)."""
