"""CPU oracle for the VQ decode path -- test infrastructure only (see vq_oracle.py)."""
