"""CPU oracle for the tklab kernels (test infrastructure only; see oracle.py)."""
