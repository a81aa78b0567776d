"""CPU oracle for CVMM (test infrastructure only; never imported by the product)."""
