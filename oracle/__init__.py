"""CPU oracle for the HiF8 hot path - test infrastructure only (see hif8_oracle.py)."""
