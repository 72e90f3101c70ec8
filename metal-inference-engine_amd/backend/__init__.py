"""The ROCm backend of the token-mixing path (rocm.py)."""
