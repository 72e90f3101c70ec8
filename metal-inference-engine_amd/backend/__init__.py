"""Backends of the token-mixing path: the protocol slice (base.py) and the ROCm implementation (rocm.py)."""
