"""pan2_amd — PAN 2's Muon Newton–Schulz hot path, native to AMD MI355X (gfx950).

Python host code (``pan2_amd.optim``, a drop-in for the reference's pan/optim)
over a C-ABI HIP library (``libpanmuon.so``, declared in include/panmuon.h).
"""
__version__ = "0.1.0"
