"""specfold_amd — SpecFold's folded multi-branch verify step on MI355X (gfx950).

Hand-written HIP kernels behind a C ABI (include/specfold_amd.h), loaded with
ctypes; PyTorch-ROCm provides device memory, streams and the plain GEMMs
(o_proj, FFN, lm_head).  Import ``specfold_amd.generate`` for the generator
classes with the reference's API.
"""

__version__ = "0.1.0"
