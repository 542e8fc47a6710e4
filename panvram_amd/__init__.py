"""panvram_amd - panvram's on-device refrel3 v1 decode path, MI355X-native (gfx950 HIP kernels behind a C ABI).

A drop-in for panvram's Python API (reference panvram/__init__.py:1-17):

    c = panvram_amd.Cohort.open(dir, device="cuda")    # reference + assemblies resident in HBM
    x = c.sample(n, W, generator=g)                    # uint8 [n, W] (bytes or tokens) on the device
    y = c.fetch(assembly, contig, start, length)       # a slice by coordinates
"""
import torch  # noqa: F401  (loads the HIP runtime libpanvram_amd.so binds to)

from . import _native
from .cohort import DATASETS, Cohort

FormatError = _native.FormatError
with_cuda = True            # the package is GPU-only: the HIP library is required (ImportError at first use otherwise)
__version__ = "0.1.0"
__all__ = ["Cohort", "DATASETS", "FormatError", "with_cuda"]
