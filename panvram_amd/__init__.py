"""panvram_amd - the refrel3 v1 decode path of panvram, written for MI355X: HIP kernels for gfx950 behind a C ABI,
with a Python `Cohort` that keeps the names, arguments and exceptions of the reference package's (reference
panvram/__init__.py:1-17, panvram/cohort.py), so that code written against it runs after changing the import.

Open a directory of archives once; the reference and every assembly's payload then stay in device memory, and each
call returns a tensor on that device:

    cohort = panvram_amd.Cohort.open("cohort_dir", device="cuda")
    gen = torch.Generator(device="cuda").manual_seed(0)
    batch = cohort.sample(1024, 8192, generator=gen)          # 1024 random windows of 8192 bases, uint8
    piece = cohort.fetch("hap001", "chr1", 10_000, 5_000)     # bases [10000, 15000) of one contig
"""
import torch  # noqa: F401  (the HIP runtime that libpanvram_amd.so binds to, loaded as torch loads it)

from . import _native
from .cohort import DATASETS, Cohort

FormatError = _native.FormatError
with_cuda = True            # the package is GPU-only: the HIP library is required (ImportError at first use otherwise)
__version__ = "0.1.0"
__all__ = ["Cohort", "DATASETS", "FormatError", "with_cuda"]
