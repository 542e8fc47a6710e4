"""Shared fixtures. `gpu` marks tests that need an MI355X (run with -m gpu); everything else runs on the CPU."""
import os
import shutil
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLDEN = os.path.join(ROOT, "tests", "golden")
for p in (ROOT, GOLDEN):
    if p not in sys.path:
        sys.path.insert(0, p)

DATASETS = ("q1k", "q4k", "q16k")
NAMES = ("synthA", "synthB")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device); run with -m gpu")


@pytest.fixture(scope="session")
def fx(tmp_path_factory):
    """The reference's six fixture archives in one directory per dataset, with the regenerated synth_ref.fa."""
    import synth_ref
    d = tmp_path_factory.mktemp("fx")
    ref = synth_ref.write(str(d / "synth_ref.fa"))
    dirs = {}
    for ds in DATASETS:
        dd = d / ds
        dd.mkdir()
        for nm in NAMES:
            shutil.copy(os.path.join(GOLDEN, f"{nm}.{ds}.rr3"), dd / f"{nm}.{ds}.rr3")
        dirs[ds] = str(dd)
    return {"ref": ref, "dirs": dirs}


@pytest.fixture(scope="session")
def oracle_ref(fx):
    from oracle import oracle as O
    return O.reference_bases(fx["ref"])


@pytest.fixture(scope="session")
def mini(tmp_path_factory):
    """The generator's `mini` cohort (3 contigs, 550 kbp; 3 haplotypes with SNVs, indels, SVs up to 8 kbp whose inserted
    sequence carries N and IUPAC bytes, fragmented contigs with reverse-complemented pieces, 50 % soft mask), q4k with
    per-block hashes. Returns {"dir", "ref", "paths", "stats"}."""
    from tests import cohortgen as G
    d = tmp_path_factory.mktemp("mini")
    st = G.make("mini", str(d), threads=4)
    paths = sorted(str(p) for p in d.glob("*.rr3"))
    return {"dir": str(d), "ref": str(d / "reference.fa"), "paths": paths, "stats": st}


@pytest.fixture(scope="session")
def wide(tmp_path_factory):
    """The `mini` shape on a 4.6 Mbp reference with runs of IUPAC codes and an N run across base 2^22, and structural
    variants of 17-40 kbp, so that start diagonals of neighbouring blocks differ by more than a compact block code
    holds (the exception paths of both compact forms). Returns {"dir", "ref", "paths"}."""
    from tests import cohortgen as G
    d = tmp_path_factory.mktemp("wide")
    G.make("mini", str(d), threads=4, ref={"lengths": [4_400_000, 200_000], "iupac_runs": 60, "n_run_at": 1 << 22},
           asm={"sv_min": 17_000, "sv_max": 40_000, "sv_per_contig": 3, "seed": 207})
    paths = sorted(str(p) for p in d.glob("*.rr3"))
    return {"dir": str(d), "ref": str(d / "reference.fa"), "paths": paths}
