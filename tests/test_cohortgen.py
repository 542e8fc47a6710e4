"""The synthetic cohort generator (tests/cohortgen) against the oracle: every archive it writes must decode to the
hashes it wrote into the header and hash section, and equal the reference's own decoder where that is built. These
cohorts carry what the reference's small fixtures do not: long literal runs with N and escape bytes, soft-mask runs,
reverse-complemented pieces."""
import numpy as np
import pytest

from oracle import oracle as O


def test_mini_archives_decode_to_their_hashes(mini):
    import xxhash
    ref = O.reference_bases(mini["ref"])
    assert len(mini["paths"]) == 3
    for p in mini["paths"]:
        A = O.Archive(p)
        assert A.Q == 4096
        for b in range(A.nblocks):                            # the hash section: every block's upper-case bytes
            assert xxhash.xxh3_64_intdigest(A.block(ref, b).tobytes()) == A.block_hash(b), (p, b)
        full = A.full(ref)
        assert full.size == A.nbases
        assert xxhash.xxh3_64_intdigest(full.tobytes()) == A.bases_xxh          # header offset 88
        assert xxhash.xxh3_64_intdigest(A.fasta(ref)) == A.fasta_xxh            # header offset 80


def test_mini_has_the_cases_it_is_for(mini):
    ref = O.reference_bases(mini["ref"])
    seen = set()
    lower = 0
    for p in mini["paths"]:
        full = O.Archive(p).full(ref)
        seen |= set(np.unique(full).tolist())
        lower += int((full >= ord("a")).sum())
    assert lower > 0                                          # soft-mask runs
    assert ord("N") in seen or ord("n") in seen               # N (reference N runs and inserted N)
    assert seen & set(b"RYKMSW")                              # escape literals (8 raw bits)


def test_mini_equals_reference_decoder(mini):
    R = O.RefDecoder.open(mini["ref"], mini["paths"], threads=4)
    if R is None:
        pytest.skip("oracle/_ref not built (reference sources absent)")
    ref = O.reference_bases(mini["ref"])
    arcs = [O.Archive(p) for p in mini["paths"]]
    rng = np.random.default_rng(11)
    for W in (1, 777, 4096, 9000):
        a = rng.integers(0, len(arcs), 500)
        s = np.array([rng.integers(0, arcs[int(i)].nbases - W + 1) for i in a], dtype=np.int64)
        rc = rng.integers(0, 2, 500).astype(np.uint8)
        for tokens in (False, True):
            x = O.windows(arcs, ref, a, s, W, rc=rc, tokens=tokens)
            y = R.windows(a, s, W, rc=rc, tokens=tokens)
            assert np.array_equal(x, y), (W, tokens)
