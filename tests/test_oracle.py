"""The CPU oracle (oracle/pv_oracle.c) pinned before it is trusted:
  - every block of the six reference fixture archives against the archive's own per-block XXH3 (upper case);
  - the whole base stream (case applied) against the header's base-stream XXH3, the rebuilt FASTA against the
    header's source-FASTA XXH3;
  - the regenerated reference against the SHA-256 the archive headers bind;
  - windows against the reference's own decoder built from its sources (oracle/_ref), where that build exists;
  - a planted mistake in the oracle's inputs is caught (a payload bit flip fails a block hash or the decode)."""
import hashlib
import os
import struct

import numpy as np
import pytest
import xxhash

from oracle import oracle as O

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
FIXTURES = [f"{nm}.{ds}.rr3" for nm in ("synthA", "synthB") for ds in ("q1k", "q4k", "q16k")]


def test_reference_sha256_matches_headers(fx, oracle_ref):
    sha = hashlib.sha256(oracle_ref.tobytes()).digest()
    for f in FIXTURES:
        h = open(os.path.join(GOLD, f), "rb").read(64)
        assert h[24:56] == sha and struct.unpack_from("<Q", h, 56)[0] == oracle_ref.size


@pytest.mark.parametrize("f", FIXTURES)
def test_every_block_hash(f, oracle_ref):
    A = O.Archive(os.path.join(GOLD, f))
    assert A.nblocks == (A.nbases + A.Q - 1) // A.Q
    for b in range(A.nblocks):
        assert xxhash.xxh3_64_intdigest(A.block(oracle_ref, b).tobytes()) == A.block_hash(b), b


@pytest.mark.parametrize("f", FIXTURES)
def test_stream_and_fasta_hash(f, oracle_ref):
    A = O.Archive(os.path.join(GOLD, f))
    assert xxhash.xxh3_64_intdigest(A.full(oracle_ref).tobytes()) == A.bases_xxh
    assert xxhash.xxh3_64_intdigest(A.fasta(oracle_ref)) == A.fasta_xxh


def test_windows_closed_forms(oracle_ref):
    """rc twice is the identity; tokens of the reverse complement are 3 - token reversed (ACGT only); case only
    differs by 0x20."""
    A = [O.Archive(os.path.join(GOLD, f"{nm}.q4k.rr3")) for nm in ("synthA", "synthB")]
    rng = np.random.default_rng(5)
    W, n = 3000, 300
    asm = rng.integers(0, 2, n)
    start = np.array([rng.integers(0, A[a].nbases - W + 1) for a in asm])
    fwd = O.windows(A, oracle_ref, asm, start, W)
    rev = O.windows(A, oracle_ref, asm, start, W, rc=np.ones(n, np.uint8))
    comp = bytes.maketrans(b"ACGTacgt", b"TGCAtgca")
    for k in range(n):
        assert rev[k].tobytes() == fwd[k].tobytes().translate(comp)[::-1]
    up = O.windows(A, oracle_ref, asm, start, W, apply_case=False)
    assert np.array_equal(up, np.where((fwd >= ord("a")) & (fwd <= ord("z")), fwd - 32, fwd))
    tf = O.windows(A, oracle_ref, asm, start, W, tokens=True)
    tr = O.windows(A, oracle_ref, asm, start, W, rc=np.ones(n, np.uint8), tokens=True)
    m = tf < 4
    assert np.array_equal(np.where(m, 3 - tf, tf)[:, ::-1], tr)


@pytest.mark.skipif(O.ref_lib() is None, reason="oracle/_ref not built (reference sources absent)")
@pytest.mark.parametrize("ds", ["q1k", "q4k", "q16k"])
def test_oracle_equals_reference_decoder(fx, oracle_ref, ds):
    paths = [os.path.join(GOLD, f"{nm}.{ds}.rr3") for nm in ("synthA", "synthB")]
    R = O.RefDecoder.open(fx["ref"], paths)
    A = [O.Archive(p) for p in paths]
    rng = np.random.default_rng(11)
    for W in (1, 13, 1024, 5000, 16385):
        n = 400
        asm = rng.integers(0, 2, n)
        start = np.array([rng.integers(0, A[a].nbases - W + 1) for a in asm])
        rc = rng.integers(0, 2, n).astype(np.uint8)
        for tok in (False, True):
            assert np.array_equal(O.windows(A, oracle_ref, asm, start, W, rc=rc, tokens=tok, threads=4),
                                  R.windows(asm, start, W, rc=rc, tokens=tok, threads=4))


def test_planted_payload_flip_is_caught(tmp_path, oracle_ref):
    """A flipped payload bit either fails a block (decode or XXH3) or leaves the bytes unchanged - never silent."""
    raw = bytearray(open(os.path.join(GOLD, "synthA.q4k.rr3"), "rb").read())
    good = O.Archive(os.path.join(GOLD, "synthA.q4k.rr3")).full(oracle_ref, apply_case=False)
    caught = 0
    for k in range(40):
        b = bytearray(raw)
        p = len(b) - 1 - (k * 97) % 3000
        b[p] ^= 1 << (k % 8)
        f = tmp_path / f"c{k}.rr3"
        f.write_bytes(bytes(b))
        A = O.Archive(str(f))
        bad = False
        for blk in range(A.nblocks):
            try:
                if xxhash.xxh3_64_intdigest(A.block(oracle_ref, blk).tobytes()) != A.block_hash(blk):
                    bad = True
            except ValueError:
                bad = True
        if not bad:
            assert np.array_equal(A.full(oracle_ref, apply_case=False), good)
        caught += bad
    assert caught > 30


def test_sample_coords_against_enumeration():
    """oracle.sample_coords pinned by brute force: the u-th draw names the u-th valid window when every (assembly,
    contig, start) with start + W <= the contig's length is listed in cohort order; contigs shorter than W (first,
    last, between) hold none. A left-sided search, an offset off by one or a dropped short contig fails this."""
    lengths = [[3, 10, 1, 7], [], [12], [2, 9, 4]]
    for W in (1, 2, 4, 7, 9, 10, 12):
        every = [(a, c, s) for a, ls in enumerate(lengths) for c, L in enumerate(ls) for s in range(L - W + 1)]
        u = np.arange(len(every), dtype=np.int64)
        co, total = O.sample_coords(lengths, W, u)
        assert total == len(every)
        assert [tuple(r[:3]) for r in co.tolist()] == every and not co[:, 3].any()
    co, total = O.sample_coords(lengths, 13, np.zeros(0, dtype=np.int64))
    assert total == 0 and co.shape == (0, 4)
    rnd = np.array([0.1, 0.5, 0.49, 0.9], dtype=np.float32)
    co, _ = O.sample_coords(lengths, 4, np.array([0, 5, 6, 20]), rnd=rnd, p=0.5)
    assert co[:, 3].tolist() == [1, 0, 1, 0]
    co, _ = O.sample_coords(lengths, 4, np.array([0, 5]), rc_all=True)
    assert co[:, 3].tolist() == [1, 1]
