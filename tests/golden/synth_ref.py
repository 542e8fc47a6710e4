"""Regenerates `synth_ref.fa`, the reference FASTA the six fixture archives in this directory were encoded against
(their headers bind it by SHA-256 at offset 24 and by size at offset 56: 750,000 bases).

The recipe is the reference's deterministic generator (reference tests/synth.py:62-67 `reference()`, with
`_rng` :14-16, `_rand_seq` :19-20 and `_fasta` :53-59): three records drawn from `random.Random(20261004)` - chrA
400,000 random ACGT, chrB 300,000, chrC 20,000 + 3,000 N + 27,000 - written with 80 bases per line. Only
`random.Random.random()` is used, whose sequence is fixed across Python versions, so the bytes (and their SHA-256)
are reproducible; tests/test_oracle.py checks the SHA-256 against all six archive headers.

    python tests/golden/synth_ref.py <out.fa>
"""
import random
import sys

RECIPE_SEED = 20261004
LINE = 80


def _draw(rng, alphabet, n):
    # one uniform index per base: int(random() * len(alphabet))
    k = len(alphabet)
    return bytes(alphabet[int(rng.random() * k)] for _ in range(n))


def records():
    rng = random.Random(RECIPE_SEED)
    a = _draw(rng, b"ACGT", 400_000)
    b = _draw(rng, b"ACGT", 300_000)
    c = _draw(rng, b"ACGT", 20_000) + b"N" * 3000 + _draw(rng, b"ACGT", 27_000)
    return [(b"chrA synthetic", a), (b"chrB", b), (b"chrC", c)]


def fasta_bytes():
    out = bytearray()
    for hdr, seq in records():
        out += b">" + hdr + b"\n"
        for i in range(0, len(seq), LINE):
            out += seq[i:i + LINE] + b"\n"
    return bytes(out)


def write(path):
    data = fasta_bytes()
    with open(path, "wb") as f:
        f.write(data)
    return path


if __name__ == "__main__":
    write(sys.argv[1])
