"""XXH3 (own implementation, panvram_amd/csrc/pv_xxh3.h) and SHA-256 (pv_sha256.h) pinned against independent
implementations: the Python `xxhash` package and hashlib."""
import ctypes
import hashlib
import os

import numpy as np
import pytest
import xxhash

from panvram_amd import _native as N


def _xxh(b):
    return N.lib().pv_xxh3_64(b, len(b))


def test_xxh3_every_short_length():
    rng = np.random.default_rng(0)
    data = rng.integers(0, 256, 4200, dtype=np.uint8).tobytes()
    for n in range(0, 4097):
        assert _xxh(data[:n]) == xxhash.xxh3_64_intdigest(data[:n]), n


@pytest.mark.parametrize("n", [1 << 16, (1 << 20) + 17, 3 * 1024 * 1024 + 1023])
def test_xxh3_long(n):
    data = os.urandom(n)
    assert _xxh(data) == xxhash.xxh3_64_intdigest(data)


@pytest.mark.parametrize("n", [0, 5, 200, 240, 241, 1024, 1025, 2048, 5000, 70000])
def test_xxh3_streaming_any_split(n):
    rng = np.random.default_rng(n)
    data = rng.integers(0, 256, n, dtype=np.uint8).tobytes()
    want = xxhash.xxh3_64_intdigest(data)
    for trial in range(20):
        cuts = sorted(set(rng.integers(0, n + 1, int(rng.integers(0, 12))).tolist())) if n else []
        pieces = [data[a:b] for a, b in zip([0] + cuts, cuts + [n])]
        bufs = [ctypes.create_string_buffer(p, len(p)) for p in pieces]
        ptrs = (ctypes.c_void_p * max(1, len(bufs)))(*[ctypes.addressof(b) for b in bufs])
        sizes = (ctypes.c_uint64 * max(1, len(bufs)))(*[len(p) for p in pieces])
        assert N.lib().pv_xxh3_64_parts(ptrs, sizes, len(pieces)) == want, (n, cuts)


def test_sha256_file_bases(tmp_path):
    rng = np.random.default_rng(1)
    for trial in range(6):
        recs = []
        body = bytearray()
        for r in range(int(rng.integers(1, 4))):
            seq = bytes(rng.choice(list(b"ACGTNacgtn"), int(rng.integers(0, 3000))).tolist())
            lw = int(rng.integers(1, 90))
            body += b">r%d x\n" % r + b"".join(seq[i:i + lw] + b"\n" for i in range(0, len(seq), lw))
            recs.append(seq)
        p = tmp_path / f"f{trial}.fa"
        p.write_bytes(bytes(body))
        out, err = ctypes.create_string_buffer(65), N.errbuf()
        assert N.lib().pv_sha256_file_bases(str(p).encode(), out, err, len(err)) == 0
        assert out.value.decode() == hashlib.sha256(b"".join(recs).upper()).hexdigest()


def test_sha256_portable_path(tmp_path):
    """The portable FIPS 180-4 code (used where libcrypto is absent), forced in a fresh process."""
    import subprocess
    import sys
    data = bytes(np.random.default_rng(2).choice(list(b"ACGTN"), 200_003).tolist())
    p = tmp_path / "p.fa"
    p.write_bytes(b">x\n" + b"\n".join(data[i:i + 61] for i in range(0, len(data), 61)) + b"\n")
    code = ("import ctypes,sys; sys.path.insert(0, %r); from panvram_amd import _native as N; o=ctypes.create_string_buffer(65); "
            "e=N.errbuf(); N.lib().pv_sha256_file_bases(%r, o, e, len(e)); print(o.value.decode())") % (
        os.path.dirname(os.path.dirname(os.path.abspath(__file__))), str(p).encode())
    env = dict(os.environ, PANVRAM_SHA256_PORTABLE="1")
    out = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True, check=True).stdout.strip()
    assert out == hashlib.sha256(data).hexdigest()


def test_xxh3_stream_handle_any_split():
    """pv_xxh3_stream_*: the digest of consecutive pieces equals xxhash of their concatenation, at every point."""
    L = N.lib()
    rng = np.random.default_rng(5)
    for total in (0, 1, 240, 241, 1023, 1024, 1025, 70_000, 300_001):
        data = rng.integers(0, 256, total, dtype=np.uint8).tobytes()
        h = L.pv_xxh3_stream_new()
        try:
            cut = sorted(set(int(x) for x in rng.integers(0, total + 1, 6))) if total else []
            prev = 0
            for c in cut + [total]:
                piece = data[prev:c]
                buf = ctypes.create_string_buffer(piece, len(piece)) if piece else None
                L.pv_xxh3_stream_update(h, buf, len(piece))
                assert L.pv_xxh3_stream_digest(h) == xxhash.xxh3_64_intdigest(data[:c]), (total, c)
                prev = c
        finally:
            L.pv_xxh3_stream_free(h)
