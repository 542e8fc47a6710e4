"""Every refusal of the archive reader, against the reference's own reader (oracle/_ref, the reference's csrc/pv_v1.h
compiled where it lies): one good fixture archive is broken in one way at a time - a header field, a section size, the
header XXH3, the bound reference, the meta frame, each meta table - with the header XXH3 recomputed where the break
lies under it, so that the check meant is the one reached. pv_cohort_open must refuse each with the reference's own
message (the check order and wording of FORMAT.md section 5), and accept the unbroken rebuild. Runs on the CPU; skipped
where oracle/_ref is not built."""
import ctypes
import os
import struct

import pytest
import xxhash

from oracle import oracle as O
from panvram_amd import _native as N

_ZSTD = ctypes.CDLL("libzstd.so.1")
_ZSTD.ZSTD_compressBound.restype = ctypes.c_size_t
_ZSTD.ZSTD_compressBound.argtypes = [ctypes.c_size_t]
_ZSTD.ZSTD_compress.restype = ctypes.c_size_t
_ZSTD.ZSTD_compress.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
_ZSTD.ZSTD_decompress.restype = ctypes.c_size_t
_ZSTD.ZSTD_decompress.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_size_t]


def _compress(b):
    cap = _ZSTD.ZSTD_compressBound(len(b))
    out = ctypes.create_string_buffer(cap)
    n = _ZSTD.ZSTD_compress(out, cap, b, len(b), 3)
    return out.raw[:n]


def _decompress(b, size):
    out = ctypes.create_string_buffer(max(size, 1))
    n = _ZSTD.ZSTD_decompress(out, size, b, len(b))
    assert n == size
    return out.raw[:size]


def _leb(v):
    out = bytearray()
    while True:
        c = v & 0x7F
        v >>= 7
        out.append(c | (0x80 if v else 0))
        if not v:
            return bytes(out)


class Parts:
    """An archive cut into header fields, reference name, meta (decompressed), block hashes and payload."""

    def __init__(self, raw):
        self.head = bytearray(raw[:136])
        nl = struct.unpack_from("<H", raw, 136)[0]
        self.name = raw[138:138 + nl]
        mz, mr, hs = (struct.unpack_from("<Q", raw, o)[0] for o in (96, 104, 112))
        p = 138 + nl
        self.meta = bytearray(_decompress(raw[p:p + mz], mr))
        self.hashes = raw[p + mz:p + mz + hs]
        self.payload = raw[p + mz + hs:]
        self.meta_z = None                       # a compressed meta section to use as is (else: compress self.meta)

    def get(self, off):
        return struct.unpack_from("<Q", self.head, off)[0]

    def put(self, off, v, fmt="<Q"):
        struct.pack_into(fmt, self.head, off, v)

    def build(self, rehash=True, sizes=True):
        mz = self.meta_z if self.meta_z is not None else _compress(bytes(self.meta))
        if sizes:
            self.put(96, len(mz))
            self.put(104, len(self.meta))
        body = bytes(self.head) + struct.pack("<H", len(self.name)) + self.name + mz + self.hashes
        if rehash:
            h = xxhash.xxh3_64()
            h.update(body[:128]); h.update(b"\0" * 8); h.update(body[136:])
            body = body[:128] + struct.pack("<Q", h.intdigest()) + body[136:]
        return body + self.payload

    def sections(self):
        """Meta offsets: end of the contig table, end of the case runs (the model tables follow)."""
        m, i = self.meta, 0
        nr = struct.unpack_from("<I", m, i)[0]; i += 4
        for _ in range(nr):
            hl = struct.unpack_from("<I", m, i)[0]; i += 4 + hl + 8 + 4
        ctg_end = i
        nrun = struct.unpack_from("<Q", m, i)[0]; i += 8
        for _ in range(2 * nrun):
            while m[i] & 0x80:
                i += 1
            i += 1
        return ctg_end, i


def _native_msg(ref, path):
    L = N.lib()
    arr = (ctypes.c_char_p * 1)(os.fsencode(path))
    out, err = ctypes.c_void_p(), N.errbuf()
    code = L.pv_cohort_open(os.fsencode(ref), ctypes.cast(arr, ctypes.c_void_p), 1, 1, 0, ctypes.byref(out), err, len(err))
    if code == 0:
        L.pv_cohort_close(out)
        return None
    assert code == N.PV_EFORMAT, (code, err.value)
    return err.value.decode()


def _ref_msg(ref, path):
    try:
        O.RefDecoder.open(ref, [path], threads=1)
        return None
    except ValueError as e:
        return str(e)


def _cases(raw):
    """(label, archive bytes) for each break, in the order of the reader's checks."""
    P = lambda: Parts(raw)                                          # noqa: E731
    out = []

    def case(label, f, **kw):
        p = P()
        r = f(p)
        out.append((label, r if isinstance(r, (bytes, bytearray)) else p.build(**kw)))

    case("short file", lambda p: raw[:100])
    case("magic", lambda p: p.head.__setitem__(0, ord("X")), rehash=False)
    case("version", lambda p: p.put(8, 2, "<I"), rehash=False)
    case("block size", lambda p: p.put(12, 8192, "<I"), rehash=False)
    case("flags", lambda p: p.put(16, 6, "<I"), rehash=False)
    case("reserved", lambda p: p.put(20, 1, "<I"), rehash=False)
    case("section sizes (file one byte short)", lambda p: p.build()[:-1])
    case("section sizes (meta size)", lambda p: p.build()[:96] + struct.pack("<Q", p.get(96) + 5) + p.build()[104:])
    case("block count", lambda p: p.put(72, p.get(72) + 1))
    case("block count (no blocks for bases)", lambda p: (p.put(64, 1), p.put(72, 0)))
    case("hash section size", lambda p: p.put(16, 0, "<I"))
    case("header XXH3", lambda p: p.put(80, p.get(80) ^ 1), rehash=False)
    case("reference SHA-256", lambda p: p.head.__setitem__(30, p.head[30] ^ 0x10))
    case("reference size", lambda p: p.put(56, p.get(56) + 1))
    def meta_size(p):
        p.meta_z = _compress(bytes(p.meta))
        p.put(96, len(p.meta_z)); p.put(104, len(p.meta) + 1)
        return p.build(sizes=False)
    case("meta decompressed size", meta_size)

    def two_frames(p):
        z = _compress(bytes(p.meta))
        p.meta_z = z + _compress(b"x")
        p.put(96, len(p.meta_z)); p.put(104, len(p.meta))
        return p.build(sizes=False)
    case("two meta frames", two_frames)

    def garbled(p):
        z = bytearray(_compress(bytes(p.meta)))
        for k in range(len(z) // 2, len(z) // 2 + 8):
            z[k] ^= 0xA5
        p.meta_z = bytes(z)
        return p.build()
    case("meta frame corrupt", garbled)
    case("record count", lambda p: struct.pack_into("<I", p.meta, 0, 1 << 30))
    case("contig length", lambda p: struct.pack_into("<Q", p.meta, 4 + 4 + struct.unpack_from("<I", p.meta, 4)[0],
                                                      struct.unpack_from("<Q", p.meta, 8 + struct.unpack_from("<I", p.meta, 4)[0])[0] + 1))
    case("line width 0", lambda p: struct.pack_into("<I", p.meta, 16 + struct.unpack_from("<I", p.meta, 4)[0], 0))

    def runs(p, count=None, gap=None):
        ce, re_ = p.sections()
        if count is not None:
            body = struct.pack("<Q", count)
        else:
            body = struct.pack("<Q", 1) + _leb(gap) + _leb(5)
        p.meta[ce:re_] = body
    case("case run count", lambda p: runs(p, count=p.get(64) + 1))
    case("case run past the end", lambda p: runs(p, gap=p.get(64) - 2))

    def model(p):
        _, i = p.sections()
        while not (p.meta[i] < 0x7E and p.meta[i] > 0 and not p.meta[i - 1] & 0x80):   # a one-byte nonzero frequency
            i += 1
        p.meta[i] += 1
    case("model tables", model)
    def block_len(p):
        # the block table is the meta's last 2 x blocks LEB128 numbers; a byte under 0x80 ends one
        ends = [i for i, c in enumerate(p.meta) if c < 0x80]
        first = ends[-2 * p.get(72) - 1] + 1                         # block 0's payload length
        assert p.meta[first] & 0x7F < 0x7F
        p.meta[first] += 1
    case("block table (payload lengths)", block_len)
    case("block table (trailing byte)", lambda p: p.meta.extend(b"\x00"))
    case("block table (truncated)", lambda p: p.meta.__delitem__(slice(len(p.meta) - 3, None)))
    return out


@pytest.mark.parametrize("ds", ["q1k", "q4k", "q16k"])
def test_refusals_match_the_reference_reader(fx, tmp_path, ds):
    if O.ref_lib() is None:
        pytest.skip("oracle/_ref (the reference's reader) is not built")
    good = os.path.join(fx["dirs"][ds], f"synthA.{ds}.rr3")
    raw = open(good, "rb").read()
    rebuilt = tmp_path / "rebuilt.rr3"
    rebuilt.write_bytes(Parts(raw).build())
    assert _native_msg(fx["ref"], str(rebuilt)) is None and _ref_msg(fx["ref"], str(rebuilt)) is None
    seen = set()
    for label, data in _cases(raw):
        p = tmp_path / "case.rr3"
        p.write_bytes(data)
        want, got = _ref_msg(fx["ref"], str(p)), _native_msg(fx["ref"], str(p))
        assert want is not None, label
        assert got == want, (label, got, want)
        seen.add(want.split("refused: ")[-1])
    assert len(seen) >= 14, seen
