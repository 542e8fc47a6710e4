"""ctypes wrapper of the CPU oracle (liboracle.so, this directory) and of the reference harness (_ref/libpv_ref.so).

TEST INFRASTRUCTURE ONLY - the parity checker. Imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg; never by the panvram_amd package.
"""
import ctypes
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
_lib = None
_ref = None


def lib():
    global _lib
    if _lib is None:
        L = ctypes.CDLL(os.path.join(HERE, "liboracle.so"))
        vp, u64, i64, u32 = ctypes.c_void_p, ctypes.c_uint64, ctypes.c_int64, ctypes.c_uint32
        L.oracle_fasta_bases.argtypes = [vp, u64]; L.oracle_fasta_bases.restype = i64
        L.oracle_open.argtypes = [vp, u64, ctypes.POINTER(vp)]; L.oracle_open.restype = ctypes.c_int
        L.oracle_close.argtypes = [vp]; L.oracle_close.restype = None
        L.oracle_decode_block.argtypes = [vp, vp, u64, u64, vp]; L.oracle_decode_block.restype = ctypes.c_int
        L.oracle_full.argtypes = [vp, vp, u64, vp, ctypes.c_int]; L.oracle_full.restype = ctypes.c_int
        L.oracle_windows.argtypes = [vp, i64, vp, u64, vp, vp, i64, i64, vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, vp]
        L.oracle_windows.restype = ctypes.c_int
        for name, rt in (("Q", u32), ("nbases", u64), ("nblocks", u64), ("fasta_xxh", u64), ("bases_xxh", u64),
                         ("has_hashes", ctypes.c_int), ("nrec", u32), ("nlow", u64)):
            f = getattr(L, "oracle_" + name); f.argtypes = [vp]; f.restype = rt
        L.oracle_block_hash.argtypes = [vp, u64]; L.oracle_block_hash.restype = u64
        L.oracle_payload_len.argtypes = [vp, u64]; L.oracle_payload_len.restype = u64
        L.oracle_payload_off.argtypes = [vp, u64]; L.oracle_payload_off.restype = u64
        L.oracle_payload_bytes.argtypes = [vp]; L.oracle_payload_bytes.restype = u64
        L.oracle_block_state.argtypes = [vp, u64]; L.oracle_block_state.restype = i64
        L.oracle_block_refbytes.argtypes = [vp, vp, u64, u64]; L.oracle_block_refbytes.restype = i64
        L.oracle_rec_hdr.argtypes = [vp, u32]; L.oracle_rec_hdr.restype = ctypes.c_char_p
        for name, rt in (("len", u64), ("boff", u64), ("lw", u32)):
            f = getattr(L, "oracle_rec_" + name); f.argtypes = [vp, u32]; f.restype = rt
        _lib = L
    return _lib


def ref_lib():
    """The reference's own decoder (oracle/_ref), or None where it was not built (no reference sources)."""
    global _ref
    if _ref is None:
        p = os.path.join(HERE, "_ref", "libpv_ref.so")
        if not os.path.exists(p):
            return None
        L = ctypes.CDLL(p)
        vp = ctypes.c_void_p
        L.ref_open.argtypes = [ctypes.c_char_p, vp, ctypes.c_int, ctypes.c_int, ctypes.c_char_p, ctypes.c_size_t]; L.ref_open.restype = vp
        L.ref_close.argtypes = [vp]
        L.ref_windows.argtypes = [vp, vp, vp, ctypes.c_int64, ctypes.c_int64, vp, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, vp]
        L.ref_windows.restype = ctypes.c_int
        L.ref_block.argtypes = [vp, ctypes.c_int64, ctypes.c_uint64, ctypes.c_int, vp]; L.ref_block.restype = ctypes.c_int
        L.ref_block_refbytes.argtypes = [vp, ctypes.c_int64, ctypes.c_uint64]; L.ref_block_refbytes.restype = ctypes.c_int64
        _ref = L
    return _ref


def _ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p) if a is not None else None


def reference_bases(path):
    """FASTA file -> numpy uint8 bases, upper case (the decoded reference)."""
    b = np.fromfile(path, dtype=np.uint8)
    n = lib().oracle_fasta_bases(_ptr(b), b.size)
    if n < 0:
        raise ValueError(f"{path}: not FASTA")
    return b[:n].copy()


class Archive:
    def __init__(self, path):
        data = np.fromfile(path, dtype=np.uint8)
        h = ctypes.c_void_p()
        rc = lib().oracle_open(_ptr(data), data.size, ctypes.byref(h))
        if rc:
            raise ValueError(f"{path}: refused by the oracle reader (code {rc})")
        self.h, self.path = h, path

    def __del__(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.oracle_close(self.h)
            self.h = None

    @property
    def Q(self):
        return lib().oracle_Q(self.h)

    @property
    def nbases(self):
        return lib().oracle_nbases(self.h)

    @property
    def nblocks(self):
        return lib().oracle_nblocks(self.h)

    @property
    def fasta_xxh(self):
        return lib().oracle_fasta_xxh(self.h)

    @property
    def bases_xxh(self):
        return lib().oracle_bases_xxh(self.h)

    def block_hash(self, b):
        return lib().oracle_block_hash(self.h, b) if lib().oracle_has_hashes(self.h) else None

    def payload_len(self, b):
        return lib().oracle_payload_len(self.h, b)

    def payload_file_offset(self, b):
        """Offset in the archive file of block b's first payload byte (the payload section ends the file)."""
        return os.path.getsize(self.path) - lib().oracle_payload_bytes(self.h) + lib().oracle_payload_off(self.h, b)

    def records(self):
        L = lib()
        return [(L.oracle_rec_hdr(self.h, r).decode(), L.oracle_rec_len(self.h, r), L.oracle_rec_boff(self.h, r), L.oracle_rec_lw(self.h, r))
                for r in range(L.oracle_nrec(self.h))]

    def block(self, ref, b):
        out = np.empty(self.Q, dtype=np.uint8)
        if lib().oracle_decode_block(self.h, _ptr(ref), ref.size, b, _ptr(out)):
            raise ValueError(f"{self.path}: block {b} failed to decode")
        n = min(self.Q, self.nbases - b * self.Q)
        return out[:n]

    def refbytes(self, ref, b):
        """bytes of block b produced by reference copies (kinds 1 and 3)"""
        return lib().oracle_block_refbytes(self.h, _ptr(ref), ref.size, b)

    def full(self, ref, apply_case=True):
        out = np.empty(max(self.nbases, 1), dtype=np.uint8)
        if lib().oracle_full(self.h, _ptr(ref), ref.size, _ptr(out), int(apply_case)):
            raise ValueError(f"{self.path}: decode failed")
        return out[:self.nbases]

    def fasta(self, ref):
        b = self.full(ref).tobytes()
        out = bytearray()
        for hdr, ln, boff, lw in self.records():
            out += b">" + hdr.encode() + b"\n"
            for x in range(0, ln, lw):
                out += b[boff + x:boff + min(ln, x + lw)] + b"\n"
        return bytes(out)


def windows(archives, ref, asm, start, W, rc=None, tokens=False, apply_case=True, threads=1):
    """The oracle's Core::windows: uint8 [n, W] (numpy). archives: list of Archive."""
    asm = np.ascontiguousarray(asm, dtype=np.int64)
    start = np.ascontiguousarray(start, dtype=np.int64)
    n = asm.size
    out = np.empty((n, W), dtype=np.uint8)
    hs = (ctypes.c_void_p * max(1, len(archives)))(*[a.h.value for a in archives])
    r = None if rc is None else np.ascontiguousarray(rc, dtype=np.uint8)
    e = lib().oracle_windows(hs, len(archives), _ptr(ref), ref.size, _ptr(asm), _ptr(start), n, W, _ptr(r), int(tokens), int(apply_case),
                             int(threads), _ptr(out))
    if e == 3:
        raise ValueError("window outside the assembly")
    if e:
        raise ValueError("block decode failed (corrupt archive)")
    return out


def sample_coords(lengths, W, u, rnd=None, p=None, rc_all=False):
    """The coordinates `sample` derives from its draws (reference panvram/cohort.py:168-194): lengths[a] lists the
    contig lengths of assembly a, in cohort order (assembly, then contig; csrc/pv_core.cpp:75-86); u are the
    torch.randint(0, total, (n,)) draws over the total number of valid starts; rnd the torch.rand(n) draws (p a
    probability), or rc_all for every window reverse-complemented. -> (int64 [n, 4] of (assembly, contig index, start
    in the contig, strand), total)."""
    tab = [(a, c, L) for a, ls in enumerate(lengths) for c, L in enumerate(ls)]
    v = np.array([max(L - W + 1, 0) for _, _, L in tab], dtype=np.int64)
    cum = np.cumsum(v)
    u = np.asarray(u, dtype=np.int64)
    k = np.searchsorted(cum, u, side="right")
    out = np.zeros((u.size, 4), dtype=np.int64)
    out[:, 0] = [tab[i][0] for i in k]
    out[:, 1] = [tab[i][1] for i in k]
    out[:, 2] = u - (cum[k] - v[k])
    if rc_all:
        out[:, 3] = 1
    elif rnd is not None:
        out[:, 3] = np.asarray(rnd) < p
    return out, int(cum[-1]) if cum.size else 0


class RefDecoder:
    """The reference's own CPU decoder (oracle/_ref harness); None-safe constructor via RefDecoder.open."""

    @classmethod
    def open(cls, reference, paths, threads=0):
        L = ref_lib()
        if L is None:
            return None
        arr = (ctypes.c_char_p * len(paths))(*[os.fsencode(p) for p in paths])
        err = ctypes.create_string_buffer(1024)
        h = L.ref_open(os.fsencode(reference), ctypes.cast(arr, ctypes.c_void_p), len(paths), int(threads), err, 1024)
        if not h:
            raise ValueError(err.value.decode())
        self = cls()
        self.h, self.L = h, L
        return self

    def __del__(self):
        if getattr(self, "h", None):
            self.L.ref_close(self.h)
            self.h = None

    def windows(self, asm, start, W, rc=None, tokens=False, apply_case=True, verify=False, threads=1):
        asm = np.ascontiguousarray(asm, dtype=np.int64)
        start = np.ascontiguousarray(start, dtype=np.int64)
        out = np.empty((asm.size, W), dtype=np.uint8)
        r = None if rc is None else np.ascontiguousarray(rc, dtype=np.uint8)
        e = self.L.ref_windows(self.h, _ptr(asm), _ptr(start), asm.size, W, _ptr(r), int(tokens), int(apply_case), int(verify), int(threads), _ptr(out))
        if e:
            raise ValueError(f"reference decoder error {e}")
        return out

    def refbytes(self, a, b):
        return self.L.ref_block_refbytes(self.h, a, b)

    def block(self, a, b, Q, nbases, verify=False):
        out = np.empty(Q, dtype=np.uint8)
        e = self.L.ref_block(self.h, a, b, int(verify), _ptr(out))
        if e:
            raise ValueError(f"reference decoder error {e}")
        return out[:min(Q, nbases - b * Q)]
