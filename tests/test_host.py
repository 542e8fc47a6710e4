"""Host side of the product through its C ABI (no GPU): open with every check, refusals with the reference's
messages, contig / info tables, FASTA rebuild and XXH3, block verification, case application, and the exported
symbol set of include/panvram_amd.h."""
import ctypes
import os
import re
import shutil

import numpy as np
import pytest
import xxhash

from oracle import oracle as O
from panvram_amd import _native as N

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
GOLD = os.path.join(ROOT, "tests", "golden")


def native_open(ref, files):
    L = N.lib()
    arr = (ctypes.c_char_p * len(files))(*[os.fsencode(f) for f in files])
    out, err = ctypes.c_void_p(), N.errbuf()
    code = L.pv_cohort_open(os.fsencode(ref), ctypes.cast(arr, ctypes.c_void_p), len(files), 2, ctypes.byref(out), err, len(err))
    return code, err.value.decode(), out.value


class Handle:
    def __init__(self, ref, files):
        code, msg, h = native_open(ref, files)
        assert code == 0, msg
        self.h = h

    def __del__(self):
        N.lib().pv_cohort_close(self.h)


def test_exports_every_declared_symbol():
    hdr = open(os.path.join(ROOT, "include", "panvram_amd.h")).read()
    names = set(re.findall(r"^\s*(?:int32_t|int64_t|uint64_t|void)\s+\**\s*(pv_\w+)\s*\(", hdr, re.M))
    assert len(names) >= 20
    L = ctypes.CDLL(N.LIB_PATH)
    for nm in sorted(names):
        assert hasattr(L, nm), nm
    assert set(N.SIGNATURES) == names
    assert N.lib().pv_abi_version() == int(re.search(r"#define PV_ABI_VERSION (\d+)", hdr).group(1))


def test_open_tables(fx):
    files = [os.path.join(fx["dirs"]["q4k"], f"{nm}.q4k.rr3") for nm in ("synthA", "synthB")]
    h = Handle(fx["ref"], files)
    L = N.lib()
    assert L.pv_cohort_block_size(h.h) == 4096 and L.pv_cohort_assemblies(h.h) == 2 and L.pv_cohort_ref_bases(h.h) == 750000
    sha = ctypes.create_string_buffer(65)
    L.pv_cohort_ref_sha256(h.h, sha)
    assert sha.value.decode() == open(files[0], "rb").read(56)[24:56].hex()
    for a, f in enumerate(files):
        A = O.Archive(f)
        x = N.AsmInfo()
        assert L.pv_asm_info_get(h.h, a, ctypes.byref(x)) == 0
        assert (x.Q, x.bases, x.blocks, x.fasta_xxh3, x.block_hashes) == (4096, A.nbases, A.nblocks, A.fasta_xxh, 1)
        recs = A.records()
        assert x.contigs == len(recs)
        for k, (hdr, ln, boff, lw) in enumerate(recs):
            nm, hd = ctypes.c_char_p(), ctypes.c_char_p()
            l2, o2, w2 = ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint32()
            assert L.pv_asm_contig(h.h, a, k, ctypes.byref(nm), ctypes.byref(hd), ctypes.byref(l2), ctypes.byref(o2), ctypes.byref(w2)) == 0
            assert (hd.value.decode(), l2.value, o2.value, w2.value) == (hdr, ln, boff, lw)
            assert nm.value.decode() == re.split(r"[ \t]", hdr)[0]


def test_pooled_arrays(fx):
    files = [os.path.join(fx["dirs"]["q1k"], f"{nm}.q1k.rr3") for nm in ("synthA", "synthB")]
    h = Handle(fx["ref"], files)
    L = N.lib()

    def arr(i, dt):
        p, n = ctypes.c_void_p(), ctypes.c_uint64()
        assert L.pv_cohort_array(h.h, i, ctypes.byref(p), ctypes.byref(n)) == 0
        return np.frombuffer((ctypes.c_uint8 * n.value).from_address(p.value), dtype=dt).copy() if n.value else np.zeros(0, dt)
    asm = arr(N.ARR_ASM, np.int64).reshape(-1, 8)
    off, st, run0 = arr(N.ARR_OFF, np.uint32), arr(N.ARR_ST, np.int64), arr(N.ARR_RUN0, np.uint32)
    low_s, low_l = arr(N.ARR_LOW_S, np.int64), arr(N.ARR_LOW_L, np.int64)
    P = arr(N.ARR_P, np.uint8)
    for a, f in enumerate(files):
        A = O.Archive(f)
        pb, bb, nbases, lb, lc = asm[a, :5]
        assert nbases == A.nbases
        for b in range(A.nblocks):
            assert off[bb + b + 1] - off[bb + b] == A.payload_len(b)
            assert st[bb + b] == O.lib().oracle_block_state(A.h, b)
            # first case run ending after the block start
            r = run0[bb + b]
            ends = low_s[lb:lb + lc] + low_l[lb:lb + lc]
            assert r == int(np.searchsorted(ends, b * 1024, side="right"))
    assert P[-64:].sum() == 0


def test_refusals(fx, tmp_path):
    good = os.path.join(fx["dirs"]["q4k"], "synthA.q4k.rr3")
    raw = open(good, "rb").read()
    ref = bytearray(open(fx["ref"], "rb").read())
    k = ref.index(b"\n") + 5
    ref[k] ^= 0x01 if ref[k] != ord("A") else 0x02
    bad_ref = tmp_path / "bad_ref.fa"
    bad_ref.write_bytes(bytes(ref))
    code, msg, _ = native_open(str(bad_ref), [good])
    assert code == N.PV_EFORMAT and "wrong reference" in msg
    for i, mut in enumerate((lambda b: b[:40] + bytes([b[40] ^ 1]) + b[41:], lambda b: b[:130] + bytes([b[130] ^ 1]) + b[131:],
                             lambda b: b[:-1], lambda b: b[:8] + b"\x02" + b[9:], lambda b: b[:12] + b"\x00\x03" + b[14:],
                             lambda b: b[:100])):
        p = tmp_path / f"bad{i}.rr3"
        p.write_bytes(mut(raw))
        code, msg, _ = native_open(fx["ref"], [str(p)])
        assert code == N.PV_EFORMAT and "refused" in msg, (i, msg)
    code, msg, _ = native_open(fx["ref"], [good, os.path.join(fx["dirs"]["q1k"], "synthB.q1k.rr3")])
    assert code == N.PV_EFORMAT and "block size" in msg
    code, msg, _ = native_open(fx["ref"], [str(tmp_path / "missing.rr3")])
    assert code == N.PV_EFORMAT and "cannot open" in msg
    notfa = tmp_path / "x.fa"
    notfa.write_bytes(b"ACGT\n")
    code, msg, _ = native_open(str(notfa), [good])
    assert code == N.PV_EFORMAT and "not FASTA" in msg


def test_fasta_layout_hash_verify_case(fx, oracle_ref):
    L = N.lib()
    for ds in ("q1k", "q16k"):
        files = [os.path.join(fx["dirs"][ds], f"{nm}.{ds}.rr3") for nm in ("synthA", "synthB")]
        h = Handle(fx["ref"], files)
        for a, f in enumerate(files):
            A = O.Archive(f)
            upper = A.full(oracle_ref, apply_case=False)
            bad = ctypes.c_int64()
            assert L.pv_verify_blocks(h.h, a, upper.ctypes.data, upper.size, ctypes.byref(bad)) == 0 and bad.value == -1
            broken = upper.copy()
            broken[A.Q + 7] ^= 1
            L.pv_verify_blocks(h.h, a, broken.ctypes.data, broken.size, ctypes.byref(bad))
            assert bad.value == 1
            cased = upper.copy()
            assert L.pv_apply_case(h.h, a, 0, cased.ctypes.data, cased.size) == 0
            assert np.array_equal(cased, A.full(oracle_ref))
            part = upper[1000:60000].copy()
            L.pv_apply_case(h.h, a, 1000, part.ctypes.data, part.size)
            assert np.array_equal(part, cased[1000:60000])
            hv, err = ctypes.c_uint64(), N.errbuf()
            assert L.pv_fasta_xxh3(h.h, a, cased.ctypes.data, cased.size, ctypes.byref(hv), err, len(err)) == 0
            assert hv.value == A.fasta_xxh
            size = L.pv_fasta_size(h.h, a)
            buf = ctypes.create_string_buffer(size)
            assert L.pv_fasta_build(h.h, a, cased.ctypes.data, cased.size, buf, size, err, len(err)) == 0
            assert buf.raw == A.fasta(oracle_ref) and xxhash.xxh3_64_intdigest(buf.raw) == A.fasta_xxh
