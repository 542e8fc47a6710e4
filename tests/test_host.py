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


def native_open(ref, files, form=0):
    L = N.lib()
    arr = (ctypes.c_char_p * len(files))(*[os.fsencode(f) for f in files])
    out, err = ctypes.c_void_p(), N.errbuf()
    code = L.pv_cohort_open(os.fsencode(ref), ctypes.cast(arr, ctypes.c_void_p), len(files), 2, form, ctypes.byref(out), err, len(err))
    return code, err.value.decode(), out.value


class Handle:
    def __init__(self, ref, files, form=0):
        code, msg, h = native_open(ref, files, form)
        assert code == 0, msg
        self.h = h

    def __del__(self):
        N.lib().pv_cohort_close(self.h)


def test_exports_every_declared_symbol():
    hdr = open(os.path.join(ROOT, "include", "panvram_amd.h")).read()
    names = set(re.findall(r"^\s*(?:int32_t|int64_t|uint64_t|void)\s*\**\s*(pv_\w+)\s*\(", hdr, re.M))
    assert len(names) >= 20
    L = ctypes.CDLL(N.LIB_PATH)
    for nm in sorted(names):
        assert hasattr(L, nm), nm
    assert set(N.SIGNATURES) == names
    assert N.lib().pv_abi_version() == int(re.search(r"#define PV_ABI_VERSION (\d+)", hdr).group(1))


def test_four_byte_transforms_equal_the_per_byte_ones():
    """The decode kernels' output transforms four bytes at a time (complement, complement keeping case, token codes,
    lower-case flags) against pvc::comp / comp_case / token (reference csrc/pv_v1.h:74-76) for every byte value in
    every byte lane, compiled for the host from the kernel source."""
    assert N.lib().pv_selftest_bytes() == 0


def test_sample_call_record_reaches_its_fields():
    """pv_sample_hip_call reads pv_sample_hip's arguments from the record: the checks that run before any HIP call see
    D, W, wait, work and the error buffer at the offsets the ctypes record (the header's field order) puts them."""
    L = N.lib()
    assert L.pv_sample_hip_call(None) == N.PV_EARG
    dev = N.DevCohort()
    err = N.errbuf()
    c = N.SampleCall(D=None, n=0, W=8, wait=N.WAIT_COUNTER, err=ctypes.addressof(err), errcap=len(err))
    assert L.pv_sample_hip_call(ctypes.byref(c)) == N.PV_EARG and err.value == b"null argument"
    c.D = ctypes.addressof(dev)
    for field, value, message in (("W", 0, b"W"), ("wait", 7, b"wait mode"), ("work", 8, b"work buffer not 16-byte aligned")):
        setattr(c, field, value)
        err.value = b""
        assert L.pv_sample_hip_call(ctypes.byref(c)) == N.PV_EARG and err.value == message, field
        setattr(c, field, {"W": 8, "wait": N.WAIT_COUNTER, "work": None}[field])


def test_windows_refusals_before_launch():
    """pv_windows_hip refuses what the reference's run_windows refuses (csrc/pv_cuda.cu:119-128) before any HIP call:
    a block size outside {1024, 2048, 4096, 16384}, W outside [0, 2^31) and n * (ceil(W / Q) + 1) >= 2^31."""
    L = N.lib()
    err = N.errbuf()
    fake = ctypes.c_void_p(16)          # never dereferenced: every case returns before a launch
    for Q, n, W, message in ((8192, 1, 10, b"block size"), (1000, 1, 10, b"block size"), (4096, 1, 1 << 31, b"W"),
                             (4096, 1, -1, b"W"), (4096, -1, 10, b"n"),
                             (4096, 1 << 29, 16385, b"too many blocks in one call (windows x blocks per window >= 2^31)"),
                             (16384, 1 << 30, 1, b"too many blocks in one call (windows x blocks per window >= 2^31)")):
        dev = N.DevCohort(Q=Q)
        err.value = b""
        code = L.pv_windows_hip(ctypes.byref(dev), fake, fake, n, W, None, 0, 1, fake, fake, None, 0, None, err, len(err))
        assert code == N.PV_EARG and err.value == message, (Q, n, W)
    # the largest call below the limit passes the checks (n = 0 launches nothing)
    dev = N.DevCohort(Q=4096)
    assert L.pv_windows_hip(ctypes.byref(dev), fake, fake, 0, 8192, None, 0, 1, fake, fake, None, 0, None, err, len(err)) == N.PV_OK


def test_fetch_refusals_before_launch():
    """pv_fetch_hip refuses before its first launch: a null cohort or record, a record not 16-byte aligned, an out
    pointer missing for W > 0, and W outside [0, 2^31) (the windows entry's W check)."""
    L = N.lib()
    err = N.errbuf()
    dev = N.DevCohort(Q=4096)
    rec = ctypes.c_void_p(4096)         # never dereferenced: every case returns before a launch
    out = ctypes.c_void_p(8192)
    cases = ((None, rec, out, 10, b"null argument"), (ctypes.byref(dev), None, out, 10, b"null argument"),
             (ctypes.byref(dev), rec, None, 10, b"null argument"),
             (ctypes.byref(dev), ctypes.c_void_p(4104), out, 10, b"coordinate record not 16-byte aligned"),
             (ctypes.byref(dev), rec, out, 1 << 31, b"W"), (ctypes.byref(dev), rec, out, -1, b"W"))
    for D, r, o, W, message in cases:
        err.value = b""
        code = L.pv_fetch_hip(D, 0, 0, W, 0, 0, o, r, None, 0, None, err, len(err))
        assert code == N.PV_EARG and err.value == message, (W, message)


def test_dispatch_serialised_reads_the_profiler_environment():
    """Under rocprofv3 counter collection (its environment variables) the library reports serialised dispatch, so that
    sample's counter wait falls back to events; without them it does not."""
    import subprocess
    import sys
    code = "from panvram_amd import _native as N; print(N.lib().pv_dispatch_serialised())"
    env = {k: v for k, v in os.environ.items() if not k.startswith("ROCPROF")}
    run = lambda e: subprocess.run([sys.executable, "-c", code], env=e, cwd=ROOT, capture_output=True, text=True, check=True).stdout.strip()
    assert run(env) == "0"
    assert run({**env, "ROCPROF_COUNTER_COLLECTION": "1"}) == "1"
    assert run({**env, "ROCPROF_COUNTERS": "pmc: SQ_WAVES"}) == "1"
    assert run({**env, "ROCPROF_COUNTER_COLLECTION": "0"}) == "0"


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


def _arr(h, i, dt):
    p, n = ctypes.c_void_p(), ctypes.c_uint64()
    assert N.lib().pv_cohort_array(h.h, i, ctypes.byref(p), ctypes.byref(n)) == 0
    return np.frombuffer((ctypes.c_uint8 * n.value).from_address(p.value), dtype=dt).copy() if n.value else np.zeros(0, dt)


def _cohort(fx, wide, which):
    if which == "wide":
        return wide["ref"], wide["paths"]
    return fx["ref"], [os.path.join(fx["dirs"]["q1k"], f"{nm}.q1k.rr3") for nm in ("synthA", "synthB")]


@pytest.mark.parametrize("which", ["fixtures", "wide"])
def test_packed_reference_gives_the_reference_bytes(fx, wide, which):
    """PV_FORM_PACKED_REF: the 2-bit words with the runs of other bytes written over them give back the plain
    reference byte for byte; the runs are maximal and hold no A/C/G/T; the bucket index points at the first run ending
    after each bucket start."""
    ref, files = _cohort(fx, wide, which)
    plain, packed = Handle(ref, files), Handle(ref, files, N.FORM_PACKED_REF)
    R = _arr(plain, N.ARR_REF, np.uint8)
    assert _arr(packed, N.ARR_REF, np.uint8).size == 0
    pw = _arr(packed, N.ARR_PW, np.uint32)
    es, el, eb = _arr(packed, N.ARR_PES, np.int64), _arr(packed, N.ARR_PEL, np.int64), _arr(packed, N.ARR_PEB, np.uint8)
    ix = _arr(packed, N.ARR_PEIX, np.uint32)
    q = np.arange(R.size, dtype=np.int64)
    got = np.frombuffer(b"ACGT", np.uint8)[(pw[q >> 4] >> (2 * (q & 15)).astype(np.uint32)) & 3]
    for a, n, b in zip(es, el, eb):
        got[a:a + n] = b
    assert np.array_equal(got, R)
    assert len(es) == N.lib().pv_cohort_ref_exceptions(packed.h) > 0
    assert not np.isin(eb, np.frombuffer(b"ACGT", np.uint8)).any()
    assert (el > 0).all() and (es[1:] >= es[:-1] + el[:-1]).all()
    touching = es[1:] == es[:-1] + el[:-1]
    assert not (touching & (eb[1:] == eb[:-1])).any()
    if which == "wide":                                    # IUPAC runs, neighbouring runs of different bytes, a run across 2^22
        assert len(set(eb.tolist())) > 5 and touching.any()
        assert ((es < (1 << 22)) & (es + el > (1 << 22))).any()
    k = np.arange(ix.size, dtype=np.int64) << 16
    assert np.array_equal(ix, np.searchsorted(es + el, k, side="right"))


@pytest.mark.parametrize("which", ["fixtures", "wide"])
def test_compact_block_table_gives_the_plain_table(fx, wide, which):
    """PV_FORM_COMPACT_BLOCKS: walking each group block by block (offsets by summed lengths, starts by the format's
    prediction plus the code, or the exception table) gives the plain OFF / ST arrays; RUN0G is the plain RUN0 of each
    group's first block."""
    ref, files = _cohort(fx, wide, which)
    plain, comp = Handle(ref, files), Handle(ref, files, N.FORM_COMPACT_BLOCKS)
    L = N.lib()
    Q = L.pv_cohort_block_size(plain.h)
    off, st, run0 = _arr(plain, N.ARR_OFF, np.uint32), _arr(plain, N.ARR_ST, np.int64), _arr(plain, N.ARR_RUN0, np.uint32)
    for i in (N.ARR_OFF, N.ARR_ST, N.ARR_RUN0):
        assert _arr(comp, i, np.uint8).size == 0
    asm, asm2 = _arr(plain, N.ARR_ASM, np.int64).reshape(-1, 8), _arr(comp, N.ARR_ASM, np.int64).reshape(-1, 8)
    assert np.array_equal(asm[:, :5], asm2[:, :5])
    go, gs, r0g = _arr(comp, N.ARR_GRP_OFF, np.int64), _arr(comp, N.ARR_GRP_ST, np.int64), _arr(comp, N.ARR_RUN0G, np.uint32)
    blen, code = _arr(comp, N.ARR_BLEN, np.uint16), _arr(comp, N.ARR_BCODE, np.int16)
    eb, est = _arr(comp, N.ARR_EXC_B, np.int64), _arr(comp, N.ARR_EXC_ST, np.int64)
    assert len(eb) == L.pv_cohort_block_exceptions(comp.h) == int((code == -32768).sum())
    if which == "wide":
        assert len(eb) > 0
    for a in range(len(files)):
        x = N.AsmInfo()
        L.pv_asm_info_get(plain.h, a, ctypes.byref(x))
        bb, g0 = int(asm2[a, 1]), int(asm2[a, 5])
        o = s = 0
        for b in range(x.blocks):
            if b % 32 == 0:
                g = g0 + b // 32
                o, s = int(go[g]), int(gs[g])
                assert r0g[g] == run0[bb + b]
            else:
                o += int(blen[bb + b - 1])
                c = int(code[bb + b])
                if c == -32768:
                    j = int(np.searchsorted(eb, bb + b))
                    assert eb[j] == bb + b
                    s = int(est[j])
                else:
                    pc = s >> 1
                    pred = pc - Q if s & 1 else pc + Q
                    s = ((pred + (c >> 1)) << 1) | (c & 1)
            assert o == off[bb + b] and s == st[bb + b], (a, b)
            assert blen[bb + b] == off[bb + b + 1] - off[bb + b]


def test_unknown_form_bits(fx):
    code, msg, _ = native_open(fx["ref"], [os.path.join(fx["dirs"]["q1k"], "synthA.q1k.rr3")], 4)
    assert code == N.PV_EARG and "form" in msg


def _direct_lookup(ent, row, slot):
    """What the one-lane-per-block decoder does with a bucket entry (layout in pv_codec.h): (symbol, lo, freq), or None
    for a failed lookup."""
    e = int(ent)
    s0, lo0 = e & 127, (e >> 7) & 0xFFF
    e1, e2, e3 = (e >> 19) & 0xFFF, (e >> 31) & 0xFFF, (e >> 43) & 0xFFF
    if s0 >= 104:
        return None
    if slot <= e3:
        i1, i2 = int(slot > e1), int(slot > e2)
        lo = e2 + 1 if i2 else e1 + 1 if i1 else lo0
        return s0 + i1 + i2, lo, (e3 if i2 else e2 if i1 else e1) + 1 - lo
    s, lo, hi = s0 + 3, e3 + 1, int(row[s0 + 4])
    while hi <= slot and s < 103:
        s, lo, hi = s + 1, hi, int(row[s + 2])
    return None if hi - lo == 0 or slot < lo else (s, lo, hi - lo)


@pytest.mark.parametrize("ds", ["q1k", "q16k"])
def test_big_context_bucket_entries(fx, ds):
    """Every slot of every big-alphabet context, looked up through its bucket entry (one load on the device) and the
    row fallback, gives the symbol and range that a search of the cumulative row gives - the symbol the reference's
    4096-entry table holds for that slot - and an all-zero context fails every slot."""
    files = [os.path.join(fx["dirs"][ds], f"{nm}.{ds}.rr3") for nm in ("synthA", "synthB")]
    h = Handle(fx["ref"], files)
    p, n = ctypes.c_void_p(), ctypes.c_uint64()
    assert N.lib().pv_cohort_array(h.h, N.ARR_TAB, ctypes.byref(p), ctypes.byref(n)) == 0
    tab = np.frombuffer((ctypes.c_uint8 * n.value).from_address(p.value), dtype=np.uint8).copy()
    GT, SMALL, BIGROW, NB, OFF = 10240, 736, 112, 32, 6144
    assert n.value == GT * len(files)
    slots = np.arange(4096)
    nonempty = 0
    for a in range(len(files)):
        t = tab[a * GT:(a + 1) * GT]
        rows = t[SMALL:SMALL + 15 * BIGROW * 2].view(np.uint16).reshape(15, BIGROW)
        ents = t[OFF:OFF + 15 * NB * 8].view(np.uint64).reshape(15, NB)
        for k in range(15):
            row = rows[k, :105].astype(np.int64)
            if row[104] == 0:
                assert all(_direct_lookup(ents[k, j], row, j * 128) is None for j in range(NB))
                continue
            nonempty += 1
            want_s = np.searchsorted(row[1:], slots, side="right")
            for slot in range(4096):
                s = int(want_s[slot])
                assert _direct_lookup(ents[k, slot // 128], row, slot) == (s, int(row[s]), int(row[s + 1] - row[s])), (a, k, slot)
    assert nonempty >= 10


def test_stream_ops_use_private_bindings_only_where_checked():
    """panvram_amd._streams picks torch's private stream bindings only on a checked torch version that has them, and
    the public calls otherwise (no GPU needed: the choice, not the calls)."""
    from panvram_amd import _streams as S

    class Fake:
        @staticmethod
        def _cuda_getCurrentStream(i):
            return (0, i, 1)

        @staticmethod
        def _cuda_setStream(a, b, c):
            return None

    on = S.StreamOps(version=S.CHECKED[0] + "0+rocm7.0", module=Fake)
    assert on.private and on.get == on._first_get and on.set == on._first_set
    for version, module in (("2.9.1", Fake), ("3.0.0", Fake), (S.CHECKED[0] + "0", object())):
        off = S.StreamOps(version=version, module=module)
        assert not off.private and off.get is S._public_get and off.set is S._public_set


def test_ring_size_follows_the_hardware_queues(monkeypatch):
    """sample's ring: one stream per hardware queue HIP gives the process besides the caller's (GPU_MAX_HW_QUEUES,
    HIP's default 4), 1 to 15; streams are picked by measuring only up to 8 queues (no GPU needed: the sizes)."""
    from panvram_amd import cohort as C
    for env, queues, ring in ((None, 4, 3), ("4", 4, 3), ("2", 2, 1), ("1", 1, 1), ("24", 24, 15), ("64", 64, 15), ("x", 4, 3)):
        if env is None:
            monkeypatch.delenv("GPU_MAX_HW_QUEUES", raising=False)
        else:
            monkeypatch.setenv("GPU_MAX_HW_QUEUES", env)
        assert C._hw_queues() == queues and C._ring_size() == ring, env
    assert C._PICK_QUEUES == 8
