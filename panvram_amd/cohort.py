"""The resident cohort: refrel3 v1 archives of many assemblies, encoded against one reference, held in MI355X memory and
decoded there by the HIP kernels of libpanvram_amd.so.

`Cohort` is a drop-in for the reference's `panvram.Cohort` (reference panvram/cohort.py:21-234). It has the same
constructor (`Cohort.open`), methods, argument meanings, return types and exception types, so a caller switches by
changing the import. Where it differs, on purpose:

- The path decodes on the GPU only. This package has no CPU decoder; the repository's CPU decoder is the test oracle
  under oracle/.
- `sample` makes the same two torch draws (randint, then rand for a strand probability) and turns them into window
  coordinates in one HIP kernel instead of a chain of torch ops. The number of valid starts per window length is read
  back once per length, not on every call.
- `fasta()` decodes on the GPU as well. The block and FASTA hashes are then checked on the host, as the reference's
  CPU `fasta(verify=True)` checks them.
"""
import ctypes
import glob
import os
import re
import threading

import torch
from torch.utils.dlpack import from_dlpack as _from_dlpack

from . import _native as N
from ._streams import ops as _streams

DATASETS = ("q4k", "q16k")

# Every device array gets this many zero bytes after its end: the decode kernel reads payloads and tables in 16-byte
# chunks and may touch up to 1 KiB past the last byte it uses.
_TAIL = 1024

# pooled arrays: (key, C-ABI id, element type, free the host copy after upload)
_POOLS = (("P", N.ARR_P, torch.uint8, True), ("off", N.ARR_OFF, torch.int32, True), ("st", N.ARR_ST, torch.int64, True),
          ("run0", N.ARR_RUN0, torch.int32, True), ("tab", N.ARR_TAB, torch.uint8, True), ("asm", N.ARR_ASM, torch.int64, False),
          ("low_s", N.ARR_LOW_S, torch.int64, False), ("low_l", N.ARR_LOW_L, torch.int64, False), ("ref", N.ARR_REF, torch.uint8, True),
          ("ctg_asm", N.ARR_CTG_ASM, torch.int64, False), ("ctg_local", N.ARR_CTG_LOCAL, torch.int64, False),
          ("ctg_boff", N.ARR_CTG_BOFF, torch.int64, False), ("ctg_len", N.ARR_CTG_LEN, torch.int64, False),
          ("pw", N.ARR_PW, torch.int32, True), ("pes", N.ARR_PES, torch.int64, False), ("pel", N.ARR_PEL, torch.int64, False),
          ("peb", N.ARR_PEB, torch.uint8, False), ("peix", N.ARR_PEIX, torch.int32, False),
          ("grp_off", N.ARR_GRP_OFF, torch.int64, True), ("grp_st", N.ARR_GRP_ST, torch.int64, True),
          ("run0g", N.ARR_RUN0G, torch.int32, True), ("blen", N.ARR_BLEN, torch.int16, True), ("bcode", N.ARR_BCODE, torch.int16, True),
          ("exc_b", N.ARR_EXC_B, torch.int64, False), ("exc_st", N.ARR_EXC_ST, torch.int64, False))

_STATUS_TEXT = "1 corrupt block, 4 bounded wait expired, 8 window outside an assembly"


def _archive_files(path, dataset, assemblies):
    """(names, files) of the cohort directory: *.<dataset>.rr3 sorted by file name, or the named subset in that order."""
    if dataset is not None and not re.fullmatch(r"q\d+k", dataset):
        raise ValueError(f"dataset: one of {DATASETS} (or another q<N>k suffix), or None for every *.rr3")
    ext = f".{dataset}.rr3" if dataset else ".rr3"
    found = {os.path.basename(f)[: -len(ext)]: f for f in glob.glob(os.path.join(path, "*" + ext))}
    if assemblies is None:
        names = sorted(found, key=lambda nm: found[nm])
    else:
        names = [str(a) for a in assemblies]
        absent = [a for a in names if a not in found]
        if absent:
            raise FileNotFoundError(f"not in {path}: {absent[:5]}")
    if not names:
        raise FileNotFoundError(f"no *{ext} in {path}")
    return names, [found[nm] for nm in names]


def _reference_file(path, first_archive, reference):
    """The reference FASTA: the argument, else <path>/reference.fa, else the file the first archive's header names
    (the name after the 136-byte fixed header, format offset 136)."""
    if reference is None:
        reference = os.path.join(path, "reference.fa")
        if not os.path.exists(reference):
            with open(first_archive, "rb") as f:
                head = f.read(138 + 65535)
            k = int.from_bytes(head[136:138], "little")
            reference = os.path.join(path, head[138:138 + k].decode())
    if not os.path.exists(reference):
        raise FileNotFoundError(f"reference {reference} not found (pass reference=)")
    return reference


def _gpu(device):
    """The torch device to decode on: a gfx950 GPU, else an error naming what was found."""
    device = torch.device(device)
    if device.type != "cuda":
        raise RuntimeError("panvram_amd decodes on the GPU only (device 'cuda' or 'cuda:N'); the CPU decoder of this "
                           "repository is its test oracle (oracle/), not part of the package")
    if device.index is None:
        device = torch.device("cuda", torch.cuda.current_device())
    arch = getattr(torch.cuda.get_device_properties(device), "gcnArchName", "") or ""
    if not arch.startswith("gfx950"):
        raise RuntimeError(f"panvram_amd is built for gfx950 (MI355X); {torch.cuda.get_device_name(device)} is {arch or 'unknown'}")
    return device


def _hw_queues():
    """The hardware queues HIP gives this process: GPU_MAX_HW_QUEUES, HIP's default 4."""
    try:
        return int(os.environ.get("GPU_MAX_HW_QUEUES", "4"))
    except ValueError:
        return 4


def _ring_size():
    """Streams for `sample`'s ring: the process's hardware queues minus the caller's, at most 15."""
    return max(1, min(15, _hw_queues() - 1))


# At most this many hardware queues, `sample` picks its ring streams by measuring (Cohort._make_ring); above it, it
# takes torch's pool streams as they come.
_PICK_QUEUES = 8


_PLAIN = (bool, int, float, type(None))

# With a ring, `sample` allocates its rows on one stream of its own that runs no work (the row stream), with
# record_stream(caller): a freed row is reused once the caller's stream has passed the point of the free, which comes
# after its wait for the call that wrote the row, so any ring stream may write it next. pv_sample_hip keeps at most 32
# calls per caller stream ahead of that stream: a call's rows are allocated before its own wait for room, so up to 33
# rows are pending (one more while the free after the oldest is being passed), plus one being allocated. The first
# call of a shape allocates and frees 40 rows (within a byte budget) so that later calls find them in the row stream's
# pool of torch's caching allocator instead of opening new segments (a device allocation each).
_PREWARM_ROWS, _PREWARM_BYTES = 40, 512 << 20
# rows of sample's own pool per row size: enough for the calls a caller's stream may have in flight (32) and the ring's,
# and a few held by the caller; at most _POOL_BYTES of them
_POOL_ROWS, _POOL_BYTES = 64, 2 << 30
_capsule = ctypes.pythonapi.PyCapsule_New
_capsule.restype = ctypes.py_object
_capsule.argtypes = [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_void_p]


def _rc_mode(reverse_complement):
    """(mode, p) of `sample`'s reverse_complement, as the reference reads it (panvram/cohort.py:182-189): True -> every
    window, no draw (1); False, None or 0 -> none (0); any other number p in (0, 1] -> torch.rand(n) < p (2; 1 and 1.0
    draw too)."""
    if reverse_complement is True:
        return 1, 1.0
    if reverse_complement is None or reverse_complement is False or reverse_complement == 0:
        return 0, 0.0
    p = float(reverse_complement)
    if not 0 < p <= 1:
        raise ValueError("reverse_complement: True, False or a probability in (0, 1]")
    return 2, p


class _SamplePlan:
    """What repeated `Cohort.sample` calls of one shape on one caller stream and ring position share: the lane stream,
    views of the draws, uniform numbers and status in the lane's work buffer, and pv_sample_hip's argument record, of
    which only the output pointers change per call."""
    __slots__ = ("lane", "caller", "lane_id", "caller_id", "row_id", "shape", "dev", "coords", "draws", "rnd", "status", "total",
                 "call", "ref", "fn", "err", "buf", "check", "pool", "take", "cpool", "ids", "bits", "dtype")

    def __init__(self, cohort, lane, caller, shape, coords, draws, rnd, status, total, call, buf, rows=None, pool=None,
                 cpool=None, ids=None):
        self.lane, self.caller, self.shape, self.dev, self.coords = lane, caller, shape, cohort.device, coords
        self.lane_id = (lane.stream_id, lane.device_index, lane.device_type) if lane is not None else None
        self.caller_id = (caller.stream_id, caller.device_index, caller.device_type)
        self.row_id = (rows.stream_id, rows.device_index, rows.device_type) if rows is not None else None
        self.draws, self.rnd, self.status, self.total, self.buf = draws, rnd, status, total, buf
        self.call, self.ref, self.fn, self.err = call, ctypes.byref(call), N.lib().pv_sample_hip_call, cohort._err
        self.check = cohort._check
        self.pool, self.take, self.cpool = pool, N.lib().pv_rows_take, cpool
        # with token ids the rows are int64 ids; `ids` (int64 [5] on the device) is kept alive for the call record
        self.ids, self.bits, self.dtype = ids, 8 if ids is None else 64, torch.uint8 if ids is None else torch.int64

    def run(self, generator, check):
        lane, setter = self.lane, _streams.set
        coords = out = None
        if self.pool is not None:
            # a row of the library's pool (reused once the caller's stream has passed the next call's wait after torch
            # frees it), so the caller's queue needs no allocator event for it
            p = self.take(self.pool, self.caller.cuda_stream, self.shape[0], self.shape[1], self.bits)
            if p:
                out = _from_dlpack(_capsule(p, b"dltensor", None))
        pooled = out is not None
        if self.cpool is not None:         # coords [n, 4] int64 likewise, from a pool of 32 n-byte rows
            p = self.take(self.cpool, self.caller.cuda_stream, self.shape[0], 4, 64)
            if p:
                coords = _from_dlpack(_capsule(p, b"dltensor", None))
        cpooled = coords is not None
        if lane is not None:
            setter(*self.row_id)
        try:
            # else the row stream's memory, used by the caller (record_stream below): a block the caller frees is reused
            # once the caller has passed the point of the free. Caller-stream memory would not do: its next owner could
            # be a ring stream, whose writes are not ordered after the caller's pending reads of the old contents.
            if out is None:
                out = torch.empty(self.shape, dtype=self.dtype, device=self.dev)
            if self.coords and coords is None:
                coords = torch.empty((self.shape[0], 4), dtype=torch.int64, device=self.dev)
            if lane is not None:
                setter(*self.lane_id)
            # the reference's torch.randint(0, total, (n,)) and torch.rand(n), drawn into the work buffer: randint and
            # rand fill their output with random_(0, total) and uniform_(0, 1), the same draws from the same generator
            self.draws.random_(0, self.total, generator=generator)
            if self.rnd is not None:
                self.rnd.uniform_(0, 1, generator=generator)
        finally:
            if lane is not None:
                setter(*self.caller_id)
        c = self.call
        c.out = out.data_ptr()
        if coords is not None:
            c.coords = coords.data_ptr()
        code = self.fn(self.ref)
        if code:
            N.raise_for(code, self.err)
        if lane is not None:
            if not pooled:
                out.record_stream(self.caller)
            if coords is not None and not cpooled:
                coords.record_stream(self.caller)
        if check:
            self.check(self.status)
        return (out, coords) if self.coords else out


def _host_bytes(ptr, nbytes):
    if not nbytes:
        return torch.empty(0, dtype=torch.uint8)
    return torch.frombuffer((ctypes.c_uint8 * nbytes).from_address(ptr), dtype=torch.uint8)


class Cohort:
    """A cohort resident on one GPU. Build it with `Cohort.open(directory, device=...)`.

    Positions are 0-based. An assembly is addressed by its name (the archive's file name without .<dataset>.rr3) or
    its index. A contig is addressed by its name (the FASTA header up to the first space or tab) or its index within
    the assembly."""

    @classmethod
    def open(cls, path, device="cuda", dataset="q4k", reference=None, threads=0, assemblies=None,
             packed_reference=False, compact_blocks=False):
        """Read every archive of one block size in directory `path` (`dataset` "q4k", "q16k", ..., or None for all
        *.rr3; `assemblies`: only these names, in this order) and their reference (`reference`, else
        path/reference.fa, else the file their header names). Each file passes all of the format's checks before
        anything is decoded: header hash, reference SHA-256 and length, sections, tables. The pooled arrays then move
        to `device` once. threads: host threads for reading (0 = all). packed_reference: hold the reference as 2 bits
        per base plus runs of other bytes; compact_blocks: hold the block table as groups of 32 blocks with 4 bytes
        per block (refused for block payloads over 65535 bytes). Both give the same windows from fewer resident
        bytes. (reference panvram/cohort.py:43-84)"""
        names, files = _archive_files(path, dataset, assemblies)
        reference = _reference_file(path, files[0], reference)
        device = _gpu(device)
        handle, err = ctypes.c_void_p(), N.errbuf()
        argv = (ctypes.c_char_p * len(files))(*[os.fsencode(f) for f in files])
        form = (N.FORM_PACKED_REF if packed_reference else 0) | (N.FORM_COMPACT_BLOCKS if compact_blocks else 0)
        code = N.lib().pv_cohort_open(os.fsencode(reference), ctypes.cast(argv, ctypes.c_void_p), len(files), int(threads), form,
                                      ctypes.byref(handle), err, len(err))
        if code:
            N.raise_for(code, err)
        return cls(handle.value, names, device)

    def __init__(self, handle, names, device):
        L = N.lib()
        self._h, self._close = handle, L.pv_cohort_close     # the close function is kept for __del__ at interpreter exit
        self.names, self.device = list(names), torch.device(device)
        self._by_name = {nm: i for i, nm in enumerate(self.names)}
        self._Q = int(L.pv_cohort_block_size(handle))
        self._ref_n = int(L.pv_cohort_ref_bases(handle))
        hexsha = ctypes.create_string_buffer(65)
        L.pv_cohort_ref_sha256(handle, hexsha)
        self._sha = hexsha.value.decode()
        self._meta = [self._load_info(i) for i in range(int(L.pv_cohort_assemblies(handle)))]
        self._ctgs = [self._load_contigs(i) for i in range(len(self._meta))]
        self._ctg_index = [{c[0]: k for k, c in enumerate(cs)} for cs in self._ctgs]
        self._upload()
        self._starts = {}             # W -> (per-contig running count of valid window starts, total)
        # a list: (start, mid, end) torch.cuda.Events around decode launches are appended; for `sample`, mid lies between
        # the decode kernel and the windows (replay and write-out) kernel, for `windows` it is None
        self.kernel_events = None
        self.kernel_events_every = 1  # sample(): bracket one launch in this many (the events add work to the stream)
        # sample(): True - the events split a launch into its decode kernels (start to mid) and its windows kernel (mid
        # to end), which keeps a large call's kernels one after another; False - (start, None, end) around the whole
        # call, which runs as an untimed call does (a large call's replay beside its heavy waves)
        self.kernel_events_split = True
        # how the caller's stream waits for a ring stream: "counter" (a counter per ring stream in signal memory, ~7 us
        # of host time per call; the runtime polls for it with a small kernel on the caller's queue, so under a tool
        # that serialises dispatches, such as rocprofv3 --pmc, the library waits with events instead), or "event" (HIP
        # events, ~16-20 us)
        self.sample_wait = "counter"
        # decode blocks with short payloads one lane per block first (the windows kernel then only replays them);
        # False: every block in the windows kernel. The bytes are the same either way.
        self.light_decode = True
        self._launches = 0
        # `sample` runs on a ring of this many streams of its own (0: on the caller's stream). It reads no caller
        # tensor, so consecutive calls need not wait for each other: one call's long serial blocks overlap the next
        # calls' work. The caller's stream waits for each call's results before anything it enqueues after the call.
        # One stream per hardware queue HIP gives the process (GPU_MAX_HW_QUEUES, default 4) besides the caller's:
        # two ring streams on one queue would serialise.
        self.sample_streams = _ring_size()
        self._ring, self._turn = [], 0
        self._callers = {}            # (stream id, device, type) -> torch Stream of a caller's current stream
        self._sample_args = {}        # W -> the constant pointer arguments of pv_sample_hip
        self._work_bytes = {}         # (n, W, light) -> bytes of pv_sample_hip's work
        # per stream: the device buffer its decode calls use for work, draws and status. Calls on one stream run in
        # order, so each reuses the buffer of the one before (no allocation per call); grown when a call needs more.
        self._stream_work = {}
        self._views = {}              # (stream, buffer, n, work bytes, rc mode) -> views of draws, uniforms, status
        self._err = N.errbuf()        # the C calls' error text (written only on failure)
        self._idx = self.device.index
        self._fast = {}               # (arguments, caller stream, ring position, ...) -> _SamplePlan
        self._prepared = set()        # (lane stream, caller stream, wait mode) whose wait state exists
        self._rows = None             # the stream sample allocates its rows on with a ring
        self._plans = {}              # assembly -> FASTA layout plan (check_full)
        self._aux = None              # the stream check_full and decode() decode on
        self._aux2 = None             # the two streams decode() copies to the host on
        self._local = threading.local()   # per thread: fetch()'s 32-byte coordinate record on the device

    def _upload(self):
        L = N.lib()
        self._pool = {}
        for key, aid, dtype, release in _POOLS:
            ptr, nb = ctypes.c_void_p(), ctypes.c_uint64()
            if L.pv_cohort_array(self._h, aid, ctypes.byref(ptr), ctypes.byref(nb)):
                raise RuntimeError(f"pooled array {key} unavailable")
            nb = nb.value
            buf = torch.zeros(nb + _TAIL, dtype=torch.uint8, device=self.device)
            if nb:
                buf[:nb].copy_(_host_bytes(ptr.value, nb))
            self._pool[key] = (buf, nb, dtype)
            if release:
                L.pv_cohort_release_array(self._h, aid)      # the device copy is the only one used from here on
        torch.cuda.synchronize(self.device)
        D = N.DevCohort()
        for field, key in (("P", "P"), ("off", "off"), ("st", "st"), ("run0", "run0"), ("tab", "tab"), ("asm_rec", "asm"),
                           ("low_s", "low_s"), ("low_l", "low_l"), ("ref", "ref"), ("pw", "pw"), ("pes", "pes"), ("pel", "pel"),
                           ("peb", "peb"), ("peix", "peix"), ("grp_off", "grp_off"), ("grp_st", "grp_st"), ("run0g", "run0g"),
                           ("blen", "blen"), ("bcode", "bcode"), ("exc_b", "exc_b"), ("exc_st", "exc_st")):
            setattr(D, field, self._pool[key][0].data_ptr())
        D.ref_n, D.nasm, D.Q = self._ref_n, len(self._meta), self._Q
        D.form = int(L.pv_cohort_form(self._h))
        D.pne, D.nexc = int(L.pv_cohort_ref_exceptions(self._h)), int(L.pv_cohort_block_exceptions(self._h))
        self._D = D
        self._Dref = ctypes.byref(D)
        self._ctg = {k: self._array(k) for k in ("ctg_asm", "ctg_local", "ctg_boff", "ctg_len")}

    def _array(self, key):
        buf, nb, dtype = self._pool[key]
        return buf[:nb].view(dtype)

    def __del__(self):
        h, close = getattr(self, "_h", None), getattr(self, "_close", None)
        if h and close is not None:
            close(h)
            self._h = None

    # ------------------------------------------------------------------ what the cohort holds
    def _load_info(self, a):
        x = N.AsmInfo()
        if N.lib().pv_asm_info_get(self._h, a, ctypes.byref(x)):
            raise IndexError(f"assembly index {a}")
        return {"path": x.path.decode(), "Q": x.Q, "bases": x.bases, "blocks": x.blocks, "file_bytes": x.file_bytes,
                "payload_bytes": x.payload_bytes, "block_hashes": bool(x.block_hashes), "fasta_xxh3": f"{x.fasta_xxh3:016x}",
                "bases_xxh3": f"{x.bases_xxh3:016x}",
                "contigs": x.contigs, "lower_case_runs": x.lower_case_runs, "reference_name": x.reference_name.decode()}

    def _load_contigs(self, a):
        L, rows = N.lib(), []
        nm, hd = ctypes.c_char_p(), ctypes.c_char_p()
        ln, off, lw = ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint32()
        while L.pv_asm_contig(self._h, a, len(rows), ctypes.byref(nm), ctypes.byref(hd), ctypes.byref(ln), ctypes.byref(off),
                              ctypes.byref(lw)) == 0:
            rows.append((nm.value.decode(), hd.value.decode(), ln.value, off.value, lw.value))
        return rows

    def __len__(self):
        return len(self.names)

    @property
    def block_size(self):
        return self._Q

    @property
    def reference_sha256(self):
        return self._sha

    @property
    def packed_reference(self):
        return bool(self._D.form & N.FORM_PACKED_REF)

    @property
    def compact_blocks(self):
        return bool(self._D.form & N.FORM_COMPACT_BLOCKS)

    def info(self, assembly):
        """Header facts of one assembly's archive (path, Q, bases, blocks, sizes, hashes, contig and case-run counts)."""
        return dict(self._meta[self._asm(assembly)])

    def contigs(self, assembly):
        """One tuple per contig of the assembly: (name, FASTA header, length, offset in the base stream, line width)."""
        return list(self._ctgs[self._asm(assembly)])

    def resident_bytes(self):
        """Device bytes per pooled array (reference included; contig tables left out) and their total."""
        out = {k: nb for k, (_, nb, _) in self._pool.items() if not k.startswith("ctg_")}
        out["total"] = sum(out.values())
        return out

    def _asm(self, a):
        if isinstance(a, str):
            try:
                return self._by_name[a]
            except KeyError:
                raise KeyError(f"no assembly {a}") from None
        i = int(a)
        if i < 0 or i >= len(self.names):
            raise IndexError(f"assembly index {i}")
        return i

    def _contig(self, a, c):
        if isinstance(c, str):
            k = self._ctg_index[a].get(c)
            if k is None:
                raise KeyError(f"no contig {c} in {self.names[a]}")
            return k
        k = int(c)
        if k < 0 or k >= len(self._ctgs[a]):
            raise IndexError(f"contig index {k}")
        return k

    # ------------------------------------------------------------------ decoding
    def _token_ids(self, token_ids):
        """token_ids (5 ints, or an int64 tensor [5]) -> an int64 tensor [5] on the cohort's device."""
        ids = torch.as_tensor(token_ids, dtype=torch.int64).reshape(-1)
        if ids.numel() != 5:
            raise ValueError("token_ids: five ids, for the tokens A/a C/c G/g T/t and anything else")
        return ids.to(self.device).contiguous()

    def _decode(self, asm, start, W, rc, tokens, apply_case, ids=None):
        """Launch the decode of windows (asm[i], start[i], W) on the current stream -> (out [n, W], status): uint8, or
        int64 token ids when `ids` (int64 [5] on the device) is given."""
        if W < 0 or W >= (1 << 31):
            raise RuntimeError("W")
        dev = self.device
        asm, start = torch.as_tensor(asm), torch.as_tensor(start)
        n = asm.numel()
        if start.numel() != n:
            raise RuntimeError("assembly and start counts differ")
        # the C entry's refusal, made before anything of that size is allocated (reference csrc/pv_cuda.cu:128)
        if n * ((W + self._Q - 1) // self._Q + 1) >= (1 << 31) and W > 0:
            raise RuntimeError("too many blocks in one call (windows x blocks per window >= 2^31)")
        asm = asm.to(dev, torch.int64).contiguous()
        start = start.to(dev, torch.int64).contiguous()
        if rc is not None:
            rc = torch.as_tensor(rc).to(dev, torch.uint8).contiguous()
            if rc.numel() != n:
                raise RuntimeError("reverse_complement mask size")
        out = torch.empty((n, W), dtype=torch.int64 if ids is not None else torch.uint8, device=dev)
        status = torch.zeros(1, dtype=torch.int32, device=dev)
        self._windows_into(asm, start, W, rc, tokens, apply_case, out, status, ids)
        return out, status

    def _stream_buffer(self, key, nbytes):
        """The work buffer of the stream with handle `key` (the current stream), at least nbytes."""
        buf = self._stream_work.get(key)
        if buf is None or buf.numel() < nbytes:
            if len(self._stream_work) >= 64:
                self._stream_work.clear()
                self._views.clear()
                self._fast.clear()
            self._views = {k: v for k, v in self._views.items() if k[0] != key}   # views of the buffer replaced
            if buf is not None:         # plans on the replaced buffer would keep it alive
                self._fast = {k: v for k, v in self._fast.items() if v.buf is not buf}
            buf = self._stream_work[key] = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
        return buf

    def _windows_into(self, asm, start, W, rc, tokens, apply_case, out, status, ids=None):
        err, ev = N.errbuf(), self.kernel_events
        with torch.cuda.device(self.device):
            stream = torch.cuda.current_stream(self.device).cuda_stream
            wb = int(N.lib().pv_windows_work_bytes(ctypes.byref(self._D), asm.numel(), W)) if self.light_decode else 0
            wp = self._stream_buffer(stream, wb).data_ptr() if wb else None
            if ev is not None:
                t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                t0.record()
            rcp = rc.data_ptr() if rc is not None else None
            if ids is not None:
                code = N.lib().pv_windows_ids_hip(ctypes.byref(self._D), asm.data_ptr(), start.data_ptr(), asm.numel(), W, rcp,
                                                  ids.data_ptr(), out.data_ptr(), status.data_ptr(), wp, wb, stream, err, len(err))
            else:
                code = N.lib().pv_windows_hip(ctypes.byref(self._D), asm.data_ptr(), start.data_ptr(), asm.numel(), W, rcp,
                                              int(bool(tokens)), int(bool(apply_case)), out.data_ptr(), status.data_ptr(), wp, wb,
                                              stream, err, len(err))
            if ev is not None:
                t1.record()
                ev.append((t0, None, t1))
        if code:
            N.raise_for(code, err)

    @staticmethod
    def _check(status):
        s = int(status.item())
        if s:
            raise RuntimeError(f"GPU decode failed (status {s}: {_STATUS_TEXT})")

    def windows(self, asm, start, W, reverse_complement=None, tokens=False, check=True, token_ids=None):
        """Window i = bases [start[i], start[i] + W) of assembly asm[i], where start counts from the beginning of the
        assembly's base stream (its contigs back to back, in file order), so a window may run across contigs.
        Returns uint8 [n, W] on the cohort's device: the FASTA's bytes with their case, or with tokens=True the codes
        A/a 0, C/c 1, G/g 2, T/t 3, anything else 4. reverse_complement: None or a bool tensor [n] choosing the
        windows to reverse-complement. check: wait for the decode and raise RuntimeError if any block failed (one
        device sync). token_ids (not in the reference's signature): five ids; the windows come back as int64 [n, W]
        with token t stored as token_ids[t] - the id lookup a training loader applies, fused into the decode.
        (reference panvram/cohort.py:134-157)"""
        ids = self._token_ids(token_ids) if token_ids is not None else None
        out, status = self._decode(asm, start, int(W), reverse_complement, tokens, True, ids)
        if check:
            self._check(status)
        return out

    def _start_table(self, W):
        """Running count over contigs of the valid starts of a W-base window (max(0, length - W + 1) per contig), and
        its total; read back once per W."""
        t = self._starts.get(W)
        if t is None:
            room = (self._ctg["ctg_len"] - (W - 1)).clamp_min(0)
            running = torch.cumsum(room, 0)
            t = (running, int(running[-1].item()) if running.numel() else 0)
            self._starts[W] = t
        return t

    def sample(self, n, W, generator=None, reverse_complement=False, tokens=False, return_coords=False, check=True, token_ids=None):
        """n random windows of W bases, each equally likely among all (assembly, contig, start) with start + W <= the
        contig's length, so no window crosses contigs. Returns uint8 [n, W] on the cohort's device, plus with
        return_coords an int64 [n, 4] tensor of (assembly, contig index, start within the contig, reverse-complemented).
        generator: a torch.Generator, whose device draws the numbers. reverse_complement: True (every window), False, or
        a probability p per window. The draws are the reference's: torch.randint(0, total, (n,)) and, for a
        probability, torch.rand(n) < p, in that order on the same generator. token_ids: as for `windows`.
        (reference panvram/cohort.py:159-194)"""
        # The first call of a shape (arguments, caller stream, generator device) sets up every stream of the ring for it
        # - its work buffer, the views of the draws and status in it, its caller-wait counter, a warm row pool, and
        # pv_sample_hip's argument record - so that this and later calls only draw, allocate their rows and make one C
        # call, with no device allocation or synchronisation.
        timed = False
        if self.kernel_events is not None:          # events bracket one call in kernel_events_every
            self._launches += 1
            timed = self._launches % max(1, int(self.kernel_events_every)) == 0
        ikey = None
        if token_ids is not None and token_ids.__class__ in (tuple, list) and all(i.__class__ is int for i in token_ids):
            ikey = tuple(token_ids)     # plain ids: a plan of their own
        if (token_ids is None or ikey is not None) and not timed and reverse_complement.__class__ in _PLAIN:
            k = self.sample_streams
            t = -1
            if k > 0:
                t = self._turn + 1
                if t >= k:
                    t = 0
            sid = _streams.get(self._idx)
            gdev = None if generator is None else generator.device
            if gdev is not None and gdev.index is None and gdev.type == "cuda":   # torch.Generator(device="cuda")
                gdev = torch.device("cuda", torch.cuda.current_device())
            # True and 1 (or 1.0) compare equal but draw differently: the key keeps them apart
            key = (n, W, reverse_complement.__class__ is bool, reverse_complement, tokens, return_coords, sid, t, k, self.sample_wait,
                   self.light_decode, gdev, ikey)
            P = self._fast.get(key)
            if P is None and n > 0 and (gdev is None or gdev == self.device) and torch.cuda.current_device() == self._idx:
                self._prepare_shape(key, int(n), int(W), reverse_complement, bool(tokens), bool(return_coords), sid, k, ikey)
                P = self._fast.get(key)
            if P is not None and torch.cuda.current_device() == self._idx:
                if t >= 0:
                    self._turn = t
                return P.run(generator, check)
        n, W = int(n), int(W)
        if W <= 0 or n < 0:
            raise ValueError("W must be positive, n non-negative")
        running, total = self._start_table(W)
        if total == 0:
            raise ValueError(f"no contig of {W} bases or more")
        mode, p = _rc_mode(reverse_complement)
        if self.sample_wait not in ("event", "counter"):
            raise ValueError('sample_wait: "event" or "counter"')
        dev, idx = self.device, self.device.index
        caller = self._caller(_streams.get(idx))
        lane = self._sample_stream() or caller
        ids = self._token_ids(token_ids) if token_ids is not None else None
        # what the call returns, allocated per call: out [n, W] (and coords [n, 4]); what it only uses, in its stream's
        # work buffer: work (assembly, start, strand per window, then the decode kernel's scratch), the draws (int64 n,
        # float32 n), status
        wb, o_draws, o_rnd, o_status = self._sample_layout(n, W, mode)
        gdev = generator.device if generator is not None else dev
        if gdev.index is None and gdev.type == "cuda":
            gdev = torch.device("cuda", torch.cuda.current_device())
        ev = self.kernel_events if timed else None
        if ids is not None and lane is not caller:
            # the decode on the ring stream reads the ids, which the caller's stream may still be writing (or copying
            # there): the ring stream waits for what the caller enqueued before this call
            lane.wait_stream(caller)
        if lane is not caller:
            torch.cuda.set_stream(self._row_stream())
        lkey = lane.cuda_stream
        try:
            out = torch.empty((n, W), dtype=torch.int64 if ids is not None else torch.uint8, device=dev)
            coords = torch.empty((n, 4), dtype=torch.int64, device=dev) if return_coords else None
            if lane is not caller:
                torch.cuda.set_stream(lane)
            lw = self._stream_buffer(lkey, o_status + 8)
            draws, rnd, status = self._buffer_views(lkey, lw, n, wb, mode, o_draws, o_rnd, o_status)
            if gdev == dev:
                torch.randint(0, total, (n,), generator=generator, out=draws)
                if rnd is not None:
                    torch.rand(n, generator=generator, out=rnd)
            else:                       # a generator on another device draws there, as in the reference
                draws.copy_(torch.randint(0, total, (n,), generator=generator, device=gdev, dtype=torch.int64))
                if rnd is not None:
                    rnd.copy_(torch.rand(n, generator=generator, device=gdev))
            if ev is not None:          # created by a first record here, recorded again around the decode launches
                t0, tm, t1 = (torch.cuda.Event(enable_timing=True) for _ in range(3))
                t0.record(lane)
                tm.record(lane)
                t1.record(lane)
                if not self.kernel_events_split:
                    tm = None
        finally:
            if lane is not caller:
                torch.cuda.set_stream(caller)
        wbase = lw.data_ptr()
        consts = self._sample_consts(W, running)
        err = self._err
        wait = N.WAIT_COUNTER if self.sample_wait == "counter" else N.WAIT_EVENT
        if lane is not caller:
            self._lane_prepare(lane, caller, wait)
        args = (self._Dref, *consts, wbase + o_draws, wbase + o_rnd if rnd is not None else None, p, mode, n, W,
                int(bool(tokens)), 1, ids.data_ptr() if ids is not None else None, wbase, wb,
                coords.data_ptr() if coords is not None else None, out.data_ptr(), wbase + o_status, lkey, caller.cuda_stream, wait,
                t0.cuda_event if ev is not None else None, tm.cuda_event if ev is not None and tm is not None else None,
                t1.cuda_event if ev is not None else None, err, len(err))
        if torch.cuda.current_device() == idx:
            code = N.lib().pv_sample_hip(*args)
        else:
            with torch.cuda.device(dev):
                code = N.lib().pv_sample_hip(*args)
        if code:
            N.raise_for(code, err)
        if ev is not None:
            ev.append((t0, tm, t1))
        if lane is not caller:                  # not to be reused before the caller's work on the results is done
            out.record_stream(caller)
            if coords is not None:
                coords.record_stream(caller)
        if check:
            self._check(status)
        return (out, coords) if return_coords else out

    def _caller(self, sid):
        """A torch Stream for the stream handle triple `sid` (the caller's current stream)."""
        caller = self._callers.get(sid)
        if caller is None:
            if len(self._callers) >= 64:
                self._callers.clear()
            caller = self._callers[sid] = torch.cuda.Stream(stream_id=sid[0], device_index=sid[1], device_type=sid[2])
        return caller

    def _sample_layout(self, n, W, mode):
        """Bytes of pv_sample_hip's work for (n, W), and the offsets of the draws, the uniform numbers and the status
        word after it in the stream's buffer."""
        wb = self._work_bytes.get((n, W, self.light_decode))
        if wb is None:
            wb = int(N.lib().pv_sample_work_bytes(ctypes.byref(self._D), n, W)) if self.light_decode else (17 * n + 255) & ~255
            self._work_bytes[(n, W, self.light_decode)] = wb
        o_draws = wb
        o_rnd = o_draws + 8 * n
        o_status = o_rnd + ((4 * n + 7) & ~7 if mode == 2 else 0)
        return wb, o_draws, o_rnd, o_status

    def _buffer_views(self, lkey, lw, n, wb, mode, o_draws, o_rnd, o_status):
        vk = (lkey, lw.data_ptr(), n, wb, mode)
        views = self._views.get(vk)
        if views is None:       # the draws, uniform numbers and status inside the stream's buffer
            if len(self._views) >= 256:
                self._views.clear()
            views = self._views[vk] = (lw[o_draws:o_rnd].view(torch.int64),
                                       lw[o_rnd:o_rnd + 4 * n].view(torch.float32) if mode == 2 else None,
                                       lw[o_status:o_status + 4].view(torch.int32))
        return views

    def _sample_consts(self, W, running):
        consts = self._sample_args.get(W)
        if consts is None:
            consts = self._sample_args[W] = (running.data_ptr(), running.numel(), self._ctg["ctg_asm"].data_ptr(),
                                             self._ctg["ctg_local"].data_ptr(), self._ctg["ctg_boff"].data_ptr())
        return consts

    def _lane_prepare(self, lane, caller, wait):
        """The wait state of a ring stream and a caller stream (counters in signal memory, events), created once per
        pair and wait mode."""
        k = (lane.cuda_stream, caller.cuda_stream, wait)
        if k not in self._prepared:
            err = N.errbuf()
            code = N.lib().pv_sample_prepare(lane.cuda_stream, caller.cuda_stream, wait, err, len(err))
            if code:
                N.raise_for(code, err)
            self._prepared.add(k)

    def _row_stream(self):
        """The stream `sample` allocates its rows on when it runs on the ring (no work is ever enqueued on it)."""
        if self._rows is None:
            self._rows = torch.cuda.Stream(device=self.device)
        return self._rows

    def _prepare_shape(self, key, n, W, reverse_complement, tokens, return_coords, sid, k, token_ids=None):
        """Plans of one sample shape for every position of the ring (the caller's stream when k is 0): key is the
        shape's plan key for position key[7]; the others differ only there. token_ids: five ints, or None."""
        if W <= 0 or n < 0:
            raise ValueError("W must be positive, n non-negative")
        running, total = self._start_table(W)
        if total == 0:
            raise ValueError(f"no contig of {W} bases or more")
        mode, p = _rc_mode(reverse_complement)
        if self.sample_wait not in ("event", "counter"):
            raise ValueError('sample_wait: "event" or "counter"')
        wait = N.WAIT_COUNTER if self.sample_wait == "counter" else N.WAIT_EVENT
        ids = self._token_ids(token_ids) if token_ids is not None else None
        esize = 1 if ids is None else 8
        caller = self._caller(sid)
        if k > 0 and len(self._ring) != k:
            self._ring = self._make_ring(k, caller)
        lanes = list(enumerate(self._ring)) if k > 0 else [(-1, None)]
        wb, o_draws, o_rnd, o_status = self._sample_layout(n, W, mode)
        consts = self._sample_consts(W, running)
        if len(self._fast) + len(lanes) > 256:
            self._fast.clear()
        rows = self._row_stream() if k > 0 else None
        pool = cpool = None
        if rows is not None and wait == N.WAIT_COUNTER and not N.lib().pv_dispatch_serialised():
            def reserve(row_bytes):
                handle = ctypes.c_void_p()
                code = N.lib().pv_rows_reserve(row_bytes, min(_POOL_ROWS, _POOL_BYTES // row_bytes), ctypes.byref(handle),
                                              self._err, len(self._err))
                if code:
                    N.raise_for(code, self._err)
                return handle.value
            pool = reserve(n * W * esize)
            if return_coords:
                cpool = reserve(32 * n)
        if rows is not None:
            # rows allocated and freed on the row stream: its pool then holds blocks of the row size
            row_bytes = n * W * esize + (32 * n if return_coords else 0)
            warm = min(_PREWARM_ROWS, _PREWARM_BYTES // max(1, row_bytes))
            torch.cuda.set_stream(rows)
            try:
                tmp = [torch.empty((n, W), dtype=torch.uint8 if ids is None else torch.int64, device=self.device)
                       for _ in range(warm)]
                if return_coords:
                    tmp += [torch.empty((n, 4), dtype=torch.int64, device=self.device) for _ in range(warm)]
                del tmp
            finally:
                torch.cuda.set_stream(caller)
        for t, lane in lanes:
            s = lane or caller
            if lane is not None:
                torch.cuda.set_stream(lane)
            try:
                lw = self._stream_buffer(s.cuda_stream, o_status + 8)
                draws, rnd, status = self._buffer_views(s.cuda_stream, lw, n, wb, mode, o_draws, o_rnd, o_status)
            finally:
                if lane is not None:
                    torch.cuda.set_stream(caller)
            if lane is not None:
                self._lane_prepare(lane, caller, wait)
            if lane is None and self.light_decode:     # (on the caller's stream) a large call's side stream, made now
                code = N.lib().pv_launch_prepare(ctypes.byref(self._D), n, W, s.cuda_stream, self._err, len(self._err))
                if code:
                    N.raise_for(code, self._err)
            wbase = lw.data_ptr()
            a = N.SampleCall(D=ctypes.addressof(self._D), cum=consts[0], ncontigs=consts[1], ctg_asm=consts[2],
                             ctg_local=consts[3], ctg_boff=consts[4], draws=wbase + o_draws,
                             rnd=wbase + o_rnd if rnd is not None else None, p=p, rcmode=mode, tokens=int(tokens), n=n,
                             W=W, apply_case=1, wait=wait, ids=ids.data_ptr() if ids is not None else None, work=wbase, work_bytes=wb, coords=None, out=None,
                             status=wbase + o_status, stream=s.cuda_stream, caller=caller.cuda_stream,
                             err=ctypes.addressof(self._err), errcap=len(self._err))
            self._fast[key[:7] + (t,) + key[8:]] = _SamplePlan(self, lane, caller, (n, W), return_coords, draws, rnd, status,
                                                                total, a, lw, rows, pool, cpool, ids)

    def _sample_stream(self):
        """The next stream of the ring `sample` runs on (None: sample_streams is 0, run on the caller's stream)."""
        k = int(self.sample_streams)
        if k <= 0:
            return None
        if len(self._ring) != k:
            self._ring = self._make_ring(k, torch.cuda.current_stream(self.device))
        self._turn = (self._turn + 1) % k
        return self._ring[self._turn]

    def _make_ring(self, k, caller):
        """k streams for `sample`'s ring, each on a hardware queue of its own and none on the caller's. HIP maps a
        process's streams onto its GPU_MAX_HW_QUEUES queues (4 by default), several streams to a queue once there are
        more streams than queues, and calls whose streams share a queue run one after another. Streams come from torch's
        pool; one is kept when pv_streams_concurrent finds it concurrent with the caller's stream and with each one kept,
        trying at most 4 k. Fewer found: the ring repeats them (calls on one stream are in order). Where a tool
        serialises dispatches nothing can be concurrent, and with more than _PICK_QUEUES queues the GPU's scheduler
        shares its queue slots among them in turns, so two queues run at once on one test and not on the next (at 24
        queues, 3 of 7 streams kept on one test were not concurrent with the caller on the next): the pool streams as
        they come, which HIP spreads over that many queues."""
        dev = self.device
        L = N.lib()
        if L.pv_dispatch_serialised() or _hw_queues() > _PICK_QUEUES:
            return [torch.cuda.Stream(device=dev) for _ in range(k)]
        err, flag = N.errbuf(), ctypes.c_int32()

        def concurrent(a, b):
            code = L.pv_streams_concurrent(a.cuda_stream, b.cuda_stream, ctypes.byref(flag), err, len(err))
            if code:
                N.raise_for(code, err)
            return flag.value == 1

        ring, first = [], None
        with torch.cuda.device(dev):
            for _ in range(4 * k):
                s = torch.cuda.Stream(device=dev)
                first = first or s
                if concurrent(caller, s) and all(concurrent(r, s) for r in ring):
                    ring.append(s)
                    if len(ring) == k:
                        break
        if not ring:
            ring = [first]
        return [ring[i % len(ring)] for i in range(k)]

    def fetch(self, assembly, contig, start, length, reverse_complement=False, tokens=False):
        """Bases [start, start + length) of one contig (0-based) -> uint8 [length] on the cohort's device; IndexError
        if the slice leaves the contig. (reference panvram/cohort.py:196-207)"""
        a = self._asm(assembly)
        name, _, clen, boff, _ = self._ctgs[a][self._contig(a, contig)]
        start, length = int(start), int(length)
        if start < 0 or length < 0 or start + length > clen:
            raise IndexError(f"{self.names[a]} {name}:{start}+{length} outside the contig ({clen} bases)")
        # windows([a], [boff + start], length, rc, tokens)[0] with the coordinates passed by value: one launch writes
        # them to a device record of this thread's (and zeroes its status word) ahead of the decode, where one-element
        # tensors would cost two synchronous host-to-device copies and a fill
        if length >= (1 << 31):
            raise RuntimeError("W")
        dev = self.device
        loc = self._local
        rec = getattr(loc, "rec", None)
        if rec is None:
            rec = loc.rec = torch.zeros(32, dtype=torch.uint8, device=dev)
            loc.status, loc.err = rec[24:28].view(torch.int32), N.errbuf()
        out = torch.empty((1, length), dtype=torch.uint8, device=dev)
        err, L, D = loc.err, N.lib(), self._Dref
        stream = torch.cuda.current_stream(dev).cuda_stream
        wb = int(L.pv_windows_work_bytes(D, 1, length)) if self.light_decode else 0
        wp = self._stream_buffer(stream, wb).data_ptr() if wb else None
        args = (D, a, boff + start, length, int(bool(reverse_complement)), int(bool(tokens)), out.data_ptr(), rec.data_ptr(), wp, wb,
                stream, err, len(err))
        ev = self.kernel_events
        if ev is not None:
            t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            t0.record()
        if torch.cuda.current_device() == self._idx:    # (the library's launches and lookups use the current device)
            code = L.pv_fetch_hip(*args)
        else:
            with torch.cuda.device(dev):
                code = L.pv_fetch_hip(*args)
        if ev is not None:
            t1.record()
            ev.append((t0, None, t1))
        if code:
            N.raise_for(code, err)
        self._check(loc.status)
        return out[0]

    _HOST_BUFS = 8          # device pieces in flight to the host

    def _stream_to_host(self, a, out, apply_case, chunk=1 << 28):
        """The assembly's whole base stream decoded on the device in `chunk`-base pieces into a pinned host tensor
        (`out` reused when large enough) -> (out, device status). The decode runs ~15x faster than PCIe, so up to
        _HOST_BUFS device buffers hold decoded pieces; piece i is copied to the host on copy stream i % 2 (two copies
        in flight move ~10 % more than one: 56 against 51 GB/s on MI355X), and a buffer is decoded into again only
        after its copy."""
        n = self._meta[a]["bases"]
        if out is None or out.numel() < n:
            out = torch.empty(n, dtype=torch.uint8, pin_memory=True)
        out = out[:n]
        chunk = int(chunk)
        if chunk <= 0:
            raise ValueError("chunk must be positive")
        dev = self.device
        if self._aux is None:
            self._aux = torch.cuda.Stream(device=dev)
        if self._aux2 is None:
            self._aux2 = [torch.cuda.Stream(device=dev) for _ in range(2)]
        ds, css = self._aux, self._aux2
        ds.wait_stream(torch.cuda.current_stream(dev))
        piece = min(chunk, max(n, 1))
        npieces = (n + chunk - 1) // chunk
        nbuf = max(1, min(self._HOST_BUFS, npieces))
        with torch.cuda.stream(ds):
            status = torch.zeros(1, dtype=torch.int32, device=dev)
            asm_t = torch.tensor([a], dtype=torch.int64, device=dev)
            starts = torch.arange(0, n, chunk, dtype=torch.int64, device=dev)
            bufs = [torch.empty(piece, dtype=torch.uint8, device=dev) for _ in range(nbuf)]
        copied = [None] * nbuf
        for i, s in enumerate(range(0, n, chunk)):
            k, b, cs = min(chunk, n - s), i % nbuf, css[i % 2]
            with torch.cuda.stream(ds):
                if copied[b] is not None:
                    ds.wait_event(copied[b])
                self._windows_into(asm_t, starts[i:i + 1], k, None, False, apply_case, bufs[b][:k].view(1, k), status)
                decoded = torch.cuda.Event()
                decoded.record(ds)
            with torch.cuda.stream(cs):
                cs.wait_event(decoded)
                out[s:s + k].copy_(bufs[b][:k], non_blocking=True)
                copied[b] = torch.cuda.Event()
                copied[b].record(cs)
        for cs in css:
            cs.synchronize()
        ds.synchronize()
        return out, status

    def decode(self, assembly, chunk=1 << 28, out=None):
        """The assembly's whole base stream (contigs back to back, case as in its FASTA) -> uint8 [bases] in pinned
        host memory; `out` is reused when large enough. Decoded on the device in `chunk`-base pieces, each copied to
        the host while the next one decodes; RuntimeError (status bits) if a block fails, as `windows` with check.
        (reference panvram/cohort.py:209-222)"""
        a = self._asm(assembly)
        out, status = self._stream_to_host(a, out, True, chunk)
        self._check(status)
        return out

    def fasta_xxh3(self, assembly, bases):
        """XXH3-64 ("%016x") of the FASTA that the contig table lays out around a decoded base stream (uint8 host
        tensor), computed without building the file. (reference csrc/pv_core.cpp:167-176)"""
        a = self._asm(assembly)
        b = bases.contiguous()
        h, err = ctypes.c_uint64(), N.errbuf()
        code = N.lib().pv_fasta_xxh3(self._h, a, b.data_ptr() if b.numel() else None, b.numel(), ctypes.byref(h), err, len(err))
        if code:
            N.raise_for(code, err)
        return f"{h.value:016x}"

    def _fasta_plan(self, a):
        """The assembly's FASTA layout: per record (FASTA offset, header offset, header length, length, base offset,
        line width) on the host and the device, the header bytes on the device, the file size."""
        plan = self._plans.get(a)
        if plan is None:
            rows, blob, f = [], bytearray(), 0
            for _, hdr, ln, boff, lw in self._ctgs[a]:
                hb = hdr.encode()
                rows.append((f, len(blob), len(hb), ln, boff, lw))
                blob += hb
                f += 2 + len(hb) + ln + ((ln + lw - 1) // lw if lw else 0)
            if f != int(N.lib().pv_fasta_size(self._h, a)):
                raise RuntimeError("FASTA layout size disagrees with the archive's record table")
            dev_rows = torch.tensor(rows, dtype=torch.int64).flatten().to(self.device)
            dev_hdrs = torch.frombuffer(bytearray(blob) or bytearray(1), dtype=torch.uint8).to(self.device)
            plan = (rows, dev_rows, dev_hdrs, f)
            self._plans[a] = plan
        return plan

    @staticmethod
    def _bases_before(rows, f):
        """Number of stream bases that precede FASTA byte offset f (rows: the plan's record table)."""
        lo, hi = 0, len(rows) - 1
        while lo < hi:
            m = (lo + hi + 1) // 2
            if rows[m][0] <= f:
                lo = m
            else:
                hi = m - 1
        fo, _, hl, ln, boff, lw = rows[lo]
        q = f - fo - hl - 2
        if q <= 0:
            return boff
        line, col = divmod(q, lw + 1)
        return boff + min(ln, line * lw + min(col, lw))

    def check_full(self, assembly, out=None):
        """Decode the whole assembly on the device, hash the FASTA it rebuilds, and compare with the source FASTA's
        XXH3 in the archive header -> (equal, hash as "%016x"). (reference panvram/cohort.py:224-229)

        Pipelined: the FASTA is produced on the device in 256 MiB pieces (decode with case, then a layout kernel that
        writes headers and line ends) and copied to pinned host memory, while the host hashes the previous piece.
        `out` (optional, pinned uint8 [bases]) also receives the decoded base stream, as the reference's does."""
        a = self._asm(assembly)
        rows, dev_rows, dev_hdrs, F = self._fasta_plan(a)
        n = self._meta[a]["bases"]
        dev, L = self.device, N.lib()
        if self._aux is None:
            self._aux = torch.cuda.Stream(device=dev)
        s = self._aux
        piece = 1 << 28
        s.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(s):
            status = torch.zeros(1, dtype=torch.int32, device=dev)
            bbuf = [torch.empty(piece + 16, dtype=torch.uint8, device=dev) for _ in range(2)]
            fbuf = [torch.empty(piece, dtype=torch.uint8, device=dev) for _ in range(2)]
            asm_t = torch.tensor([a], dtype=torch.int64, device=dev)
        pins = [torch.empty(piece, dtype=torch.uint8, pin_memory=True) for _ in range(2)]
        if out is not None and out.numel() < n:
            raise ValueError("out: a pinned uint8 tensor of at least the assembly's length")
        done = [torch.cuda.Event(), torch.cuda.Event()]
        hs = L.pv_xxh3_stream_new()
        if not hs:
            raise MemoryError("XXH3 state")
        err = N.errbuf()
        try:
            pending = None
            for i, f0 in enumerate(range(0, F, piece)):
                f1 = min(F, f0 + piece)
                b0, b1 = self._bases_before(rows, f0), self._bases_before(rows, f1)
                k = i % 2
                with torch.cuda.stream(s):
                    if b1 > b0:
                        start = torch.tensor([b0], dtype=torch.int64, device=dev)
                        self._windows_into(asm_t, start, b1 - b0, None, False, True, bbuf[k][:b1 - b0].view(1, -1), status)
                        if out is not None:
                            out[b0:b1].copy_(bbuf[k][:b1 - b0], non_blocking=True)
                    code = L.pv_fasta_layout_hip(bbuf[k].data_ptr(), b0, b1 - b0, dev_rows.data_ptr(), len(rows), dev_hdrs.data_ptr(),
                                                 f0, f1 - f0, fbuf[k].data_ptr(), s.cuda_stream, err, len(err))
                    if code:
                        N.raise_for(code, err)
                    pins[k][:f1 - f0].copy_(fbuf[k][:f1 - f0], non_blocking=True)
                    done[k].record(s)
                if pending is not None:                  # hash the previous piece while the device makes this one
                    pk, plen = pending
                    done[pk].synchronize()
                    L.pv_xxh3_stream_update(hs, pins[pk].data_ptr(), plen)
                pending = (k, f1 - f0)
            if pending is not None:
                done[pending[0]].synchronize()
                L.pv_xxh3_stream_update(hs, pins[pending[0]].data_ptr(), pending[1])
            h = f"{L.pv_xxh3_stream_digest(hs):016x}"
        finally:
            L.pv_xxh3_stream_free(hs)
        s.synchronize()
        if int(status.item()):
            raise N.FormatError(f"{self._meta[a]['path']}: block decode failed")
        return h == self._meta[a]["fasta_xxh3"], h

    def fasta(self, assembly, verify=True):
        """The assembly's FASTA file, byte for byte. With verify, every block's XXH3 (when the archive has them) and the
        rebuilt file's XXH3 must match the archive. Decoded on the device (upper case), checked and finished on the
        host. (reference panvram/cohort.py:231-234; csrc/pv_core.cpp:138-159)"""
        a = self._asm(assembly)
        meta, L = self._meta[a], N.lib()
        host, status = self._stream_to_host(a, None, False)
        if int(status.item()):
            raise N.FormatError(f"{meta['path']}: block decode failed")
        n = host.numel()
        p = host.data_ptr() if n else None
        if verify:
            first_bad = ctypes.c_int64()
            L.pv_verify_blocks(self._h, a, p, n, ctypes.byref(first_bad))
            if first_bad.value >= 0:
                raise N.FormatError(f"{meta['path']}: block XXH3 mismatch")
        L.pv_apply_case(self._h, a, 0, p, n)
        size = int(L.pv_fasta_size(self._h, a))
        buf, err = ctypes.create_string_buffer(size), N.errbuf()
        code = L.pv_fasta_build(self._h, a, p, n, buf, size, err, len(err))
        if code:
            N.raise_for(code, err)
        if verify:
            h = ctypes.c_uint64()
            L.pv_fasta_xxh3(self._h, a, p, n, ctypes.byref(h), err, len(err))
            if f"{h.value:016x}" != meta["fasta_xxh3"]:
                raise N.FormatError(f"{meta['path']}: FASTA XXH3 differs from the header")
        return buf.raw
