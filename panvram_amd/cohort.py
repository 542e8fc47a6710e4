"""panvram_amd.Cohort - a pangenome cohort resident on one MI355X as refrel3 v1 archives against one decoded reference;
windows and coordinate slices decoded on the card by the HIP kernels of libpanvram_amd.so.

The class mirrors the reference's panvram.Cohort (reference panvram/cohort.py:38-251): same constructor
(`Cohort.open`), same methods and argument meanings, same exceptions and messages, so a caller switches by changing
the import. Differences, all deliberate:
  * decoding runs on the GPU only (device "cuda"/"cuda:N" on ROCm); there is no CPU decoder in the product - the CPU
    decoder of this repository lives in oracle/ as the test checker;
  * `fasta()` decodes on the GPU too, then checks every block XXH3 and the FASTA XXH3 on the host, as the reference's
    CPU `fasta(verify=True)` does;
  * the per-W count of valid window starts is cached as a Python int with the per-W cumulative table (the reference
    reads it back from the device on every `sample` call, cohort.py:189) - same draws, one sync fewer per call.
"""
import ctypes
import glob
import os
import re

import torch

from . import _native as N

DATASETS = ("q4k", "q16k")
_PAD = 1024  # zero bytes after every device array: kernels read 16-byte chunks and 256-byte payload windows past a start


def _arch_ok(device):
    p = torch.cuda.get_device_properties(device)
    arch = getattr(p, "gcnArchName", "") or ""
    if not arch.startswith("gfx950"):
        raise RuntimeError(f"panvram_amd is built for gfx950 (MI355X); {torch.cuda.get_device_name(device)} is {arch or 'unknown'}")


def _host_view(ptr, nbytes):
    if not nbytes:
        return torch.empty(0, dtype=torch.uint8)
    return torch.frombuffer((ctypes.c_uint8 * nbytes).from_address(ptr), dtype=torch.uint8)


class Cohort:
    """Open with Cohort.open(dir, device=...). Coordinates are 0-based; a contig is its FASTA header up to the first
    space or tab, or its index in the assembly; an assembly is its name (archive file name without .<dataset>.rr3) or
    its index."""

    def __init__(self, handle, names, device):
        self._h, self.names, self.device = handle, list(names), torch.device(device)
        self._close = N.lib().pv_cohort_close     # held so that __del__ still works while modules are torn down
        L = N.lib()
        self._index = {n: i for i, n in enumerate(self.names)}
        self._n = int(L.pv_cohort_assemblies(handle))
        self._Q = int(L.pv_cohort_block_size(handle))
        self._ref_n = int(L.pv_cohort_ref_bases(handle))
        sha = ctypes.create_string_buffer(65)
        L.pv_cohort_ref_sha256(handle, sha)
        self._sha = sha.value.decode()
        self._contigs = [self._read_contigs(i) for i in range(self._n)]
        self._ctg_names = [{c[0]: k for k, c in enumerate(cs)} for cs in self._contigs]
        self._infos = [self._read_info(i) for i in range(self._n)]
        if self.device.type != "cuda":
            raise RuntimeError("panvram_amd decodes on the GPU only (device 'cuda' / 'cuda:N'); the CPU decoder of this "
                               "repository is the test oracle (oracle/), not part of the package")
        _arch_ok(self.device)
        self._dev = {}
        for key, aid, dtype in (("P", N.ARR_P, torch.uint8), ("off", N.ARR_OFF, torch.int32), ("st", N.ARR_ST, torch.int64),
                                ("run0", N.ARR_RUN0, torch.int32), ("tab", N.ARR_TAB, torch.uint8), ("asm", N.ARR_ASM, torch.int64),
                                ("low_s", N.ARR_LOW_S, torch.int64), ("low_l", N.ARR_LOW_L, torch.int64), ("ref", N.ARR_REF, torch.uint8),
                                ("ctg_asm", N.ARR_CTG_ASM, torch.int64), ("ctg_local", N.ARR_CTG_LOCAL, torch.int64),
                                ("ctg_boff", N.ARR_CTG_BOFF, torch.int64), ("ctg_len", N.ARR_CTG_LEN, torch.int64)):
            ptr, nb = ctypes.c_void_p(), ctypes.c_uint64()
            if L.pv_cohort_array(handle, aid, ctypes.byref(ptr), ctypes.byref(nb)):
                raise RuntimeError(f"pooled array {key} unavailable")
            nb = nb.value
            dev = torch.empty(nb + _PAD, dtype=torch.uint8, device=self.device)
            if nb:
                dev[:nb].copy_(_host_view(ptr.value, nb))
            dev[nb:].zero_()
            self._dev[key] = (dev, nb, dtype)
            if aid in (N.ARR_P, N.ARR_OFF, N.ARR_ST, N.ARR_RUN0, N.ARR_TAB, N.ARR_REF):
                L.pv_cohort_release_array(handle, aid)      # the device copy is the only one needed from here on
        torch.cuda.synchronize(self.device)
        self._ctg = {k: self._typed(k) for k in ("ctg_asm", "ctg_local", "ctg_boff", "ctg_len")}
        D = N.DevCohort()
        D.P, D.off, D.st, D.run0, D.tab, D.asm_rec, D.low_s, D.low_l, D.ref = (
            self._dev[k][0].data_ptr() for k in ("P", "off", "st", "run0", "tab", "asm", "low_s", "low_l", "ref"))
        D.ref_n, D.nasm, D.Q = self._ref_n, self._n, self._Q
        self._D = D
        self._valid = {}
        self.kernel_events = None   # a list to collect (start, end) torch.cuda.Events around each decode launch

    def _typed(self, key):
        dev, nb, dtype = self._dev[key]
        return dev[:nb].view(dtype)

    def __del__(self):
        h, close = getattr(self, "_h", None), getattr(self, "_close", None)
        if h and close is not None:
            close(h)
            self._h = None

    @classmethod
    def open(cls, path, device="cuda", dataset="q4k", reference=None, threads=0, assemblies=None,
             packed_reference=False, compact_blocks=False):
        """Open the cohort directory `path`: every `*.<dataset>.rr3` in it (sorted by name; `assemblies` = a list of
        names to take only those) and the reference they were encoded against - `reference` if given, else
        `path/reference.fa`, else the file named in the archives' header in `path`. Every archive is checked before
        any decode (header XXH3, reference SHA-256 and size, sections, tables). One block size per cohort.
        device: "cuda" or "cuda:N". (reference panvram/cohort.py:60-100)"""
        if packed_reference or compact_blocks:
            raise NotImplementedError("the compact resident forms (packed_reference, compact_blocks) are not built yet in panvram_amd")
        if dataset is not None and not re.fullmatch(r"q\d+k", dataset):
            raise ValueError(f"dataset: {DATASETS} (or another q<N>k suffix), or None for every *.rr3")
        pat = f"*.{dataset}.rr3" if dataset else "*.rr3"
        files = sorted(glob.glob(os.path.join(path, pat)))
        suffix = f".{dataset}.rr3" if dataset else ".rr3"
        names = [os.path.basename(f)[: -len(suffix)] for f in files]
        if assemblies is not None:
            want = list(assemblies)
            have = dict(zip(names, files))
            missing = [a for a in want if a not in have]
            if missing:
                raise FileNotFoundError(f"not in {path}: {missing[:5]}")
            names, files = want, [have[a] for a in want]
        if not files:
            raise FileNotFoundError(f"no {pat} in {path}")
        if reference is None:
            cand = os.path.join(path, "reference.fa")
            if not os.path.exists(cand):
                with open(files[0], "rb") as f:
                    h = f.read(138 + 65535)
                nl = h[136] | h[137] << 8
                cand = os.path.join(path, h[138:138 + nl].decode())
            reference = cand
        if not os.path.exists(reference):
            raise FileNotFoundError(f"reference {reference} not found (pass reference=)")
        device = torch.device(device)
        if device.type == "cuda" and device.index is None:
            device = torch.device("cuda", torch.cuda.current_device())
        L = N.lib()
        arr = (ctypes.c_char_p * len(files))(*[os.fsencode(f) for f in files])
        out, err = ctypes.c_void_p(), N.errbuf()
        code = L.pv_cohort_open(os.fsencode(reference), ctypes.cast(arr, ctypes.c_void_p), len(files), int(threads), ctypes.byref(out), err, len(err))
        if code:
            N.raise_for(code, err)
        return cls(out.value, names, device)

    # ------------------------------------------------------------------ description
    def __len__(self):
        return len(self.names)

    @property
    def block_size(self):
        return self._Q

    @property
    def reference_sha256(self):
        return self._sha

    def _read_contigs(self, a):
        L = N.lib()
        nm, hd = ctypes.c_char_p(), ctypes.c_char_p()
        ln, off, lw = ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint32()
        out, k = [], 0
        while L.pv_asm_contig(self._h, a, k, ctypes.byref(nm), ctypes.byref(hd), ctypes.byref(ln), ctypes.byref(off), ctypes.byref(lw)) == 0:
            out.append((nm.value.decode(), hd.value.decode(), ln.value, off.value, lw.value))
            k += 1
        return out

    def _read_info(self, a):
        x = N.AsmInfo()
        if N.lib().pv_asm_info_get(self._h, a, ctypes.byref(x)):
            raise IndexError(f"assembly index {a}")
        return {"path": x.path.decode(), "Q": x.Q, "bases": x.bases, "blocks": x.blocks, "file_bytes": x.file_bytes,
                "payload_bytes": x.payload_bytes, "block_hashes": bool(x.block_hashes), "fasta_xxh3": f"{x.fasta_xxh3:016x}",
                "contigs": x.contigs, "lower_case_runs": x.lower_case_runs, "reference_name": x.reference_name.decode()}

    def info(self, assembly):
        return dict(self._infos[self._asm(assembly)])

    def contigs(self, assembly):
        """[(name, header, length, offset in the base stream, line width)] of an assembly."""
        return list(self._contigs[self._asm(assembly)])

    def resident_bytes(self):
        """Bytes of the cohort on its device (reference included), by component."""
        d = {k: nb for k, (_, nb, _) in self._dev.items() if not k.startswith("ctg_")}
        d["total"] = sum(d.values())
        return d

    # ------------------------------------------------------------------ decode
    def _asm(self, a):
        if isinstance(a, str):
            if a not in self._index:
                raise KeyError(f"no assembly {a}")
            return self._index[a]
        a = int(a)
        if not 0 <= a < len(self.names):
            raise IndexError(f"assembly index {a}")
        return a

    def _contig(self, a, c):
        if isinstance(c, str):
            if c not in self._ctg_names[a]:
                raise KeyError(f"no contig {c} in {self.names[a]}")
            return self._ctg_names[a][c]
        c = int(c)
        if not 0 <= c < len(self._ctg_names[a]):
            raise IndexError(f"contig index {c}")
        return c

    def _launch(self, asm, start, W, reverse_complement, tokens, apply_case):
        W = int(W)
        if W < 0 or W >= (1 << 31):
            raise RuntimeError("W")
        dev = self.device
        asm = torch.as_tensor(asm).to(dev, torch.int64).contiguous()
        start = torch.as_tensor(start).to(dev, torch.int64).contiguous()
        n = asm.numel()
        if start.numel() != n:
            raise RuntimeError("assembly and start counts differ")
        out = torch.empty((n, W), dtype=torch.uint8, device=dev)
        status = torch.zeros(1, dtype=torch.int32, device=dev)
        rc = None
        if reverse_complement is not None:
            rc = torch.as_tensor(reverse_complement).to(dev, torch.uint8).contiguous()
            if rc.numel() != n:
                raise RuntimeError("reverse_complement mask size")
        err = N.errbuf()
        ev = self.kernel_events
        with torch.cuda.device(dev):
            stream = torch.cuda.current_stream(dev).cuda_stream
            if ev is not None:
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record()
            code = N.lib().pv_windows_hip(ctypes.byref(self._D), asm.data_ptr(), start.data_ptr(), n, W,
                                          rc.data_ptr() if rc is not None else None, int(bool(tokens)), int(bool(apply_case)),
                                          out.data_ptr(), status.data_ptr(), stream, err, len(err))
            if ev is not None:
                e1.record()
                ev.append((e0, e1))
        if code:
            N.raise_for(code, err)
        return out, status

    def windows(self, asm, start, W, reverse_complement=None, tokens=False, check=True):
        """Bases [start, start + W) of assembly asm[i] (start = offset in the assembly's base stream: contigs
        concatenated in file order) for every i -> uint8 [n, W] on the cohort's device. reverse_complement: None or a
        bool tensor [n]. tokens: A/a 0, C/c 1, G/g 2, T/t 3, anything else 4; else the FASTA's bytes, case kept.
        check: wait for the kernel and raise if any block failed to decode (one device sync).
        (reference panvram/cohort.py:151-174)"""
        out, status = self._launch(asm, start, W, reverse_complement, tokens, True)
        if check:
            s = int(status.item())
            if s:
                raise RuntimeError(f"GPU decode failed (status {s}: 1 corrupt block, 4 bounded wait expired, 8 window outside an assembly)")
        return out

    def sample(self, n, W, generator=None, reverse_complement=False, tokens=False, return_coords=False, check=True):
        """n windows of W bases, uniform over every (assembly, contig, start) with start + W <= contig length (a
        window never crosses contigs) -> uint8 [n, W] on the cohort's device. generator: a torch.Generator (its device
        draws the numbers). reverse_complement: False, True, or p in (0, 1) - each window reverse-complemented with
        probability p. return_coords: also an int64 [n, 4] tensor (assembly, contig index, start in the contig,
        reverse-complemented 0/1). (reference panvram/cohort.py:176-211; the same torch draws in the same order)"""
        n, W = int(n), int(W)
        if W <= 0 or n < 0:
            raise ValueError("W must be positive, n non-negative")
        if W not in self._valid:
            v = (self._ctg["ctg_len"] - W + 1).clamp_min(0)
            cum = torch.cumsum(v, 0)
            total = int(cum[-1].item()) if cum.numel() else 0
            self._valid[W] = (cum, v, total)
        cum, v, total = self._valid[W]
        if total == 0:
            raise ValueError(f"no contig of {W} bases or more")
        gdev = generator.device if generator is not None else self.device
        u = torch.randint(0, total, (n,), generator=generator, device=gdev, dtype=torch.int64).to(self.device)
        k = torch.searchsorted(cum, u, right=True)
        pos = u - (cum[k] - v[k])
        asm = self._ctg["ctg_asm"][k]
        start = self._ctg["ctg_boff"][k] + pos
        if reverse_complement is True:
            rc = torch.ones(n, dtype=torch.bool, device=self.device)
        elif reverse_complement is False or reverse_complement is None or reverse_complement == 0:
            rc = None
        else:
            p = float(reverse_complement)
            if not 0 < p <= 1:
                raise ValueError("reverse_complement: False, True or a probability")
            rc = (torch.rand(n, generator=generator, device=gdev) < p).to(self.device)
        x = self.windows(asm, start, W, rc, tokens, check)
        if not return_coords:
            return x
        strand = rc.to(torch.int64) if rc is not None else torch.zeros(n, dtype=torch.int64, device=self.device)
        return x, torch.stack([asm, self._ctg["ctg_local"][k], pos, strand], 1)

    def fetch(self, assembly, contig, start, length, reverse_complement=False, tokens=False):
        """Bases [start, start + length) of a contig (0-based) -> uint8 [length] on the cohort's device.
        (reference panvram/cohort.py:213-224)"""
        a = self._asm(assembly)
        c = self._contig(a, contig)
        name, _, clen, boff, _ = self._contigs[a][c]
        start, length = int(start), int(length)
        if start < 0 or length < 0 or start + length > clen:
            raise IndexError(f"{self.names[a]} {name}:{start}+{length} outside the contig ({clen} bases)")
        asm = torch.tensor([a], dtype=torch.int64)
        st = torch.tensor([boff + start], dtype=torch.int64)
        rc = torch.tensor([bool(reverse_complement)]) if reverse_complement else None
        return self.windows(asm, st, length, rc, tokens)[0]

    def decode(self, assembly, chunk=1 << 28, out=None):
        """The whole base stream of an assembly (contigs concatenated, case as in the FASTA) decoded on the cohort's
        device in chunks of `chunk` bases -> uint8 [bases] on the host (pinned; `out` reused if given).
        (reference panvram/cohort.py:226-239)"""
        a = self._asm(assembly)
        n = self._infos[a]["bases"]
        if out is None or out.numel() < n:
            out = torch.empty(n, dtype=torch.uint8, pin_memory=True)
        out = out[:n]
        asm = torch.tensor([a], dtype=torch.int64)
        for s in range(0, n, chunk):
            k = min(chunk, n - s)
            out[s:s + k].copy_(self.windows(asm, torch.tensor([s], dtype=torch.int64), k)[0], non_blocking=False)
        return out

    def fasta_xxh3(self, assembly, bases):
        """XXH3 ("%016x") of the FASTA rebuilt from a decoded base stream (uint8 CPU tensor) and the contig table.
        (reference csrc/pv_core.cpp:167-176, Core.fasta_xxh3)"""
        a = self._asm(assembly)
        b = bases.contiguous()
        if b.device.type != "cpu" or b.dtype != torch.uint8:
            raise N.FormatError("bases: uint8 CPU tensor of the assembly's length")
        h, err = ctypes.c_uint64(), N.errbuf()
        code = N.lib().pv_fasta_xxh3(self._h, a, b.data_ptr() if b.numel() else None, b.numel(), ctypes.byref(h), err, len(err))
        if code:
            N.raise_for(code, err)
        return f"{h.value:016x}"

    def check_full(self, assembly, out=None):
        """Full decode on the cohort's device, the FASTA rebuilt from it (layout from the contig table) hashed with
        XXH3 -> (equal to the header's source XXH3, the hash "%016x"). (reference panvram/cohort.py:241-246)"""
        a = self._asm(assembly)
        h = self.fasta_xxh3(a, self.decode(a, out=out))
        return h == self._infos[a]["fasta_xxh3"], h

    def fasta(self, assembly, verify=True):
        """Full decode of an assembly -> the FASTA file's bytes. verify: every block XXH3 (if present) and the XXH3 of
        the rebuilt FASTA against the header's (the source file's). (reference panvram/cohort.py:248-251 and
        csrc/pv_core.cpp:138-159; decoded on the GPU here, hashes checked on the host)"""
        a = self._asm(assembly)
        info = self._infos[a]
        n, path, L = info["bases"], info["path"], N.lib()
        host = torch.empty(n, dtype=torch.uint8, pin_memory=True)
        asm = torch.tensor([a], dtype=torch.int64)
        chunk = 1 << 28
        for s in range(0, n, chunk):
            k = min(chunk, n - s)
            x, status = self._launch(asm, torch.tensor([s], dtype=torch.int64), k, None, False, False)
            if int(status.item()):
                raise N.FormatError(f"{path}: block decode failed")
            host[s:s + k].copy_(x[0])
        p = host.data_ptr() if n else None
        if verify:
            bad = ctypes.c_int64()
            L.pv_verify_blocks(self._h, a, p, n, ctypes.byref(bad))
            if bad.value >= 0:
                raise N.FormatError(f"{path}: block XXH3 mismatch")
        L.pv_apply_case(self._h, a, 0, p, n)
        size = int(L.pv_fasta_size(self._h, a))
        buf = ctypes.create_string_buffer(size)
        err = N.errbuf()
        code = L.pv_fasta_build(self._h, a, p, n, buf, size, err, len(err))
        if code:
            N.raise_for(code, err)
        data = buf.raw
        if verify:
            h, err = ctypes.c_uint64(), N.errbuf()
            N.lib().pv_fasta_xxh3(self._h, a, p, n, ctypes.byref(h), err, len(err))
            if f"{h.value:016x}" != info["fasta_xxh3"]:
                raise N.FormatError(f"{path}: FASTA XXH3 differs from the header")
        return data
