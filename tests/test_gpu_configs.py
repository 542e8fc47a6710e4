"""The five configurations of the benchmark on the GPU path, each generated on the box by tests/cohortgen at its full
size and checked against the CPU decoder (the reference's own, oracle/_ref, where it was built; the oracle port
otherwise) at the coordinates the GPU returned:

  config 1  tiny q4k cohort: sample(256, 8192), generator seeded 0, every window; every block hash and FASTA hash of
            every haplotype (fasta(verify=True)) and check_full
  config 2  mid q4k cohort: 1000 x sample(1024, 8192, tokens, reverse_complement=0.5, return_coords), generator
            seeded 0: the first batch whole, then 11 windows of every batch (1.07 %)
  config 3  mid q16k cohort: 65,536 fetch slices of 5,000 bases as one batch (every 100th checked, and single fetch()
            calls equal to their rows), and sample(1024, W) for W in {1024, 4096, 8192, 32768, 65536}
  config 4  one 3.1 Gbp haplotype: decode() equals the archive's base-stream XXH3, check_full equals its FASTA XXH3,
            and random windows
  config 5  558 haplotypes of the 3.1 Gbp reference: 10,000 x sample(1024, 8192, reverse_complement=0.5), half uint8
            and half tokens, 11 windows of every batch (1.07 %) and the first batch of each form whole; one batch of
            65,536 windows (1 % checked)

The reference's gate protocol (tests/test_gate.py:22-58) and test_synth.py:127-145 are the model. Cohorts go to
/dev/shm (or PANVRAM_TEST_DATA) under the names bench.py uses, so one box generates each once. Run with -m gpu."""
import json
import os
import shutil
import tempfile
import time

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PROGRESS = os.path.join(ROOT, "gpurun_out", "gpu_tests_progress.log")
SPOT = 11                                      # windows checked per batch of 1024 (1.07 %)


def _note(msg):
    """A line in the progress file: pytest holds the tests' own output until they end, and these steps take minutes."""
    os.makedirs(os.path.dirname(PROGRESS), exist_ok=True)
    with open(PROGRESS, "a") as f:
        f.write(f"{time.strftime('%H:%M:%S')} {msg}\n")


def _cohort_dir(config):
    """The preset's cohort directory, generated unless a complete one is there (bench.py's layout and stamp)."""
    from tests import cohortgen as G
    base = os.environ.get("PANVRAM_TEST_DATA") or os.environ.get("PANVRAM_BENCH_DIR")
    if not base:
        base = "/dev/shm" if os.path.isdir("/dev/shm") and shutil.disk_usage("/dev/shm").free > 60e9 else tempfile.gettempdir()
    d = os.path.join(base, "panvram_bench_" + config)
    stamp = os.path.join(d, "stamp.json")
    want = {"config": config, "assemblies": None, "version": 2}
    if os.path.exists(stamp) and json.load(open(stamp)) == want:
        return d
    shutil.rmtree(d, ignore_errors=True)
    os.makedirs(d)
    os.environ["COHORTGEN_PROGRESS"] = PROGRESS
    t = time.time()
    st = G.make(config, d, threads=min(16, os.cpu_count() or 1))
    json.dump(want, open(stamp, "w"))
    _note(f"{config}: generated in {time.time() - t:.0f} s {st}")
    return d


class _Cpu:
    """The CPU decoder over the cohort's archives: the reference's (oracle/_ref) or the oracle port."""

    def __init__(self, d, c):
        paths = [c.info(i)["path"] for i in range(len(c))]
        ref = os.path.join(d, "reference.fa")
        self.T = min(16, os.cpu_count() or 1)
        self.R = O.RefDecoder.open(ref, paths, threads=self.T)
        if self.R is None:
            self.ref = O.reference_bases(ref)
            self.arcs = [O.Archive(p) for p in paths]

    def windows(self, asm, start, W, rc=None, tokens=False):
        if self.R is not None:
            return self.R.windows(asm, start, W, rc=rc, tokens=tokens, threads=self.T)
        return O.windows(self.arcs, self.ref, asm, start, W, rc=rc, tokens=tokens, threads=self.T)


def _open(config, dataset="q4k"):
    import panvram_amd
    d = _cohort_dir(config)
    t = time.time()
    c = panvram_amd.Cohort.open(d, device="cuda", dataset=dataset)
    _note(f"{config}: opened {len(c)} assemblies in {time.time() - t:.1f} s, {c.resident_bytes()['total'] / 1e9:.2f} GB resident")
    cpu = _Cpu(d, c)
    return d, c, cpu


def _stream_starts(c, co):
    """Stream offsets of sample's (assembly, contig, start) coordinates."""
    offs = [[ctg[3] for ctg in c.contigs(a)] for a in range(len(c))]
    return np.array([offs[a][k] + s for a, k, s, _ in co.tolist()], dtype=np.int64)


def _spot_loop(c, cpu, batches, W, gen, **kw):
    """`batches` sample(1024, W) calls with the same generator, SPOT windows of each gathered on the device; then the
    CPU decoder at those windows' coordinates. Returns the number of windows checked."""
    n = 1024
    rows = torch.empty((batches * SPOT, W), dtype=torch.uint8, device="cuda")
    coords = torch.empty((batches * SPOT, 4), dtype=torch.int64, device="cuda")
    pick = torch.tensor([(k * 97 + 13) % n for k in range(SPOT)], device="cuda")
    for i in range(batches):
        x, co = c.sample(n, W, generator=gen, return_coords=True, **kw)          # status checked on every call
        rows[i * SPOT:(i + 1) * SPOT] = x.index_select(0, pick)
        coords[i * SPOT:(i + 1) * SPOT] = co.index_select(0, pick)
    co = coords.cpu().numpy()
    y = cpu.windows(co[:, 0], _stream_starts(c, co), W, rc=co[:, 3].astype(np.uint8), tokens=kw.get("tokens", False))
    x = rows.cpu().numpy()
    bad = [i for i in range(len(x)) if not np.array_equal(x[i], y[i])]
    assert not bad, f"{len(bad)} of {len(x)} windows differ, first at batch {bad[0] // SPOT}"
    return len(x)


def _whole_batch(c, cpu, n, W, gen, **kw):
    x, co = c.sample(n, W, generator=gen, return_coords=True, **kw)
    co = co.cpu().numpy()
    y = cpu.windows(co[:, 0], _stream_starts(c, co), W, rc=co[:, 3].astype(np.uint8), tokens=kw.get("tokens", False))
    assert np.array_equal(x.cpu().numpy(), y)
    return co


@pytest.mark.timeout(900)
def test_config1_tiny():
    d, c, cpu = _open("tiny")
    g = torch.Generator(device="cuda").manual_seed(0)
    _whole_batch(c, cpu, 256, 8192, g)                              # the configuration's workload, every window
    for a in range(len(c)):
        assert c.info(a)["block_hashes"]
        fa = c.fasta(a, verify=True)                                # every block's XXH3 and the FASTA's
        assert fa.startswith(b">")
        ok, h = c.check_full(a)
        assert ok and h == c.info(a)["fasta_xxh3"]
    _note("config 1: sample(256, 8192) equal, every block and FASTA hash verified")


@pytest.mark.timeout(900)
def test_config2_mid_tokens_rc():
    d, c, cpu = _open("mid")
    g = torch.Generator(device="cuda").manual_seed(0)
    kw = dict(tokens=True, reverse_complement=0.5)
    co = _whole_batch(c, cpu, 1024, 8192, g, **kw)
    assert 0 < co[:, 3].sum() < 1024
    checked = _spot_loop(c, cpu, 999, 8192, g, **kw)                 # with the first: the configuration's 1000 batches
    for a in (0, len(c) - 1):
        ok, _ = c.check_full(a)
        assert ok
    _note(f"config 2: 1000 batches, first whole + {checked} spot windows equal")


@pytest.mark.timeout(900)
def test_config3_mid16_fetch_and_w_sweep():
    d, c, cpu = _open("mid16", "q16k")
    assert c.block_size == 16384
    rng = np.random.default_rng(3)
    L, nf = 5000, 65536
    ctg = [(a, k, ln, off) for a in range(len(c)) for k, (_, _, ln, off, _) in enumerate(c.contigs(a)) if ln >= L]
    pick = rng.integers(0, len(ctg), nf)
    asm = np.array([ctg[i][0] for i in pick], dtype=np.int64)
    local = np.array([rng.integers(0, ctg[i][2] - L + 1) for i in pick], dtype=np.int64)
    start = np.array([ctg[i][3] for i in pick], dtype=np.int64) + local
    x = c.windows(torch.from_numpy(asm).cuda(), torch.from_numpy(start).cuda(), L).cpu().numpy()
    sel = np.arange(0, nf, 100)
    assert np.array_equal(x[sel], cpu.windows(asm[sel], start[sel], L))
    for i in range(0, 40):                                          # single fetch() calls give the batch's rows
        j = int(pick[i])
        y = c.fetch(ctg[j][0], ctg[j][1], int(local[i]), L).cpu().numpy()
        assert np.array_equal(y, x[i]), i
    g = torch.Generator(device="cuda").manual_seed(0)
    for W in (1024, 4096, 8192, 32768, 65536):
        xs, co = c.sample(1024, W, generator=g, return_coords=True)
        co = co.cpu().numpy()[::16]
        y = cpu.windows(co[:, 0], _stream_starts(c, co), W)
        assert np.array_equal(xs.cpu().numpy()[::16], y), W
    _note("config 3: 65,536 fetches (656 checked) and the W sweep equal")


@pytest.mark.timeout(900)
def test_config4_full_stream():
    import xxhash
    d, c, cpu = _open("full")
    n = c.info(0)["bases"]
    assert n > 3_000_000_000
    t = time.time()
    host = c.decode(0)
    _note(f"config 4: decode() of {n} bases in {time.time() - t:.2f} s")
    assert f"{xxhash.xxh3_64_intdigest(host.numpy()):016x}" == c.info(0)["bases_xxh3"]
    ok, h = c.check_full(0)
    assert ok and h == c.info(0)["fasta_xxh3"]
    rng = np.random.default_rng(4)
    W = 100_000
    start = rng.integers(0, n - W, 64).astype(np.int64)
    asm = np.zeros(64, np.int64)
    x = c.windows(torch.from_numpy(asm).cuda(), torch.from_numpy(start).cuda(), W).cpu().numpy()
    assert np.array_equal(x, cpu.windows(asm, start, W))
    assert all(np.array_equal(x[i], host.numpy()[start[i]:start[i] + W]) for i in range(64))
    # fetch() slices long enough for the large-call path (over 16,384 slots), the coordinates passed by value
    comp = np.frombuffer(bytes.maketrans(b"ACGTacgt", b"TGCAtgca"), dtype=np.uint8)
    for ci, (_, _, n_c, boff, _) in enumerate(c.contigs(0)[:2]):
        L = min(n_c, 80_000_000)
        s = (n_c - L) // 2
        y = c.fetch(0, ci, s, L).cpu().numpy()
        assert np.array_equal(y, host.numpy()[boff + s:boff + s + L]), ci
        yr = c.fetch(0, ci, s, L, reverse_complement=True).cpu().numpy()
        assert np.array_equal(yr, comp[host.numpy()[boff + s:boff + s + L]][::-1]), ci
    _note("config 4: base-stream XXH3, FASTA XXH3, windows and 80 Mbp fetches equal")


@pytest.mark.timeout(1200)
def test_config5_headline_spot_check():
    d, c, cpu = _open("headline")
    assert len(c) == 558
    g = torch.Generator(device="cuda").manual_seed(0)
    _whole_batch(c, cpu, 1024, 8192, g)
    _whole_batch(c, cpu, 1024, 8192, g, tokens=True, reverse_complement=0.5)
    checked = _spot_loop(c, cpu, 5000, 8192, g, reverse_complement=0.5)
    _note(f"config 5: 5000 uint8 batches, {checked} spot windows equal")
    checked += _spot_loop(c, cpu, 5000, 8192, g, tokens=True, reverse_complement=0.5)
    _note(f"config 5: 10,000 batches, {checked} spot windows equal")
    x, co = c.sample(65536, 8192, generator=g, return_coords=True)
    co = co.cpu().numpy()[::100]
    assert np.array_equal(x.cpu().numpy()[::100], cpu.windows(co[:, 0], _stream_starts(c, co), 8192))
    _note("config 5: a batch of 65,536 windows (656 checked) equal")
    _fetch_draw_check(c, cpu, 1000)
    _note("config 5: 1000 fetches of 1 .. 2^20 bases equal")
    # long single windows (245 covering blocks each, across contigs of one assembly's stream), plain and reverse
    # complemented with tokens
    rng = np.random.default_rng(55)
    W = 1_000_000
    asm = rng.integers(0, len(c), 16).astype(np.int64)
    start = np.array([rng.integers(0, c.info(int(a))["bases"] - W + 1) for a in asm], dtype=np.int64)
    rc = rng.integers(0, 2, 16).astype(np.uint8)
    a_t, s_t = torch.from_numpy(asm).cuda(), torch.from_numpy(start).cuda()
    assert np.array_equal(c.windows(a_t, s_t, W).cpu().numpy(), cpu.windows(asm, start, W))
    x = c.windows(a_t, s_t, W, reverse_complement=torch.from_numpy(rc).cuda().bool(), tokens=True).cpu().numpy()
    assert np.array_equal(x, cpu.windows(asm, start, W, rc=rc, tokens=True))
    _note("config 5: 16 windows of 1 Mbp equal, plain and reverse-complemented tokens")


def _fetch_draw_check(c, cpu, calls):
    """`calls` fetch() calls drawn as the reference's 558-assembly run draws them (scripts/cohort558.py:73-87):
    assembly uniform, contig by length, length 1 + 2^(20 u) capped at the contig, start uniform; each compared with the
    CPU decoder at the same stream coordinates (the reference compares with its own CPU decoder, :88-89)."""
    import random
    rng = random.Random(20261005)
    bad = []
    for i in range(calls):
        a = rng.randrange(len(c))
        ctgs = c.contigs(a)
        p = rng.randrange(sum(r[2] for r in ctgs))
        ci = 0
        while p >= ctgs[ci][2]:
            p -= ctgs[ci][2]
            ci += 1
        n = ctgs[ci][2]
        L = min(n, 1 + int(2 ** (rng.random() * 20)))
        s = rng.randrange(n - L + 1)
        z = c.fetch(a, ci, s, L).cpu().numpy()
        y = cpu.windows(np.array([a], dtype=np.int64), np.array([ctgs[ci][3] + s], dtype=np.int64), L)[0]
        if not np.array_equal(z, y):
            bad.append((i, a, ci, s, L))
    assert not bad, f"{len(bad)} of {calls} fetches differ from the CPU decoder, first {bad[0]}"
