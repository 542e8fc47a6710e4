"""GPU parity on the reference's fixture archives (the coverage of reference tests/test_synth.py:38-124 on the HIP
path): every window, slice and whole contig from panvram_amd on the GPU is byte-identical to the CPU oracle at the
same coordinates (and through it to the archives' own block / stream / FASTA XXH3). Run with -m gpu."""
import os
import random

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

DS = ["q1k", "q4k", "q16k"]


def _open(fx, ds):
    import panvram_amd
    return panvram_amd.Cohort.open(fx["dirs"][ds], device="cuda", dataset=ds, reference=fx["ref"])


def _arcs(fx, ds, c):
    return [O.Archive(os.path.join(fx["dirs"][ds], f"{nm}.{ds}.rr3")) for nm in c.names]


def _starts(c, co):
    return np.array([c.contigs(int(a))[int(ci)][3] + int(s) for a, ci, s, _ in co], dtype=np.int64)


@pytest.mark.parametrize("ds", DS)
def test_sample_windows_equal_oracle(fx, oracle_ref, ds):
    c = _open(fx, ds)
    assert c.names == ["synthA", "synthB"] and c.block_size == {"q1k": 1024, "q4k": 4096, "q16k": 16384}[ds]
    A = _arcs(fx, ds, c)
    g = torch.Generator(device="cuda").manual_seed(7)
    for W in (1, 13, 1024, 4096, 5000, 16385):
        x, co = c.sample(300, W, generator=g, return_coords=True)
        assert x.shape == (300, W) and x.dtype == torch.uint8 and x.device.type == "cuda"
        co = co.cpu().numpy()
        assert (co[:, 3] == 0).all()
        for a, ci, s, _ in co:                      # windows never cross contigs
            assert s + W <= c.contigs(int(a))[int(ci)][2]
        y = O.windows(A, oracle_ref, co[:, 0], _starts(c, co), W)
        assert np.array_equal(x.cpu().numpy(), y), (ds, W)
    for W in (100, 8192):
        x, co = c.sample(200, W, generator=g, reverse_complement=0.5, tokens=True, return_coords=True)
        co = co.cpu().numpy()
        assert 0 < co[:, 3].sum() < 200
        y = O.windows(A, oracle_ref, co[:, 0], _starts(c, co), W, rc=co[:, 3].astype(np.uint8), tokens=True)
        assert np.array_equal(x.cpu().numpy(), y), (ds, W)


@pytest.mark.parametrize("ds", DS)
def test_fetch_and_whole_contigs(fx, oracle_ref, ds):
    c = _open(fx, ds)
    A = _arcs(fx, ds, c)
    full = [a.full(oracle_ref) for a in A]
    comp = bytes.maketrans(b"ACGTacgt", b"TGCAtgca")
    tok = bytes(0 if ch in b"Aa" else 1 if ch in b"Cc" else 2 if ch in b"Gg" else 3 if ch in b"Tt" else 4 for ch in range(256))
    rng = random.Random(11)
    for _ in range(200):
        a = rng.randrange(len(c))
        ctgs = c.contigs(a)
        ci = rng.randrange(len(ctgs))
        name, _, n, boff, _ = ctgs[ci]
        L = min(n, int(2 ** (rng.random() * 15)))
        s = rng.randrange(n - L + 1)
        rc, tk = rng.random() < 0.3, rng.random() < 0.3
        y = c.fetch(c.names[a] if rng.random() < 0.5 else a, name if rng.random() < 0.5 else ci, s, L, reverse_complement=rc, tokens=tk)
        want = full[a][boff + s:boff + s + L].tobytes()
        if rc:
            want = want.translate(comp)[::-1]
        if tk:
            want = want.translate(tok)
        assert y.shape == (L,) and y.cpu().numpy().tobytes() == want
    for a in range(len(c)):
        for name, _, n, boff, _ in c.contigs(a):
            assert c.fetch(a, name, 0, n).cpu().numpy().tobytes() == full[a][boff:boff + n].tobytes()


@pytest.mark.parametrize("ds", ["q4k", "q16k"])
def test_fetch_status_is_per_call(fx, oracle_ref, tmp_path, ds):
    """fetch() over a block that fails to decode raises (status bit 1), and the next fetch, of another block, returns
    that block's bytes: every fetch starts from a zero status word (at q4k the decode kernel writes the call's record
    and clears it, at q16k a kernel of its own does)."""
    import shutil
    import panvram_amd
    src = os.path.join(fx["dirs"][ds], f"synthA.{ds}.rr3")
    A = O.Archive(src)
    full = A.full(oracle_ref)
    Q, b = A.Q, 3
    raw = open(src, "rb").read()
    d = tmp_path / ds
    d.mkdir()
    bad = None
    for k in range(8 * min(A.payload_len(b), 8)):          # a bit of block b's payload whose flip the oracle refuses
        cand = bytearray(raw)
        cand[A.payload_file_offset(b) + k // 8] ^= 1 << (k % 8)
        (d / f"synthA.{ds}.rr3").write_bytes(bytes(cand))
        try:
            O.Archive(str(d / f"synthA.{ds}.rr3")).block(oracle_ref, b)
        except ValueError:
            bad = cand
            break
    assert bad is not None
    shutil.copy(fx["ref"], d / "synth_ref.fa")
    c = panvram_amd.Cohort.open(str(d), device="cuda", dataset=ds)

    def where(pos):                                           # stream position -> (contig index, position in it)
        for ci, (_, _, n, boff, _) in enumerate(c.contigs(0)):
            if boff <= pos < boff + n:
                return ci, pos - boff
        raise AssertionError(pos)

    for rep in range(3):
        ci, s = where(b * Q + 17 + rep)
        with pytest.raises(RuntimeError, match="status 1"):
            c.fetch(0, ci, s, 1)
        for g in (b + 2, b - 2):
            ci, s = where(g * Q + 5 + rep)
            L = min(100, c.contigs(0)[ci][2] - s)
            y = c.fetch(0, ci, s, L, reverse_complement=bool(rep & 1))
            want = full[g * Q + 5 + rep:g * Q + 5 + rep + L].tobytes()
            if rep & 1:
                want = want.translate(bytes.maketrans(b"ACGTacgt", b"TGCAtgca"))[::-1]
            assert y.cpu().numpy().tobytes() == want, (rep, g)


def test_gpu_equals_cpu_at_returned_coordinates(fx, oracle_ref):
    """reference tests/test_synth.py:79-89 - sample(4096, 777, rc=0.5) on the GPU == the CPU decoder's windows."""
    c = _open(fx, "q4k")
    g = torch.Generator(device="cuda").manual_seed(3)
    x, co = c.sample(4096, 777, generator=g, reverse_complement=0.5, return_coords=True)
    co = co.cpu().numpy()
    y = O.windows(_arcs(fx, "q4k", c), oracle_ref, co[:, 0], _starts(c, co), 777, rc=co[:, 3].astype(np.uint8), threads=4)
    assert np.array_equal(x.cpu().numpy(), y)
    R = O.RefDecoder.open(fx["ref"], [os.path.join(fx["dirs"]["q4k"], f"{nm}.q4k.rr3") for nm in c.names])
    if R is not None:
        assert np.array_equal(x.cpu().numpy(), R.windows(co[:, 0], _starts(c, co), 777, rc=co[:, 3].astype(np.uint8), threads=4))


@pytest.mark.parametrize("ds", DS)
def test_sample_coordinates_follow_the_reference_draws(fx, ds):
    """sample's coordinates equal the reference's (panvram/cohort.py:168-194) for the same generator state: a copy of
    the generator replays its draws (torch.randint(0, total, (n,)), then torch.rand(n) for a probability), the oracle
    maps them to (assembly, contig, start, strand), and both generators end in the same state. Through the shape's
    prepared path (repeated calls), the first call, and the per-call path (token_ids as a tensor); n of 1, 300 and 5,000 (the
    large-call path)."""
    c = _open(fx, ds)
    lengths = [[ct[2] for ct in c.contigs(a)] for a in range(len(c))]
    g = torch.Generator(device="cuda").manual_seed(11)
    for n, W, rc in ((1, 1, False), (300, 13, 0.5), (300, 4096, True), (5000, 777, 0.25), (300, 13, 0.5), (300, 13, 0.5)):
        for ids in (None, (0, 1, 2, 3, 4), torch.arange(5)):      # no ids, the prepared path's ids, the per-call path's
            g2 = torch.Generator(device="cuda")
            g2.set_state(g.get_state())
            _, total = O.sample_coords(lengths, W, np.zeros(0, dtype=np.int64))
            u = torch.randint(0, total, (n,), generator=g2, device="cuda", dtype=torch.int64).cpu().numpy()
            r = torch.rand(n, generator=g2, device="cuda").cpu().numpy() if rc not in (True, False) else None
            want, _ = O.sample_coords(lengths, W, u, rnd=r, p=rc, rc_all=rc is True)
            x, co = c.sample(n, W, generator=g, reverse_complement=rc, tokens=ids is not None, return_coords=True, token_ids=ids)
            assert x.shape == (n, W)
            assert np.array_equal(co.cpu().numpy(), want), (ds, n, W, rc, ids)
            assert torch.equal(g.get_state(), g2.get_state()), (ds, n, W, rc, ids)


@pytest.mark.parametrize("ds", DS)
def test_fasta_decode_check_full(fx, oracle_ref, ds):
    c = _open(fx, ds)
    A = _arcs(fx, ds, c)
    for i in range(len(c)):
        assert c.fasta(i) == A[i].fasta(oracle_ref)
        ok, h = c.check_full(i)
        assert ok and h == c.info(i)["fasta_xxh3"]
        d = c.decode(i, chunk=50_000)        # many chunks, ragged last one
        assert np.array_equal(d.numpy(), A[i].full(oracle_ref))


def test_windows_crossing_blocks_and_contigs(fx, oracle_ref):
    """windows() takes stream offsets: windows may cross contig boundaries and start / end on block edges."""
    c = _open(fx, "q1k")
    A = _arcs(fx, "q1k", c)
    n0 = c.info(0)["bases"]
    starts = [0, 1, 1023, 1024, 1025, 2047, n0 - 3000, n0 - 1025, n0 - 1024]
    for W in (1, 1023, 1024, 1025, 3000):
        st = [s for s in starts if 0 <= s and s + W <= n0]
        x = c.windows(torch.zeros(len(st), dtype=torch.int64), torch.tensor(st), W)
        y = O.windows(A, oracle_ref, np.zeros(len(st), np.int64), np.array(st), W)
        assert np.array_equal(x.cpu().numpy(), y)


@pytest.mark.parametrize("ds,light", [("q4k", True), ("q4k", False), ("q1k", True), ("q16k", True), ("q16k", False)])
def test_large_call_windows_api(fx, oracle_ref, ds, light):
    """windows() over 6000 windows of 8192 bases (18,000 slots at q4k, 54,000 at q1k: past the one-kernel path's 16,384):
    the header pass, the heavy kernel (long blocks decoded into heavy areas beside the light lanes), the spill pass (the
    fixtures' long blocks outnumber the areas several times over), then the replay; random strands, tokens, and windows
    that start on and next to block edges. At q16k (9000 windows, 18,000 slots) there are no heavy areas: the long
    blocks all go to the spill pass. With light_decode off every block is in the windows kernel."""
    c = _open(fx, ds)
    c.light_decode = light
    A = _arcs(fx, ds, c)
    rng = np.random.default_rng(23)
    n, W = (9000 if ds == "q16k" else 6000), 8192
    asm = rng.integers(0, len(c), n).astype(np.int64)
    nb = np.array([c.info(int(a))["bases"] for a in asm], dtype=np.int64)
    start = (rng.random(n) * (nb - W + 1)).astype(np.int64)
    start[:40] = (start[:40] // c.block_size) * c.block_size + np.arange(40) % 3 - 1   # on, before and after a block edge
    start = np.clip(start, 0, nb - W)
    rc = rng.integers(0, 2, n).astype(np.uint8)
    for tokens in (False, True):
        x = c.windows(torch.from_numpy(asm).cuda(), torch.from_numpy(start).cuda(), W,
                      reverse_complement=torch.from_numpy(rc.astype(bool)).cuda(), tokens=tokens)
        y = O.windows(A, oracle_ref, asm, start, W, rc=rc, tokens=tokens, threads=8)
        assert np.array_equal(x.cpu().numpy(), y), tokens


@pytest.mark.parametrize("ds", ["q4k", "q1k"])
def test_large_call_timed_and_untimed_orders(fx, oracle_ref, ds):
    """A large sample() call on the caller's stream with timing events (kernel_events) runs its kernels in the timed
    order: the heavy waves into their areas, the whole-slot pass, then a replay of every slot between the runtime's two
    events. Without events the heavy waves replay their own slots and the whole-slot pass follows the replay of the
    light slots. Both return the oracle's rows at the call's coordinates: 6000 windows of 8192 bases with random
    strands (18,000 slots at q4k, 54,000 at q1k; on the fixtures most long blocks go to the whole-slot pass)."""
    c = _open(fx, ds)
    A = _arcs(fx, ds, c)
    c.sample_streams = 0
    for timed in (True, False):
        c.kernel_events = [] if timed else None
        g = torch.Generator(device="cuda").manual_seed(31)
        x, co = c.sample(6000, 8192, generator=g, reverse_complement=0.5, return_coords=True)
        torch.cuda.synchronize()
        if timed:
            assert len([e for e in c.kernel_events if e[1] is not None]) == 1
        c.kernel_events = None
        co = co.cpu().numpy()
        y = O.windows(A, oracle_ref, co[:, 0], _starts(c, co), 8192, rc=co[:, 3].astype(np.uint8), threads=8)
        assert np.array_equal(x.cpu().numpy(), y), timed


def test_q16k_large_call_long_windows_and_token_ids(fx, oracle_ref):
    """The q16k large-call path beyond the replay's window buffer (1,000 windows of 20,000 bases: 3,000 slots, the
    replay with the whole block in LDS) against the oracle, and token_ids through the window-buffer replay (3,000
    windows of 6,000 bases) against the loader's lut[windows(tokens=True)]."""
    c = _open(fx, "q16k")
    A = _arcs(fx, "q16k", c)
    rng = np.random.default_rng(29)
    for n, W in ((1000, 20000), (3000, 6000)):
        asm = rng.integers(0, len(c), n).astype(np.int64)
        nb = np.array([c.info(int(a))["bases"] for a in asm], dtype=np.int64)
        start = (rng.random(n) * (nb - W + 1)).astype(np.int64)
        rc = rng.integers(0, 2, n).astype(bool)
        a_t, s_t, rc_t = torch.from_numpy(asm).cuda(), torch.from_numpy(start).cuda(), torch.from_numpy(rc).cuda()
        if W > 8192:
            x = c.windows(a_t, s_t, W, reverse_complement=rc_t)
            y = O.windows(A, oracle_ref, asm, start, W, rc=rc.astype(np.uint8), threads=8)
            assert np.array_equal(x.cpu().numpy(), y)
        else:
            lut = torch.tensor([11, 22, 33, 44, 55], dtype=torch.int64)
            ids = c.windows(a_t, s_t, W, reverse_complement=rc_t, token_ids=lut)
            tok = c.windows(a_t, s_t, W, reverse_complement=rc_t, tokens=True)
            assert torch.equal(ids, lut.cuda()[tok.long()])
            y = O.windows(A, oracle_ref, asm, start, W, rc=rc.astype(np.uint8), tokens=True, threads=8)
            assert np.array_equal(tok.cpu().numpy(), y)


def test_q16k_window_buffer_follows_w(fx, oracle_ref):
    """The q16k large-call replay allocates its window buffer, and the case bitmask right after it, for the call's W
    (W + 64 bytes rounded to 32): calls of over 2,048 slots at W from 1 to 8,192, on and next to the rounding steps,
    with random strands, uint8 and tokens, against the oracle."""
    c = _open(fx, "q16k")
    A = _arcs(fx, "q16k", c)
    rng = np.random.default_rng(31)
    for W in (1, 16, 31, 33, 100, 1000, 4033, 8192):
        n = 2100                                      # 4,200 slots: the large-call path
        asm = rng.integers(0, len(c), n).astype(np.int64)
        nb = np.array([c.info(int(a))["bases"] for a in asm], dtype=np.int64)
        start = (rng.random(n) * (nb - W + 1)).astype(np.int64)
        rc = rng.integers(0, 2, n).astype(np.uint8)
        a_t, s_t, rc_t = torch.from_numpy(asm).cuda(), torch.from_numpy(start).cuda(), torch.from_numpy(rc.astype(bool)).cuda()
        for tokens in (False, True):
            x = c.windows(a_t, s_t, W, reverse_complement=rc_t, tokens=tokens)
            y = O.windows(A, oracle_ref, asm, start, W, rc=rc, tokens=tokens, threads=8)
            assert np.array_equal(x.cpu().numpy(), y), (W, tokens)


def test_status_and_argument_errors(fx):
    c = _open(fx, "q4k")
    n0 = c.info(0)["bases"]
    with pytest.raises(RuntimeError, match="status 8"):
        c.windows(torch.tensor([0]), torch.tensor([n0 - 5]), 6)
    with pytest.raises(RuntimeError, match="status 8"):
        c.windows(torch.tensor([2]), torch.tensor([0]), 6)
    with pytest.raises(RuntimeError, match="status 8"):
        c.windows(torch.tensor([0]), torch.tensor([-1]), 6)
    x = c.windows(torch.tensor([0, 1]), torch.tensor([5, 5]), 0)
    assert x.shape == (2, 0)
    x = c.windows(torch.zeros(0, dtype=torch.int64), torch.zeros(0, dtype=torch.int64), 10)
    assert x.shape == (0, 10)
    with pytest.raises(IndexError):
        name, _, n, _, _ = c.contigs(0)[0]
        c.fetch(0, name, n - 5, 6)
    with pytest.raises(ValueError):
        c.sample(4, 10 ** 9)
    # the reference's argument checks (csrc/pv_cuda.cu:119-128), before anything of the call's size is allocated
    z = torch.zeros(1, dtype=torch.int64).expand(1 << 29)
    with pytest.raises(RuntimeError, match="too many blocks in one call"):
        c.windows(z, z, 16385)
    with pytest.raises(RuntimeError, match="^W$"):
        c.windows(torch.tensor([0]), torch.tensor([0]), 1 << 31)
    with pytest.raises(RuntimeError, match="assembly and start counts differ"):
        c.windows(torch.tensor([0, 0]), torch.tensor([0]), 5)


def test_corrupt_payload_never_silent(fx, oracle_ref, tmp_path):
    """reference tests/test_synth.py:127-145 on the GPU path: a payload bit flipped -> fasta() raises FormatError or
    returns exactly the source FASTA; sample() either raises (status 1) or returns the oracle's bytes."""
    import panvram_amd
    import shutil
    raw = bytearray(open(os.path.join(fx["dirs"]["q4k"], "synthA.q4k.rr3"), "rb").read())
    want = O.Archive(os.path.join(fx["dirs"]["q4k"], "synthA.q4k.rr3")).fasta(oracle_ref)
    caught = 0
    for k in range(40):
        b = bytearray(raw)
        p = len(b) - 1 - (k * 97) % 3000
        b[p] ^= 1 << (k % 8)
        d = tmp_path / f"c{k}"
        d.mkdir()
        (d / "synthA.q4k.rr3").write_bytes(bytes(b))
        shutil.copy(fx["ref"], d / "synth_ref.fa")
        c = panvram_amd.Cohort.open(str(d), device="cuda")
        try:
            fa = c.fasta(0)
        except panvram_amd.FormatError:
            caught += 1
            continue
        assert fa == want
    assert caught > 0
