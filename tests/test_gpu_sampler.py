"""The sample coordinate kernel (pv_sample_coords_hip) against torch's own searchsorted / gather on the same draws, and
Cohort.sample's returned coordinates against the reference's torch formulation from the same generator state
(reference panvram/cohort.py:176-189). Run with -m gpu."""
import ctypes

import numpy as np
import pytest
import torch

from panvram_amd import _native as N

pytestmark = pytest.mark.gpu


def _torch_coords(length, asm, local, boff, W, u, r, p, mode):
    room = (length - W + 1).clamp_min(0)
    cum = torch.cumsum(room, 0)
    k = torch.searchsorted(cum, u, right=True)
    pos = u - (cum[k] - room[k])
    strand = (torch.ones_like(u) if mode == 1 else (r < p).to(torch.int64) if mode == 2 else torch.zeros_like(u))
    return torch.stack([asm[k], local[k], pos, strand], 1), boff[k] + pos


@pytest.mark.parametrize("m", [1, 5, 64, 65, 4097, 20000])
def test_coords_kernel_equals_torch(m):
    dev = "cuda"
    g = torch.Generator(device="cpu").manual_seed(m)
    length = torch.randint(0, 50_000, (m,), generator=g) * (torch.rand(m, generator=g) < 0.8)   # many too-short contigs
    length[m // 2] = 60_000
    asm = torch.randint(0, 600, (m,), generator=g)
    local = torch.randint(0, 30, (m,), generator=g)
    boff = torch.randint(0, 1 << 40, (m,), generator=g)
    length, asm, local, boff = (t.to(dev, torch.int64) for t in (length, asm, local, boff))
    L = N.lib()
    for W, mode, p in ((1, 0, 0.0), (4096, 2, 0.3), (50_001, 1, 1.0), (8192, 2, 1.0)):
        room = (length - W + 1).clamp_min(0)
        cum = torch.cumsum(room, 0)
        total = int(cum[-1])
        n = 3000
        u = torch.randint(0, total, (n,), device=dev, dtype=torch.int64)
        u[:3] = torch.tensor([0, total - 1, int(cum[0]) if int(cum[0]) < total else 0], device=dev)
        r = torch.rand(n, device=dev)
        wasm = torch.empty(n, dtype=torch.int64, device=dev)
        wstart = torch.empty(n, dtype=torch.int64, device=dev)
        wrc = torch.empty(n, dtype=torch.uint8, device=dev)
        coords = torch.empty((n, 4), dtype=torch.int64, device=dev)
        status = torch.full((1,), 77, dtype=torch.int32, device=dev)
        err = N.errbuf()
        code = L.pv_sample_coords_hip(cum.data_ptr(), m, asm.data_ptr(), local.data_ptr(), boff.data_ptr(), u.data_ptr(),
                                      r.data_ptr(), p, mode, n, wasm.data_ptr(), wstart.data_ptr(), wrc.data_ptr(),
                                      coords.data_ptr(), status.data_ptr(), torch.cuda.current_stream().cuda_stream, err, len(err))
        assert code == 0, err.value
        want, want_start = _torch_coords(length, asm, local, boff, W, u, r, p, mode)
        assert torch.equal(coords, want), (m, W)
        assert torch.equal(wasm, want[:, 0]) and torch.equal(wstart, want_start)
        if mode:
            assert torch.equal(wrc.to(torch.int64), want[:, 3])
        assert int(status.item()) == 0


def test_cohort_sample_coords_follow_the_generator(fx):
    import panvram_amd
    c = panvram_amd.Cohort.open(fx["dirs"]["q4k"], device="cuda", dataset="q4k", reference=fx["ref"])
    ctg = [(a, k, ln, off) for a in range(len(c)) for k, (_, _, ln, off, _) in enumerate(c.contigs(a))]
    length = torch.tensor([t[2] for t in ctg], device="cuda")
    asm = torch.tensor([t[0] for t in ctg], device="cuda")
    local = torch.tensor([t[1] for t in ctg], device="cuda")
    boff = torch.tensor([t[3] for t in ctg], device="cuda")
    c.sample_streams = 0              # one ring position: the second call of a shape runs the first call's plan
    for W, rc in ((1, False), (5000, 0.3), (16385, True)):
        g = torch.Generator(device="cuda").manual_seed(W)
        for rep in range(2):
            state = g.get_state()
            _, co = c.sample(500, W, generator=g, reverse_complement=rc, return_coords=True)
            after = g.get_state()
            g.set_state(state)
            room = (length - W + 1).clamp_min(0)
            total = int(torch.cumsum(room, 0)[-1])
            u = torch.randint(0, total, (500,), generator=g, device="cuda", dtype=torch.int64)
            mode = 1 if rc is True else 2 if rc else 0
            r = torch.rand(500, generator=g, device="cuda") if mode == 2 else None
            want, _ = _torch_coords(length, asm, local, boff, W, u, r, float(rc), mode)
            assert torch.equal(co, want), (W, rep)
            assert torch.equal(g.get_state(), after), (W, rep)   # the generator advanced as torch's draws advance it


@pytest.mark.parametrize("wait", ["event", "counter"])
@pytest.mark.parametrize("streams", [0, 1, 3, 7])
def test_stream_ring_equals_caller_stream(fx, streams, wait):
    """sample() on a ring of streams returns what it returns on the caller's stream (sample_streams = 0), and the
    caller's stream sees each call's results: copies enqueued right after each call, on the caller's stream, hold
    the same bytes. Covers a ring larger than HIP's hardware queue count (streams then share queues), both ways of
    making the caller wait, and ring streams used for the first time (a fresh cohort's ring)."""
    import panvram_amd
    c = panvram_amd.Cohort.open(fx["dirs"]["q4k"], device="cuda", dataset="q4k", reference=fx["ref"])
    c.sample_wait = wait
    runs = {}
    for k in (0, streams):
        c.sample_streams = k
        g = torch.Generator(device="cuda").manual_seed(1234)
        outs = []
        for i in range(24):
            W = (5000, 1, 16385)[i % 3]
            x, co = c.sample(64, W, generator=g, reverse_complement=0.5 if i % 2 else False, return_coords=True,
                             check=False)
            outs.append((x.clone(), co.clone()))         # enqueued on the caller's stream right after the call
            del x, co                                    # the buffer goes back to the allocator at once
        torch.cuda.synchronize()
        runs[k] = outs
    for (a, ca), (b, cb) in zip(runs[0], runs[streams]):
        assert torch.equal(ca, cb) and torch.equal(a, b)


@pytest.mark.parametrize("streams", [0, 2])
def test_plans_across_buffer_growth(fx, streams):
    """Repeated shapes run through call plans; a larger call on the same ring position replaces that stream's work
    buffer (and drops the plans on it). Every call's rows equal `windows` at its returned coordinates (a path with no
    plans), including the calls right after the growth."""
    import panvram_amd
    c = panvram_amd.Cohort.open(fx["dirs"]["q4k"], device="cuda", dataset="q4k", reference=fx["ref"])
    c.sample_streams = streams
    g = torch.Generator(device="cuda").manual_seed(99)
    offs = [[ctg[3] for ctg in c.contigs(a)] for a in range(len(c))]
    for i, n in enumerate((64, 64, 64, 512, 64, 64, 2048, 64, 512, 512)):
        W = 3000
        x, co = c.sample(n, W, generator=g, reverse_complement=0.5 if i % 2 else False, return_coords=True)
        cc = co.cpu().tolist()
        asm = torch.tensor([a for a, _, _, _ in cc], dtype=torch.int64, device="cuda")
        start = torch.tensor([offs[a][k] + s for a, k, s, _ in cc], dtype=torch.int64, device="cuda")
        rc = torch.tensor([r for _, _, _, r in cc], dtype=torch.uint8, device="cuda")
        y = c.windows(asm, start, W, reverse_complement=rc)
        assert torch.equal(x, y), (i, n)


def test_timed_calls_between_plan_calls(fx):
    """With kernel_events set, one call in kernel_events_every runs the general path with timing events (the windows
    kernel's own start and end from its launch) and the others run plans; all return the rows `windows` gives at their
    coordinates, and every timed call leaves a (start, mid, end) triple with positive, ordered times."""
    import panvram_amd
    c = panvram_amd.Cohort.open(fx["dirs"]["q4k"], device="cuda", dataset="q4k", reference=fx["ref"])
    c.sample_streams, c.kernel_events, c.kernel_events_every = 3, [], 3
    g = torch.Generator(device="cuda").manual_seed(7)
    offs = [[ctg[3] for ctg in c.contigs(a)] for a in range(len(c))]
    for i in range(9):
        x, co = c.sample(200, 4500, generator=g, return_coords=True)
        cc = co.cpu().tolist()
        asm = torch.tensor([a for a, _, _, _ in cc], dtype=torch.int64, device="cuda")
        start = torch.tensor([offs[a][k] + s for a, k, s, _ in cc], dtype=torch.int64, device="cuda")
        assert torch.equal(x, c.windows(asm, start, 4500)), i
    torch.cuda.synchronize()
    ev, c.kernel_events = c.kernel_events, None
    ev = [e for e in ev if e[1] is not None]     # `windows` calls append (start, None, end) on every call
    assert len(ev) == 3
    for t0, tm, t1 in ev:
        decode_ms, windows_ms = t0.elapsed_time(tm), tm.elapsed_time(t1)
        assert 0 < decode_ms < 1000 and 0 < windows_ms < 1000, (decode_ms, windows_ms)


def test_true_and_one_draw_as_the_reference(fx):
    """reverse_complement=True draws no uniform numbers and 1 / 1.0 draw torch.rand(n) (reference panvram/cohort.py:182-189):
    calls alternating the two on one generator leave it where the reference's torch calls leave it, whichever form a
    call plan was first made for."""
    import panvram_amd
    c = panvram_amd.Cohort.open(fx["dirs"]["q4k"], device="cuda", dataset="q4k", reference=fx["ref"])
    ctg = [ln for a in range(len(c)) for (_, _, ln, _, _) in c.contigs(a)]
    W, n = 700, 128
    total = sum(max(0, ln - W + 1) for ln in ctg)
    g, r = (torch.Generator(device="cuda").manual_seed(5) for _ in range(2))
    for i, rc in enumerate((True, 1.0, True, 1, 1.0, True, True, 1)):
        _, co = c.sample(n, W, generator=g, reverse_complement=rc, return_coords=True)
        torch.randint(0, total, (n,), generator=r, device="cuda", dtype=torch.int64)
        if rc is not True:
            torch.rand(n, generator=r, device="cuda")
        assert torch.equal(g.get_state(), r.get_state()), (i, rc)
        assert int(co[:, 3].sum()) == n                  # p = 1: every window reverse-complemented either way


@pytest.mark.parametrize("streams", [0, 3])
def test_repeated_shape_allocates_nothing_new(fx, streams):
    """After the first call of a shape (which sets up every ring stream: work buffer, wait counter, a warm row pool),
    later calls open no new segment of torch's caching allocator and set up no stream again."""
    import panvram_amd
    c = panvram_amd.Cohort.open(fx["dirs"]["q4k"], device="cuda", dataset="q4k", reference=fx["ref"])
    c.sample_streams = streams
    g = torch.Generator(device="cuda").manual_seed(17)
    for rc in (False, 0.5):
        x = c.sample(1024, 8192, generator=g, reverse_complement=rc, check=False)
        del x
        torch.cuda.synchronize()
        seg0 = torch.cuda.memory_stats()["segment.all.allocated"]
        prepared = len(c._prepared)
        for _ in range(60):
            x = c.sample(1024, 8192, generator=g, reverse_complement=rc, check=False)
            del x
        torch.cuda.synchronize()
        assert torch.cuda.memory_stats()["segment.all.allocated"] == seg0, rc
        assert len(c._prepared) == prepared
        c.sample(1024, 8192, generator=g, reverse_complement=rc)         # status of the last call checked


@pytest.mark.parametrize("coords", [False, True])
def test_pooled_rows_reused_only_after_the_caller_passes(fx, coords):
    """With the ring, sample's rows (and coordinates) come from the library's own pools as DLPack tensors. A row the
    caller holds is not handed out again; a row freed while the caller's stream still has work reading it is handed out
    again only after that work (copies enqueued on the caller's stream before the free keep the call's bytes). Every
    row equals the caller-stream path's (no pool) from the same generator, and the pools' rows were reused."""
    import ctypes
    import panvram_amd
    c = panvram_amd.Cohort.open(fx["dirs"]["q4k"], device="cuda", dataset="q4k", reference=fx["ref"])
    n, W, calls = 64, 5000, 200

    def run(streams):
        c.sample_streams = streams
        g = torch.Generator(device="cuda").manual_seed(5)
        held, copies = [], []
        for i in range(calls):
            x = c.sample(n, W, generator=g, reverse_complement=0.5, check=False, return_coords=coords)
            x, co = x if coords else (x, None)
            if i % 10 == 0:
                held.append((x, co))                     # kept by the caller: its rows are not reused
            copies.append((x[:, :96].clone(), co.clone() if coords else None))     # enqueued before the free below
            del x, co
        torch.cuda.synchronize()
        return held, copies

    want_held, want_copies = run(0)
    held, copies = run(3)
    assert all(x.is_cuda and x.dtype == torch.uint8 and x.shape == (n, W) for x, _ in held)
    assert all(co.is_cuda and co.dtype == torch.int64 and co.shape == (n, 4) for _, co in held if coords)
    for i, (a, b) in enumerate(zip(want_copies + want_held, copies + held)):
        assert torch.equal(a[0], b[0]), i
        assert not coords or torch.equal(a[1], b[1]), i
    plan = next(p for k, p in c._fast.items() if p.pool is not None and k[5] == coords)
    assert (plan.cpool is not None) == coords
    for pool in (plan.pool, plan.cpool) if coords else (plan.pool,):
        total, free = ctypes.c_int32(), ctypes.c_int32()
        assert N.lib().pv_rows_count(pool, ctypes.byref(total), ctypes.byref(free)) == 0
        assert 0 < total.value < calls                   # fewer rows than calls: rows were handed out again
        assert free.value == total.value - len(held)


def test_token_ids_on_the_ring_equal_the_per_call_path(fx):
    """sample with five plain int ids takes a prepared plan of its own on the ring (int64 rows from the library's row
    pool); an ids tensor takes the per-call path. Call after call, both equal the uint8 token output of the same draws
    mapped through the ids."""
    import panvram_amd
    c = panvram_amd.Cohort.open(fx["dirs"]["q4k"], device="cuda", dataset="q4k", reference=fx["ref"])
    c.sample_streams = 3
    ids = (7, 11, 13, 17, 19)
    lut = torch.tensor(ids, dtype=torch.int64, device="cuda")
    for how in (ids, torch.tensor(ids)):
        g = torch.Generator(device="cuda").manual_seed(23)
        g2 = torch.Generator(device="cuda").manual_seed(23)
        held = []
        for i in range(40):
            x = c.sample(256, 3000, generator=g, reverse_complement=0.5, tokens=True, token_ids=how)
            y = c.sample(256, 3000, generator=g2, reverse_complement=0.5, tokens=True)
            assert x.dtype == torch.int64 and x.shape == (256, 3000)
            assert torch.equal(x, lut[y.long()]), (type(how), i)
            if i % 8 == 0:
                held.append((x, lut[y.long()]))
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(held):
            assert torch.equal(a, b), (type(how), i)
    assert any(k[-1] == ids for k in c._fast)


def test_token_ids_written_on_the_caller_stream_just_before(fx):
    """An ids tensor that a kernel on the caller's stream writes right before sample() (behind ~20 ms of other work
    there): the ring stream the call runs on waits for it, so every row holds the new ids, never the old ones."""
    import panvram_amd
    c = panvram_amd.Cohort.open(fx["dirs"]["q4k"], device="cuda", dataset="q4k", reference=fx["ref"])
    c.sample_streams = 3
    new = torch.tensor((7, 11, 13, 17, 19), dtype=torch.int64, device="cuda")
    for i in range(4):
        ids = torch.full((5,), 1000 + i, dtype=torch.int64, device="cuda")
        torch.cuda.synchronize()
        torch.cuda._sleep(50_000_000)             # the caller's stream busy for a while
        ids.copy_(new)                            # then the ids written there
        g = torch.Generator(device="cuda").manual_seed(31 + i)
        g2 = torch.Generator(device="cuda").manual_seed(31 + i)
        x = c.sample(256, 3000, generator=g, reverse_complement=0.5, tokens=True, token_ids=ids)
        y = c.sample(256, 3000, generator=g2, reverse_complement=0.5, tokens=True)
        assert torch.equal(x, new[y.long()]), i


def test_ring_streams_run_at_once(fx):
    """sample's ring streams run at the same time as each other and as the caller's stream: pv_streams_concurrent
    (two one-wave kernels of 100 us released together end together) holds for every pair the ring picked, and not for
    a stream and itself (one kernel after the other)."""
    import panvram_amd
    from panvram_amd import cohort as C
    if N.lib().pv_dispatch_serialised():
        pytest.skip("dispatches serialised by a tool: nothing runs at once")
    if C._hw_queues() > C._PICK_QUEUES:
        pytest.skip("above 8 hardware queues the ring takes torch's pool streams as they come")
    c = panvram_amd.Cohort.open(fx["dirs"]["q4k"], device="cuda", dataset="q4k", reference=fx["ref"])
    c.sample_streams = 3
    c.sample(64, 5000, generator=torch.Generator(device="cuda").manual_seed(5))
    torch.cuda.synchronize()
    L, err, flag = N.lib(), N.errbuf(), ctypes.c_int32()

    def concurrent(a, b):
        assert L.pv_streams_concurrent(a.cuda_stream, b.cuda_stream, ctypes.byref(flag), err, len(err)) == 0, err.value
        return flag.value == 1

    caller = torch.cuda.current_stream()
    ring = list(dict.fromkeys(c._ring))
    assert len(c._ring) == 3 and ring
    assert not concurrent(caller, caller)
    for i, s in enumerate(ring):
        assert concurrent(caller, s), i
        for r in ring[:i]:
            assert concurrent(r, s), i


def test_stream_ops_agree_with_the_public_calls():
    """The stream triple the sample path reads and sets (torch's private bindings where checked) equals what
    torch.cuda.current_stream reports, for the default stream and for a side stream made current."""
    from panvram_amd import _streams as S
    ops = S.StreamOps()
    dev = torch.cuda.current_device()
    cur = torch.cuda.current_stream(dev)
    assert tuple(ops.get(dev)) == (cur.stream_id, cur.device_index, cur.device_type)
    if torch.__version__.startswith(S.CHECKED):
        assert ops.private
    side = torch.cuda.Stream()
    ops.set(side.stream_id, side.device_index, side.device_type)
    try:
        now = torch.cuda.current_stream(dev)
        assert (now.stream_id, now.device_index, now.device_type) == (side.stream_id, side.device_index, side.device_type)
        assert tuple(ops.get(dev)) == (side.stream_id, side.device_index, side.device_type)
    finally:
        ops.set(cur.stream_id, cur.device_index, cur.device_type)
    assert torch.cuda.current_stream(dev) == cur
