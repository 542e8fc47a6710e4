"""pv_windows_hip_noalloc (the decode with its scratch in a file-scope device array) against pv_windows_hip with a
caller-allocated work buffer, through the C ABI: two calls in a row, the second smaller than the first (what the first
left in the array must not show), byte-identical rows and equal status words, and the clear refusal of a call whose
scratch would exceed the array. Run with -m gpu."""
import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle as O
from panvram_amd import _native as N

pytestmark = pytest.mark.gpu


def _coords(c, n, W, seed):
    """n valid (assembly, stream start) pairs of W-base windows, and a strand mask."""
    rng = np.random.default_rng(seed)
    asm, start = [], []
    for _ in range(n):
        a = int(rng.integers(len(c)))
        nb = c.info(a)["bases"]
        asm.append(a)
        start.append(int(rng.integers(0, nb - W + 1)))
    rc = rng.integers(0, 2, n).astype(np.uint8)
    return np.array(asm, np.int64), np.array(start, np.int64), rc


def _call(c, fn, asm, start, W, rc, tokens, apply_case, work=None):
    dev = c.device
    a, s = torch.from_numpy(asm).to(dev), torch.from_numpy(start).to(dev)
    r = torch.from_numpy(rc).to(dev) if rc is not None else None
    out = torch.full((asm.size, W), 0xAB, dtype=torch.uint8, device=dev)
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    err = N.errbuf()
    stream = torch.cuda.current_stream(dev).cuda_stream
    args = [c._Dref, a.data_ptr(), s.data_ptr(), asm.size, W, r.data_ptr() if r is not None else None, int(tokens), int(apply_case),
            out.data_ptr(), status.data_ptr()]
    if fn == "pv_windows_hip":
        args += [work.data_ptr() if work is not None else None, work.numel() if work is not None else 0]
    code = getattr(N.lib(), fn)(*args, stream, err, len(err))
    assert code == 0, err.value
    torch.cuda.synchronize()
    return out.cpu().numpy(), int(status.item())


@pytest.mark.parametrize("ds", ["q4k", "q16k"])
def test_noalloc_equals_work_buffer_entry(fx, oracle_ref, ds):
    import panvram_amd
    c = panvram_amd.Cohort.open(fx["dirs"][ds], device="cuda", dataset=ds, reference=fx["ref"])
    arcs = [O.Archive(f"{fx['dirs'][ds]}/{nm}.{ds}.rr3") for nm in c.names]
    for i, (n, W, tokens, apply_case, use_rc) in enumerate(((1024, 8192, False, True, False), (100, 3000, True, False, True))):
        asm, start, rc = _coords(c, n, W, 100 + i)
        rc = rc if use_rc else None
        wb = int(N.lib().pv_windows_work_bytes(c._Dref, n, W))
        work = torch.empty(max(wb, 1), dtype=torch.uint8, device=c.device)
        got, st_got = _call(c, "pv_windows_hip_noalloc", asm, start, W, rc, tokens, apply_case)
        want, st_want = _call(c, "pv_windows_hip", asm, start, W, rc, tokens, apply_case, work)
        assert st_got == st_want == 0, (ds, i)
        assert np.array_equal(got, want), (ds, i)
        y = O.windows(arcs, oracle_ref, asm, start, W, rc=rc, tokens=tokens, apply_case=apply_case)
        assert np.array_equal(got, y), (ds, i)


def test_noalloc_q16k_past_the_array_runs_without_scratch(fx):
    """At q16k a call whose light-block slots would not fit the array (22,000 windows of 8,192 bases: 44,000 slots,
    33.8 MB) runs with no scratch, every block by the windows kernel's wave decoder, and returns what pv_windows_hip
    with a work buffer returns (light lanes, whole-slot passes and the replay)."""
    import panvram_amd
    c = panvram_amd.Cohort.open(fx["dirs"]["q16k"], device="cuda", dataset="q16k", reference=fx["ref"])
    n, W = 22_000, 8192
    asm, start, _ = _coords(c, n, W, 7)
    work = torch.empty(int(N.lib().pv_windows_work_bytes(c._Dref, n, W)), dtype=torch.uint8, device=c.device)
    got, st_got = _call(c, "pv_windows_hip_noalloc", asm, start, W, None, False, True)
    want, st_want = _call(c, "pv_windows_hip", asm, start, W, None, False, True, work)
    assert st_got == st_want == 0
    assert np.array_equal(got, want)


def test_noalloc_status_and_refusal(fx):
    import panvram_amd
    c = panvram_amd.Cohort.open(fx["dirs"]["q4k"], device="cuda", dataset="q4k", reference=fx["ref"])
    n0 = c.info(0)["bases"]
    got, st = _call(c, "pv_windows_hip_noalloc", np.array([0, 0], np.int64), np.array([0, n0 - 5], np.int64), 6, None, False, True)
    assert st == 8                                            # a window outside its assembly
    assert np.array_equal(got[1], np.full(6, 0xAB, np.uint8))  # and its row is not written
    err = N.errbuf()
    z = torch.zeros(20_000, dtype=torch.int64, device="cuda")
    out = torch.empty((20_000, 8192), dtype=torch.uint8, device="cuda")
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    code = N.lib().pv_windows_hip_noalloc(c._Dref, z.data_ptr(), z.data_ptr(), 20_000, 8192, None, 0, 1, out.data_ptr(),
                                          status.data_ptr(), torch.cuda.current_stream().cuda_stream, err, len(err))
    assert code == N.PV_EARG and b"over the" in err.value and b"pv_windows_hip with a work buffer" in err.value


def test_graph_capture_refused(fx, oracle_ref):
    """A call that uses a work buffer refuses a stream that is being captured into a graph (its list and done words
    carry a number drawn on the host per launch, which a replay would repeat): PV_EARG from pv_windows_hip_noalloc and
    from pv_windows_hip with a work buffer, nothing launched into the capture; the same stream decodes normally once
    the capture has ended. The captured graph is never replayed."""
    import panvram_amd
    c = panvram_amd.Cohort.open(fx["dirs"]["q4k"], device="cuda", dataset="q4k", reference=fx["ref"])
    n, W = 64, 8192
    asm, start, _ = _coords(c, n, W, 3)
    a, s = torch.from_numpy(asm).cuda(), torch.from_numpy(start).cuda()
    out = torch.full((n, W), 0xAB, dtype=torch.uint8, device="cuda")
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    work = torch.empty(int(N.lib().pv_windows_work_bytes(c._Dref, n, W)), dtype=torch.uint8, device="cuda")
    side = torch.cuda.Stream()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    codes = {}
    with torch.cuda.graph(g, stream=side):
        status.zero_()                     # (one node, so that the graph is not empty)
        cs = torch.cuda.current_stream().cuda_stream
        for fn in ("pv_windows_hip_noalloc", "pv_windows_hip"):
            err = N.errbuf()
            args = [c._Dref, a.data_ptr(), s.data_ptr(), n, W, None, 0, 1, out.data_ptr(), status.data_ptr()]
            if fn == "pv_windows_hip":
                args += [work.data_ptr(), work.numel()]
            codes[fn] = (getattr(N.lib(), fn)(*args, cs, err, len(err)), err.value)
    torch.cuda.synchronize()
    for fn, (code, msg) in codes.items():
        assert code == N.PV_EARG and b"captured" in msg, (fn, code, msg)
    assert int((out != 0xAB).sum().item()) == 0             # nothing ran
    with torch.cuda.stream(side):
        got, st = _call(c, "pv_windows_hip_noalloc", asm, start, W, None, False, True)
    assert st == 0
    arcs = [O.Archive(f"{fx['dirs']['q4k']}/{nm}.q4k.rr3") for nm in c.names]
    assert np.array_equal(got, O.windows(arcs, oracle_ref, asm, start, W))
