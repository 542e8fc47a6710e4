"""sample's queue mode (Cohort.sample_queue): one resident kernel takes the (window, covering block) slots of every posted
call. It must return what the ring path returns from the same generator - the same draws, so the same coordinates and
rows - for every form (uint8, tokens, reverse complement, coordinates), at block sizes 4096 and 16384, with more calls
in flight than its descriptor ring holds, across the kernel leaving when idle and across stop_queue(). Rows are also
checked against `windows` at the returned coordinates (a path with no queue). Run with -m gpu."""
import time

import pytest
import torch

from panvram_amd import _native as N

pytestmark = pytest.mark.gpu


def _calls(W_set, n_set):
    """(n, W, reverse_complement, tokens) of a mixed sequence of calls."""
    out = []
    for i in range(40):
        rc = (False, 0.5, True)[i % 3]
        out.append((n_set[i % len(n_set)], W_set[i % len(W_set)], rc, i % 4 == 3))
    return out


def _run(c, seq, seed, queue):
    c.sample_queue = queue
    g = torch.Generator(device="cuda").manual_seed(seed)
    outs = []
    for n, W, rc, tok in seq:
        x, co = c.sample(n, W, generator=g, reverse_complement=rc, tokens=tok, return_coords=True, check=False)
        outs.append((x.clone(), co.clone()))          # enqueued on the caller's stream right after the call
        del x, co
    torch.cuda.synchronize()
    return outs


def _equal_to_windows(c, x, co, W, tokens=False):
    offs = [[ctg[3] for ctg in c.contigs(a)] for a in range(len(c))]
    cc = co.cpu().tolist()
    asm = torch.tensor([a for a, _, _, _ in cc], dtype=torch.int64, device="cuda")
    start = torch.tensor([offs[a][k] + s for a, k, s, _ in cc], dtype=torch.int64, device="cuda")
    rc = torch.tensor([r for _, _, _, r in cc], dtype=torch.uint8, device="cuda")
    return torch.equal(x, c.windows(asm, start, W, reverse_complement=rc, tokens=tokens))


@pytest.mark.timeout(300)
@pytest.mark.parametrize("ds", ["q4k", "q16k"])
def test_queue_equals_ring(fx, ds):
    import panvram_amd
    c = panvram_amd.Cohort.open(fx["dirs"][ds], device="cuda", dataset=ds, reference=fx["ref"])
    c.sample_streams = 3
    seq = _calls((5000, 1, 16385, 8192), (64, 1, 333, 1024 if ds == "q4k" else 700))
    ring = _run(c, seq, 7, False)
    queue = _run(c, seq, 7, True)
    assert c._queue is not None                        # the calls went through the queue
    for i, ((a, ca), (b, cb)) in enumerate(zip(ring, queue)):
        assert torch.equal(ca, cb), i
        assert torch.equal(a, b), (i, seq[i])
    n, W, rc, tok = seq[0]
    assert _equal_to_windows(c, queue[0][0], queue[0][1], W, tok)
    c.stop_queue()


@pytest.mark.timeout(300)
def test_queue_status_check_and_windows(mini):
    """Checked calls (a status read per call) in queue mode; each call's rows equal `windows` at its coordinates."""
    import panvram_amd
    c = panvram_amd.Cohort.open(mini["dir"], device="cuda", dataset="q4k", reference=mini["ref"])
    c.sample_queue = True
    g = torch.Generator(device="cuda").manual_seed(3)
    for i, (n, W) in enumerate(((256, 8192), (1000, 3000), (1, 1), (64, 40000))):
        tok = i % 2 == 1
        x, co = c.sample(n, W, generator=g, reverse_complement=0.5, tokens=tok, return_coords=True)
        assert _equal_to_windows(c, x, co, W, tok), (n, W)
    c.stop_queue()


@pytest.mark.timeout(300)
def test_queue_many_in_flight_idle_and_restart(fx):
    """Three times the descriptor ring's calls without a check (the host waits for ring entries), then a pause longer
    than the kernel's idle time (it leaves; the next call launches it again), then stop_queue() and more calls (a new
    queue): every call equals the ring path's call from the same generator."""
    import panvram_amd
    c = panvram_amd.Cohort.open(fx["dirs"]["q4k"], device="cuda", dataset="q4k", reference=fx["ref"])
    c.sample_streams = 2
    seq = [(128, 4096, 0.5, False)] * (3 * N.QUEUE_RING)

    def phases(queue):
        c.sample_queue = queue
        g = torch.Generator(device="cuda").manual_seed(11)
        res = []
        for phase in range(3):
            for n, W, rc, tok in seq if phase == 0 else seq[:5]:
                x = c.sample(n, W, generator=g, reverse_complement=rc, check=False)
                res.append(x.clone())
            torch.cuda.synchronize()
            if queue and phase == 0:
                time.sleep(0.6)                        # past the resident kernel's idle time
            if queue and phase == 1:
                c.stop_queue()
        return res

    ring, queue = phases(False), phases(True)
    assert len(ring) == len(queue)
    for i, (a, b) in enumerate(zip(ring, queue)):
        assert torch.equal(a, b), i
    c.stop_queue()
