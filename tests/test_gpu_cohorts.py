"""GPU parity on generated cohorts (tests/cohortgen `mini`): long literal runs with N and escape bytes (the literal-pair
path and its fallback), soft-mask runs, reverse-complemented pieces, fragmented contigs. Every byte the HIP path
returns equals the CPU oracle at the same coordinates. Run with -m gpu."""
import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _open(mini):
    import panvram_amd
    return panvram_amd.Cohort.open(mini["dir"], device="cuda", dataset="q4k", reference=mini["ref"])


def _starts(c, co):
    return np.array([c.contigs(int(a))[int(ci)][3] + int(s) for a, ci, s, _ in co], dtype=np.int64)


@pytest.mark.parametrize("light", [True, False])
def test_mini_sample_equals_oracle(mini, light):
    """Both decoders: blocks with short payloads one lane per block (then replayed by the windows kernel), and every
    block in the windows kernel."""
    c = _open(mini)
    c.light_decode = light
    ref = O.reference_bases(mini["ref"])
    arcs = [O.Archive(p) for p in mini["paths"]]
    assert [a.path for a in arcs] == [c.info(i)["path"] for i in range(len(c))]
    g = torch.Generator(device="cuda").manual_seed(3)
    for W in (1, 100, 4096, 8192, 20000):
        for tokens in (False, True):
            x, co = c.sample(400, W, generator=g, reverse_complement=0.5, tokens=tokens, return_coords=True)
            co = co.cpu().numpy()
            y = O.windows(arcs, ref, co[:, 0], _starts(c, co), W, rc=co[:, 3].astype(np.uint8), tokens=tokens)
            assert np.array_equal(x.cpu().numpy(), y), (W, tokens)


def test_mini_large_batch(mini):
    """A batch past the one-kernel path (6000 windows of 8192 bases = 18,000 slots > 16,384): the header pass and the
    heavy list. Half of this cohort's blocks are long, far more than the list's areas (one per 64 slots), so most long
    blocks go to spill_kernel, which does them whole."""
    c = _open(mini)
    ref = O.reference_bases(mini["ref"])
    arcs = [O.Archive(p) for p in mini["paths"]]
    g = torch.Generator(device="cuda").manual_seed(11)
    x, co = c.sample(6000, 8192, generator=g, reverse_complement=0.5, return_coords=True)
    co = co.cpu().numpy()
    y = O.windows(arcs, ref, co[:, 0], _starts(c, co), 8192, rc=co[:, 3].astype(np.uint8), threads=8)
    assert np.array_equal(x.cpu().numpy(), y)


@pytest.mark.parametrize("light", [True, False])
def test_mini_every_block(mini, light):
    """One window per block of every assembly (block-aligned, and shifted by half a block), against the oracle."""
    c = _open(mini)
    c.light_decode = light
    ref = O.reference_bases(mini["ref"])
    arcs = [O.Archive(p) for p in mini["paths"]]
    for shift in (0, 2048):
        a, s = [], []
        for i, A in enumerate(arcs):
            for b in range(A.nblocks):
                st = min(b * 4096 + shift, A.nbases - 4096)
                a.append(i); s.append(st)
        a, s = np.array(a, dtype=np.int64), np.array(s, dtype=np.int64)
        x = c.windows(torch.from_numpy(a).cuda(), torch.from_numpy(s).cuda(), 4096)
        y = O.windows(arcs, ref, a, s, 4096)
        assert np.array_equal(x.cpu().numpy(), y), shift


def test_mini_decode_and_check_full(mini):
    c = _open(mini)
    ref = O.reference_bases(mini["ref"])
    for i, p in enumerate(mini["paths"]):
        A = O.Archive(p)
        full = c.decode(i)
        assert np.array_equal(full.cpu().numpy() if hasattr(full, "cpu") else np.asarray(full), A.full(ref)), p
        ok, h = c.check_full(i)
        assert ok and h == c.info(i)["fasta_xxh3"], (p, h)


def test_mini_device_fasta_equals_host_fasta(mini):
    """The device FASTA layout (pv_fasta_layout_hip) over random piece boundaries == the host-built, hash-verified
    FASTA; check_full agrees with the header with and without `out`."""
    from panvram_amd import _native as N
    c = _open(mini)
    L = N.lib()
    rng = np.random.default_rng(2)
    for i in range(len(c)):
        want = c.fasta(i, verify=True)
        rows, dev_rows, dev_hdrs, F = c._fasta_plan(i)
        assert F == len(want)
        n = c.info(i)["bases"]
        bases = c.windows(torch.tensor([i]), torch.tensor([0]), n)[0]
        got = torch.empty(F, dtype=torch.uint8, device="cuda")
        cuts = sorted(set([0, F] + [int(x) for x in rng.integers(0, F, 7)]))
        for f0, f1 in zip(cuts[:-1], cuts[1:]):
            b0, b1 = c._bases_before(rows, f0), c._bases_before(rows, f1)
            err = N.errbuf()
            code = L.pv_fasta_layout_hip(bases[b0:].data_ptr(), b0, b1 - b0, dev_rows.data_ptr(), len(rows), dev_hdrs.data_ptr(),
                                         f0, f1 - f0, got[f0:].data_ptr(), torch.cuda.current_stream().cuda_stream, err, len(err))
            assert code == 0, err.value
        assert got.cpu().numpy().tobytes() == want, i
        ok, h = c.check_full(i)
        assert ok and h == c.info(i)["fasta_xxh3"]
        out = torch.zeros(n, dtype=torch.uint8, pin_memory=True)
        ok2, h2 = c.check_full(i, out=out)
        assert ok2 and h2 == h
        assert torch.equal(out, bases.cpu())


def test_token_ids_fused(mini):
    """windows / sample with token_ids == the loader's lut[windows(tokens=True).long()] (reference
    tools/megatron/panvram_loader.py:96-97), with reverse complement."""
    c = _open(mini)
    lut = torch.tensor([50, 7, 1 << 40, -3, 99], dtype=torch.int64, device="cuda")
    g = torch.Generator(device="cuda").manual_seed(9)
    state = g.get_state()
    ids, co = c.sample(300, 3000, generator=g, reverse_complement=0.5, return_coords=True, token_ids=lut)
    g.set_state(state)
    tok, co2 = c.sample(300, 3000, generator=g, reverse_complement=0.5, return_coords=True, tokens=True)
    assert ids.dtype == torch.int64 and ids.shape == (300, 3000)
    assert torch.equal(co, co2) and torch.equal(ids, lut[tok.long()])
    a = co[:, 0]
    s = torch.tensor(_starts(c, co.cpu().numpy()), device="cuda")
    rc = co[:, 3].bool()
    w_ids = c.windows(a, s, 3000, reverse_complement=rc, token_ids=lut.tolist())
    assert torch.equal(w_ids, ids)
