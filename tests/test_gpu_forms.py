"""The compact resident forms on the GPU (reference tests/test_synth.py:148-159, test_compact_forms_resident_bytes):
Cohort.open(packed_reference=, compact_blocks=) holds fewer bytes and returns, byte for byte, what the CPU oracle
returns at the same coordinates - on the reference's fixtures (q1k, q4k, q16k), on the generated `mini` cohort (soft
mask, reverse-complemented pieces) and on `wide` (IUPAC runs in the reference, an N run across base 2^22, block
starts in the compact table's exception list). Run with -m gpu."""
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu

FORMS = [(True, False), (False, True), (True, True)]
IDS = ["packed", "compact", "packed-compact"]


def _starts(c, co):
    return np.array([c.contigs(int(a))[int(ci)][3] + int(s) for a, ci, s, _ in co], dtype=np.int64)


def _check(c, arcs, ref, seed, Ws, n=300):
    g = torch.Generator(device="cuda").manual_seed(seed)
    for W in Ws:
        for rc, tokens in ((False, False), (0.5, True), (0.5, False)):
            x, co = c.sample(n, W, generator=g, reverse_complement=rc, tokens=tokens, return_coords=True)
            co = co.cpu().numpy()
            y = O.windows(arcs, ref, co[:, 0], _starts(c, co), W, rc=co[:, 3].astype(np.uint8), tokens=tokens)
            assert np.array_equal(x.cpu().numpy(), y), (W, rc, tokens)


def _every_block(c, arcs, ref, Q):
    a, s = [], []
    for i, A in enumerate(arcs):
        for b in range(A.nblocks):
            a.append(i); s.append(min(b * Q + Q // 2, max(0, A.nbases - Q)))
    a, s = np.array(a, dtype=np.int64), np.array(s, dtype=np.int64)
    x = c.windows(torch.from_numpy(a).cuda(), torch.from_numpy(s).cuda(), Q)
    assert np.array_equal(x.cpu().numpy(), O.windows(arcs, ref, a, s, Q))


@pytest.mark.parametrize("form", FORMS, ids=IDS)
@pytest.mark.parametrize("ds", ["q1k", "q4k", "q16k"])
def test_forms_on_fixtures(fx, oracle_ref, ds, form):
    import panvram_amd
    base = panvram_amd.Cohort.open(fx["dirs"][ds], device="cuda", dataset=ds, reference=fx["ref"])
    c = panvram_amd.Cohort.open(fx["dirs"][ds], device="cuda", dataset=ds, reference=fx["ref"], packed_reference=form[0],
                                compact_blocks=form[1])
    assert (c.packed_reference, c.compact_blocks) == form
    assert c.resident_bytes()["total"] < base.resident_bytes()["total"]
    arcs = [O.Archive(os.path.join(fx["dirs"][ds], f"{nm}.{ds}.rr3")) for nm in c.names]
    _check(c, arcs, oracle_ref, 11, (1, 1000, 5000, 16385))
    _every_block(c, arcs, oracle_ref, c.block_size)
    # the reference's own check: windows at the default form's sampled coordinates are the same
    g = torch.Generator(device="cuda").manual_seed(5)
    x, co = base.sample(500, 3000, generator=g, return_coords=True)
    start = torch.from_numpy(_starts(base, co.cpu().numpy())).cuda()
    assert torch.equal(c.windows(co[:, 0], start, 3000), x)


@pytest.mark.parametrize("form", FORMS, ids=IDS)
@pytest.mark.parametrize("cohort", ["mini", "wide"])
def test_forms_on_generated_cohorts(request, cohort, form):
    import panvram_amd
    m = request.getfixturevalue(cohort)
    c = panvram_amd.Cohort.open(m["dir"], device="cuda", dataset="q4k", reference=m["ref"], packed_reference=form[0],
                                compact_blocks=form[1])
    ref = O.reference_bases(m["ref"])
    arcs = [O.Archive(p) for p in m["paths"]]
    _check(c, arcs, ref, 3, (100, 4096, 20000), n=400)
    _every_block(c, arcs, ref, 4096)
    for i, A in enumerate(arcs):
        assert np.array_equal(np.asarray(c.decode(i)), A.full(ref))
        ok, h = c.check_full(i)
        assert ok and h == c.info(i)["fasta_xxh3"], (i, h)
