"""Corrupt payloads on the GPU decode paths (reference tests/test_synth.py:127-145 and the status bit 1 of
csrc/pv_cuda.cu:37): a bit flipped inside one block's payload makes `windows` and `sample` raise RuntimeError with
status bit 1 exactly when the CPU oracle fails that block, and return the oracle's bytes when the flipped stream still
decodes. Each of the kernel paths that decode a block is covered: the light decoder's lanes (payloads of at most 32
bytes), the heavy role's waves (longer payloads in small calls), the heavy list's waves and the whole-slot waves past
its areas (calls past 16,384 slots), and the windows kernel's own wave decoder (light_decode off, and the longer
payloads at q16k). Run with -m gpu."""
import os
import shutil

import numpy as np
import pytest
import torch

from oracle import oracle as O

pytestmark = pytest.mark.gpu


def _flip(src, dst_dir, arc, b, k):
    """Copy of archive `src` into dst_dir with bit k % 8 of payload byte (k * 7) % len of block b flipped."""
    raw = bytearray(open(src, "rb").read())
    n = arc.payload_len(b)
    pos = arc.payload_file_offset(b) + (k * 7) % n
    raw[pos] ^= 1 << (k % 8)
    os.makedirs(dst_dir, exist_ok=True)
    p = os.path.join(dst_dir, os.path.basename(src))
    open(p, "wb").write(bytes(raw))
    return p


def _oracle_block(path, ref, b, Q, nbases):
    """Case-applied bytes of block b as the oracle decodes them, or None when the oracle fails the block."""
    a = O.Archive(path)
    blen = min(Q, nbases - b * Q)
    try:
        return O.windows([a], ref, np.array([0]), np.array([b * Q]), blen)[0]
    except ValueError:
        return None


def _gpu_block(c, b, Q, nbases, repeat=None):
    """Block b as windows() returns it (one window; or `repeat` windows of it, all rows), or None on status bit 1."""
    blen = min(Q, nbases - b * Q)
    n = repeat or 1
    try:
        x = c.windows(torch.zeros(n, dtype=torch.int64), torch.full((n,), b * Q, dtype=torch.int64), blen).cpu().numpy()
        return x if repeat else x[0]
    except RuntimeError as e:
        assert "status 1" in str(e), str(e)
        return None


@pytest.mark.parametrize("ds", ["q4k", "q16k"])
def test_corrupt_block_status_follows_oracle(fx, oracle_ref, tmp_path, ds):
    import panvram_amd
    src = os.path.join(fx["dirs"][ds], f"synthA.{ds}.rr3")
    arc = O.Archive(src)
    Q, nb, nbases = arc.Q, arc.nblocks, arc.nbases
    ctg_len = arc.records()[0][1]                       # contig 1 starts at base 0
    inside = [b for b in range(nb) if (b + 1) * Q <= ctg_len]
    pl = {b: arc.payload_len(b) for b in inside}
    light = [b for b in inside if pl[b] <= 32][:3]
    heavy = sorted((b for b in inside if pl[b] > 32), key=lambda b: -pl[b])[:3]
    assert heavy and (light or ds == "q16k")
    failed = decoded = 0
    for b in light + heavy:
        for k in range(4):
            d = str(tmp_path / f"{ds}_{b}_{k}")
            p = _flip(src, d, arc, b, k)
            shutil.copy(fx["ref"], os.path.join(d, "synth_ref.fa"))
            want = _oracle_block(p, oracle_ref, b, Q, nbases)
            c = panvram_amd.Cohort.open(d, device="cuda", dataset=ds)
            for light_decode in (True, False):
                c.light_decode = light_decode
                got = _gpu_block(c, b, Q, nbases)
                assert (got is None) == (want is None), (ds, b, k, light_decode)
                if want is not None:
                    assert np.array_equal(got, want), (ds, b, k, light_decode)
                # fetch() (coordinates by value): the block as a slice of the first contig, which starts at base 0
                try:
                    fz = c.fetch(0, 0, b * Q, min(Q, nbases - b * Q)).cpu().numpy()
                    assert want is not None and np.array_equal(fz, want), (ds, b, k, light_decode, "fetch")
                except RuntimeError as e:
                    assert "status 1" in str(e) and want is None, (ds, b, k, light_decode, "fetch", str(e))
                if light_decode:
                    # the same block in every window of a call past the one-kernel path (8200 windows of two slots):
                    # at q4k the header pass, the heavy list's areas, the whole-slot waves past them, or the light
                    # lanes; at q16k the light lanes and the wave decoder of the one-kernel path
                    got = _gpu_block(c, b, Q, nbases, repeat=8200)
                    assert (got is None) == (want is None), (ds, b, k, "large")
                    if want is not None:
                        assert all(np.array_equal(r, want) for r in got), (ds, b, k, "large")
                # sample(): every window is the whole first contig (the only start of a window that long), so each
                # covers block b
                try:
                    x = c.sample(4, ctg_len, generator=torch.Generator(device="cuda").manual_seed(k))
                    assert want is not None, (ds, b, k, light_decode)
                    full = O.windows([O.Archive(p)], oracle_ref, np.zeros(1, np.int64), np.zeros(1, np.int64), ctg_len)[0]
                    assert all(np.array_equal(r, full) for r in x.cpu().numpy())
                except RuntimeError as e:
                    assert "status 1" in str(e) and want is None, (ds, b, k, light_decode, str(e))
            failed += want is None
            decoded += want is not None
    assert failed > 0
