"""Synthetic cohorts for the benchmark configurations (ctypes over libcohortgen.so, this directory).

`make(name, out_dir, **overrides)` writes `out_dir/reference.fa` and the haplotype archives of a preset:

  tiny      config 1: 4 contigs x 4 Mbp, 41 % GC, 10 N runs of 1-50 kbp, soft mask 50 % (runs geometric, mean 300);
            4 haplotypes: SNV 1e-3, indels 1e-4 (geometric mean 3, max 50), 2 SVs per contig (1-20 kbp); q4k
  mid       config 2: 256 Mbp over 16 contigs (log-uniform 1-40 Mbp, rescaled), same base / N / mask model;
            32 haplotypes, every contig cut into 2-30 pieces; q4k
  mid16     config 3: config 2 encoded at q16k
  full      config 4: 3.1 Gbp over 24 contigs on a chromosome-like size profile (248 Mbp .. 16.5 kbp), 8 % of bases in
            centromere-like N regions holding 171-bp satellite arrays of 1-3 Mbp; 1 haplotype + 200 SVs of 1-100 kbp
  headline  config 5: the config-4 reference + 558 haplotypes (SNV 1e-3, indels 1e-4, 200 SVs of 1-100 kbp each), q4k

Details the configurations leave open are fixed here: uniform alternative base for SNVs, 50/50 insertion /
deletion for indels and SVs, random upper-case inserted sequence, case following the source position, pieces of
fragmented contigs reverse-complemented with probability 1/2 (config 2), line widths 60 / 70 alternating.
Test and benchmark infrastructure only.
"""
import ctypes
import math
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "libcohortgen.so")


class RefParams(ctypes.Structure):
    _fields_ = [("seed", ctypes.c_uint64), ("ncontigs", ctypes.c_int32), ("line_width", ctypes.c_int32),
                ("lengths", ctypes.POINTER(ctypes.c_uint64)), ("gc", ctypes.c_double),
                ("n_runs", ctypes.c_int32), ("n_run_min", ctypes.c_uint64), ("n_run_max", ctypes.c_uint64),
                ("centro_frac", ctypes.c_double), ("sat_min", ctypes.c_uint64), ("sat_max", ctypes.c_uint64),
                ("sat_monomer", ctypes.c_int32), ("mask_mean", ctypes.c_double), ("iupac_runs", ctypes.c_int32),
                ("n_run_at", ctypes.c_uint64)]


class AsmParams(ctypes.Structure):
    _fields_ = [("seed", ctypes.c_uint64), ("n_asm", ctypes.c_int32), ("Q", ctypes.c_int32), ("line_width_a", ctypes.c_int32),
                ("line_width_b", ctypes.c_int32), ("block_hashes", ctypes.c_int32), ("threads", ctypes.c_int32),
                ("zstd_level", ctypes.c_int32), ("snv_rate", ctypes.c_double), ("indel_rate", ctypes.c_double),
                ("indel_mean", ctypes.c_double), ("indel_max", ctypes.c_uint32), ("sv_per_contig", ctypes.c_int32),
                ("sv_per_asm", ctypes.c_int32), ("sv_min", ctypes.c_uint64), ("sv_max", ctypes.c_uint64),
                ("frag_min", ctypes.c_int32), ("frag_max", ctypes.c_int32), ("rc_piece", ctypes.c_double), ("prefix", ctypes.c_char_p),
                ("ins_odd", ctypes.c_double)]


# chromosome-like size profile (Mbp, T2T-like ordering), rescaled so the 23 large contigs + 16.5 kbp sum to 3.1 Gbp
_CHR = [248.4, 242.7, 201.1, 193.6, 182.0, 172.1, 160.6, 146.3, 150.6, 134.8, 135.1, 133.3, 113.6, 101.2, 99.8, 96.3,
        84.3, 80.1, 61.7, 66.2, 45.1, 51.3, 154.3]


def _chrom_lengths():
    big = 3_100_000_000 - 16_569
    s = sum(_CHR)
    out = [int(x / s * big) for x in _CHR]
    out[0] += big - sum(out)
    return out + [16_569]


def _mid_lengths(seed=2):
    import random
    r = random.Random(seed)
    raw = [math.exp(r.uniform(math.log(1e6), math.log(40e6))) for _ in range(16)]
    s = sum(raw)
    out = [int(x / s * 256_000_000) for x in raw]
    out[0] += 256_000_000 - sum(out)
    return out


def presets():
    base_asm = dict(snv_rate=1e-3, indel_rate=1e-4, indel_mean=3.0, indel_max=50, line_width_a=60, line_width_b=70,
                    block_hashes=1, zstd_level=3, frag_min=0, frag_max=0, rc_piece=0.0, sv_per_contig=0, sv_per_asm=0, ins_odd=0.0)
    base_ref = dict(gc=0.41, line_width=60, n_runs=10, n_run_min=1, n_run_max=50_000, centro_frac=0.0, sat_min=0, sat_max=0,
                    sat_monomer=171, mask_mean=300.0, iupac_runs=0, n_run_at=0)
    tiny = dict(ref=dict(base_ref, seed=101, lengths=[4_000_000] * 4),
                asm=dict(base_asm, seed=201, n_asm=4, Q=4096, sv_per_contig=2, sv_min=1, sv_max=20_000))
    mid = dict(ref=dict(base_ref, seed=102, lengths=_mid_lengths(), n_runs=40),
               asm=dict(base_asm, seed=202, n_asm=32, Q=4096, sv_per_contig=2, sv_min=1, sv_max=20_000, frag_min=2, frag_max=30, rc_piece=0.5))
    mid16 = dict(ref=mid["ref"], asm=dict(mid["asm"], Q=16384))
    big_ref = dict(base_ref, seed=104, lengths=_chrom_lengths(), n_runs=0, centro_frac=0.08, sat_min=1_000_000, sat_max=3_000_000,
                   mask_mean=0.0)
    full = dict(ref=big_ref, asm=dict(base_asm, seed=204, n_asm=1, Q=4096, sv_per_asm=200, sv_min=1_000, sv_max=100_000))
    headline = dict(ref=big_ref, asm=dict(base_asm, seed=205, n_asm=558, Q=4096, sv_per_asm=200, sv_min=1_000, sv_max=100_000,
                                          block_hashes=0))
    # small stand-ins with the same edit model, for CPU tests of the generator itself
    mini = dict(ref=dict(base_ref, seed=103, lengths=[300_000, 200_000, 50_000], n_runs=3, n_run_max=5_000),
                asm=dict(base_asm, seed=203, n_asm=3, Q=4096, sv_per_contig=2, sv_min=1, sv_max=8_000, frag_min=2, frag_max=5, rc_piece=0.5,
                         snv_rate=3e-3, indel_rate=1e-3, ins_odd=0.004))
    return {"tiny": tiny, "mid": mid, "mid16": mid16, "full": full, "headline": headline, "mini": mini}


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def make(name, out_dir, threads=None, ref=None, asm=None):
    """Write preset `name` into out_dir (created). ref / asm: dicts overriding preset fields.
    Returns a dict of statistics (bases, blocks, payload bytes, files, file bytes, reference bases)."""
    if not os.path.exists(LIB):
        build()
    p = presets()[name]
    rp, ap = dict(p["ref"], **(ref or {})), dict(p["asm"], **(asm or {}))
    os.makedirs(out_dir, exist_ok=True)
    L = ctypes.CDLL(LIB)
    L.cg_make_cohort.argtypes = [ctypes.c_char_p, ctypes.POINTER(RefParams), ctypes.POINTER(AsmParams), ctypes.POINTER(ctypes.c_uint64),
                                 ctypes.c_char_p, ctypes.c_size_t]
    L.cg_make_cohort.restype = ctypes.c_int
    lens = (ctypes.c_uint64 * len(rp["lengths"]))(*rp["lengths"])
    R = RefParams(seed=rp["seed"], ncontigs=len(rp["lengths"]), line_width=rp["line_width"], lengths=lens, gc=rp["gc"],
                  n_runs=rp["n_runs"], n_run_min=rp["n_run_min"], n_run_max=rp["n_run_max"], centro_frac=rp["centro_frac"],
                  sat_min=rp["sat_min"], sat_max=rp["sat_max"], sat_monomer=rp["sat_monomer"], mask_mean=rp["mask_mean"],
                  iupac_runs=rp["iupac_runs"], n_run_at=rp["n_run_at"])
    A = AsmParams(prefix=b"h", threads=int(threads or min(16, os.cpu_count() or 1)), **{k: v for k, v in ap.items()})
    stats = (ctypes.c_uint64 * 6)()
    err = ctypes.create_string_buffer(1024)
    if L.cg_make_cohort(os.fsencode(out_dir), ctypes.byref(R), ctypes.byref(A), stats, err, len(err)):
        raise RuntimeError(err.value.decode())
    keys = ("bases", "blocks", "payload_bytes", "files", "file_bytes", "ref_bases")
    return dict(zip(keys, list(stats)))
