#!/usr/bin/env python3
"""bench.py - the headline benchmark of the MI355X refrel3 v1 decode path.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config headline|tiny|mid|mid16|full] [--assemblies A]

A step is one `Cohort.sample(n=1024, W=8192)` call (uint8 windows, the reference's default form, reference
scripts/cohort558.py:116-133) over a synthetic cohort built on this box by tests/cohortgen (the headline preset by
default: a 3.1 Gbp reference + 558 haplotypes, q4k, resident in HBM). W untimed steps, then K timed steps between two
device syncs, check=False inside (as the reference's bench.py:41-43), the decode status checked after.

One JSON line on stdout (progress on stderr). Beside `value` it carries:
  roofline      per kernel of a call, timed with HIP events on the launch stream in a pass of launches one at a time
                after the timed loop, against 8 TB/s HBM: the decode kernel (algorithmic bytes: the covering blocks'
                payloads + 16 B of block table each, the touched assemblies' entropy models, the draws) and the
                windows kernel (the reference bytes the
                copies read, and W output bytes per window). The line's own `achieved`/`frac` are the whole call's
                algorithmic bytes over the dominant (longer) kernel's time; `kernels` has each kernel's own bytes over
                its own time, `call` all algorithmic bytes over both kernels' time.
                `traffic` is the HBM bytes per launch the committed rocprofv3 FETCH_SIZE / WRITE_SIZE passes measured
                (profiles/headline_traffic.json). The decode kernel is latency-bound: `latency` sets it beside one
                call of the batch's longest covering block alone, its serial rANS chain. Beside them both kernels'
                times while launches overlap on the ring (an untimed pass after the timed loop)
  sync_per_call the reference's own protocol for its published figure (scripts/cohort558.py:54-72): a sync before and
                after each sample(1024, 8192, return_coords=True) with the status check on, median of --sync-calls
                calls; on the ring and (sync_per_call_caller_stream) on the caller's stream
  default_queues the ring's rate and the synchronous figure under HIP's default of 4 hardware queues (a 3-stream
                ring), from a child process started before this one makes any GPU call
  cpu_baseline  the reference's own CPU decoder (oracle/_ref, built from its sources; the oracle port if absent) on
                the same coordinates, host threads (<= 16) and one thread
  variants      the tokens + reverse-complement form (with events on each launch), BASELINE config 2's form (tokens
                + rc 0.5 + coordinates, timed as the main loop and spot-checked), a large-n batch (n = 65536) for the
                roofline fraction, the compact resident forms (packed_reference + compact_blocks) on the same workload,
                and single synchronous fetch() latency over 1000 coordinates drawn as the reference's 558-assembly run
                draws them, each fetch checked against the CPU decoder, the ten slowest timed again with events
  spot_check    windows of the first timed batch against the CPU decoder, byte for byte
"""
import argparse
import json
import os
import random
import shutil
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "windows/s (n=1024, W=8192, 558-asm q4k); decoded bytes/s vs HBM peak"
PUBLISHED = 1_401_185        # reference's published sample(1024, 8192), 558 HPRC asm q4k, RTX PRO 6000 Blackwell
                             # (reference logs/colab-cohort558-blackwell-2026-10-05.txt:16)
HBM_PEAK = 8.0e12            # MI355X HBM3E, bytes/s
TABLE_BYTES = 16             # block table bytes read per block: u32 offset, i64 start diagonal, u32 first case run
MODEL_BYTES = 2 * 1827       # an assembly's entropy model: a 16-bit frequency per symbol of its 61 contexts (1,827
                             # symbols; format section 2.3), the input every block decode of that assembly needs
ROOF_LAUNCHES = 50           # launches of the roofline pass (one at a time, events on each)


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def data_dir(args):
    if args.data:
        return args.data
    base = os.environ.get("PANVRAM_BENCH_DIR")
    if not base:
        base = "/dev/shm" if os.path.isdir("/dev/shm") and shutil.disk_usage("/dev/shm").free > 60e9 else (os.environ.get("TMPDIR") or "/tmp")
    name = args.config + (f"_a{args.assemblies}" if args.assemblies else "")
    return os.path.join(base, "panvram_bench_" + name)


def ensure_cohort(args, d):
    from tests import cohortgen as G
    stamp = os.path.join(d, "stamp.json")
    want = {"config": args.config, "assemblies": args.assemblies, "version": 2}
    if os.path.exists(stamp) and json.load(open(stamp)) == want:
        log(f"bench: reusing cohort in {d}")
        return None
    shutil.rmtree(d, ignore_errors=True)
    os.makedirs(d)
    t = time.time()
    threads = min(16, os.cpu_count() or 1)
    st = G.make(args.config, d, threads=threads, asm={"n_asm": args.assemblies} if args.assemblies else None)
    st["seconds"] = round(time.time() - t, 1)
    json.dump(want, open(stamp, "w"))
    log(f"bench: generated {args.config} cohort in {st['seconds']} s ({threads} threads): {st}")
    return st


def measured_traffic(args, c):
    """HBM bytes per launch of each kernel of this workload, as the rocprofv3 FETCH_SIZE / WRITE_SIZE passes whose
    summary is committed in profiles/ measured them (each counter scaled by its reading for a plain copy of known
    size): {kernel: bytes}; {} for a workload that was not profiled."""
    p = os.path.join(ROOT, "profiles", "headline_traffic.json")
    if args.assemblies or c.block_size != 4096 or not os.path.exists(p):
        return {}
    if args.config == "full":
        w = json.load(open(p))["workloads"].get("full")
    elif args.config == "headline" and args.W == 8192:
        w = json.load(open(p))["workloads"].get(f"n={args.n}")
    else:
        return {}
    return {k: v["bytes_per_launch"] for k, v in w["kernels"].items()} if w else {}


def b_parts(c, off_host, asm_rec, coords, W, refbytes):
    """Algorithmic bytes of one batch by part: (payload + the 16 B of block table this build reads, per covering block;
    the entropy models of the assemblies the batch touches; the reference bytes the covering blocks' copies read;
    W output bytes per window)."""
    Q = c.block_size
    pay = ref = out = 0
    touched = set()
    for a, s in coords:
        blk_base = int(asm_rec[a, 1])
        touched.add(a)
        for b in range(s // Q, (s + W - 1) // Q + 1):
            bb = blk_base + b
            pay += int(off_host[bb + 1]) - int(off_host[bb]) + TABLE_BYTES
            ref += refbytes(a, b)
        out += W
    return pay, MODEL_BYTES * len(touched), ref, out


def longest_blocks(c, off_host, asm_rec, coords, W, k=3):
    """The k covering blocks of a batch with the longest payloads: (payload bytes, assembly, block)."""
    Q = c.block_size
    seen = {}
    for a, s in coords:
        for b in range(s // Q, (s + W - 1) // Q + 1):
            bb = int(asm_rec[a, 1]) + b
            seen[(a, b)] = int(off_host[bb + 1]) - int(off_host[bb])
    return sorted(((p, a, b) for (a, b), p in seen.items()), reverse=True)[:k]


def sync_per_call(c, n, W, g, calls):
    """The anchor's own protocol (reference scripts/cohort558.py:54-72): a device sync before and after each
    sample(n, W, return_coords=True) call with its status check on, median over `calls` calls. The shape's first call
    (its setup) is made untimed first."""
    import torch
    c.sample(n, W, generator=g, return_coords=True)
    ts = []
    for _ in range(calls):
        torch.cuda.synchronize()
        t = time.perf_counter()
        c.sample(n, W, generator=g, return_coords=True)
        torch.cuda.synchronize()
        ts.append(time.perf_counter() - t)
    ts.sort()
    med = statistics.median(ts)
    return {"windows_per_s": round(n / med), "median_ms": round(med * 1e3, 4), "p10_ms": round(ts[len(ts) // 10] * 1e3, 4),
            "p90_ms": round(ts[len(ts) * 9 // 10] * 1e3, 4), "calls": calls, "sample_streams": c.sample_streams,
            "protocol": "torch.cuda.synchronize() before and after each sample(n, W, return_coords=True) call, check on; median"}


def ring_child(args, d):
    """The ring's rate and the synchronous figure in a process of its own with the hardware queues of --hw-queues
    (the default-queues figure): one JSON line."""
    import torch
    import panvram_amd
    c = panvram_amd.Cohort.open(d, device="cuda:0", dataset="q4k")
    n, W, K = args.n, args.W, args.steps
    g = torch.Generator(device="cuda:0").manual_seed(args.seed)
    for _ in range(args.warmup):
        c.sample(n, W, generator=g, check=False)
    c.sample(n, W, generator=g)
    torch.cuda.synchronize()
    t = time.perf_counter()
    for _ in range(K):
        c.sample(n, W, generator=g, check=False)
    torch.cuda.synchronize()
    sec = time.perf_counter() - t
    c.sample(n, W, generator=g)                                      # status checked after
    out = {"windows_per_s": round(K * n / sec), "ms_per_step": round(sec * 1e3 / K, 4), "steps": K, "warmup": args.warmup,
           "hw_queues": int(os.environ["GPU_MAX_HW_QUEUES"]), "sample_streams": c.sample_streams,
           "sync_per_call": sync_per_call(c, n, W, g, args.sync_calls)}
    print(json.dumps(out), flush=True)


def run_ring_child(args, d, queues):
    """ring_child in a child process started before this process makes any GPU call (HIP reads GPU_MAX_HW_QUEUES once,
    when it starts) -> its JSON, or {"error": ...}."""
    import subprocess
    cmd = [sys.executable, os.path.abspath(__file__), "--ring-child", "--hw-queues", str(queues), "--steps", str(args.steps),
           "--warmup", str(args.warmup), "--data", d, "--config", args.config, "--n", str(args.n), "--W", str(args.W),
           "--seed", str(args.seed), "--sync-calls", str(args.sync_calls)]
    if args.assemblies:
        cmd += ["--assemblies", str(args.assemblies)]
    log(f"bench: ring with GPU_MAX_HW_QUEUES={queues} in a child process")
    try:
        p = subprocess.run(cmd, stdout=subprocess.PIPE, timeout=600, text=True)
    except subprocess.TimeoutExpired:
        return {"error": "child timed out"}
    lines = [ln for ln in p.stdout.splitlines() if ln.startswith("{")]
    if p.returncode or not lines:
        return {"error": f"child exit status {p.returncode}"}
    return json.loads(lines[-1])


def _events_mean_ms(ev):
    """Mean duration of the bracketed decode launches (first to last event)."""
    return statistics.mean(e[0].elapsed_time(e[-1]) for e in ev)


def _split_ms(ev):
    """Mean durations (decode kernel, windows kernel) of `sample` launches: start to mid, mid to end."""
    return statistics.mean(e[0].elapsed_time(e[1]) for e in ev), statistics.mean(e[1].elapsed_time(e[2]) for e in ev)


def bench_full_stream(args, d, gen):
    """Config 4: the whole base stream of one 3.1 Gbp haplotype. Device decode (windows of 2^28 bases, back to back),
    decode() into pinned host memory (PCIe included), check_full (device FASTA + host XXH3), and the reference CPU
    decoder over the same stream in 4 Mbp windows on the host's threads."""
    import numpy as np
    import torch
    import panvram_amd
    from oracle import oracle as O
    t = time.time()
    c = panvram_amd.Cohort.open(d, device="cuda:0", dataset="q4k")
    t_open = time.time() - t
    if args.calib_copy_mb:              # a copy of known size, which calibrates the byte counters of a rocprofv3 pass
        src = torch.ones(args.calib_copy_mb << 20, dtype=torch.uint8, device="cuda:0")
        torch.empty_like(src).copy_(src)
        torch.cuda.synchronize()
        del src
    n = c.info(0)["bases"]
    piece = 1 << 28
    a_t = torch.tensor([0], device="cuda:0")
    starts = [torch.tensor([s], device="cuda:0") for s in range(0, n, piece)]

    def device_decode():
        return [c.windows(a_t, st, min(piece, n - s), check=False) for st, s in zip(starts, range(0, n, piece))]
    device_decode()
    torch.cuda.synchronize()
    reps = max(1, args.steps // 200)
    c.kernel_events = []
    t = time.perf_counter()
    for _ in range(reps):
        outs = device_decode()
        del outs
    torch.cuda.synchronize()
    dev_s = (time.perf_counter() - t) / reps
    ev, c.kernel_events = c.kernel_events, None
    kms = _events_mean_ms(ev)
    host = torch.empty(n, dtype=torch.uint8, pin_memory=True)
    c.decode(0, out=host)
    t = time.perf_counter()
    c.decode(0, out=host)
    d2h_s = time.perf_counter() - t
    c.check_full(0)
    t = time.perf_counter()
    ok, h = c.check_full(0)
    cf_s = time.perf_counter() - t
    fasta_bytes = c._fasta_plan(0)[3]
    # algorithmic bytes of one 2^28-base launch: payload + 16 B per block + reference bytes read by copies + output
    off = c._array("off").cpu().numpy().view(np.uint32)
    nb = c.info(0)["blocks"]
    payload = int(off[nb]) - int(off[0])
    cpu = None
    R = O.RefDecoder.open(os.path.join(d, "reference.fa"), [c.info(0)["path"]], threads=min(16, os.cpu_count() or 1))
    sample_blocks = range(0, nb, max(1, nb // 2000))
    refb = sum(R.refbytes(0, b) for b in sample_blocks) * nb / len(sample_blocks) if R is not None else float(n)
    alg = (payload + 16 * nb + refb + n) / len(starts)
    tk = measured_traffic(args, c)
    traffic = round(sum(tk.values())) if len(tk) == 5 else None
    if R is not None and not args.no_cpu:
        T = min(16, os.cpu_count() or 1)
        W4 = 1 << 22
        st = np.arange(0, n - W4 + 1, W4, dtype=np.int64)
        a0 = np.zeros(st.size, dtype=np.int64)
        R.windows(a0[:T], st[:T], W4, threads=T)
        t = time.perf_counter()
        R.windows(a0, st, W4, threads=T)
        el = time.perf_counter() - t
        cpu = {"value": round(st.size * W4 / el), "unit": "bases/s", "cores": T, "kind": "reference",
               "sample": f"{st.size} windows of 4 Mbp covering the stream, {T} threads"}
    out = {
        "metric": "decoded bases/s, full-stream decode of one 3.1 Gbp haplotype on the device (config 4)",
        "value": round(n / dev_s), "unit": "bases/s", "n_gpus": 1, "steps": reps, "warmup": 1,
        "ms_per_step": round(dev_s * 1e3, 3), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "u8", "data": "synthetic",
        "config": {"workload": "full: decode(assembly) as windows of 2^28 bases; then decode() to pinned host memory and check_full",
                   "bases": n, "blocks": nb, "open_s": round(t_open, 1), "generate_s": gen["seconds"] if gen else None},
        "roofline": {"bound": "hbm", "achieved": round(alg / (kms * 1e-3) / 1e9, 2), "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                     "frac": round(alg / (kms * 1e-3) / HBM_PEAK, 5), "traffic": traffic, "kernel_ms": round(kms, 4),
                     "algorithmic_bytes_per_launch": round(alg),
                     "traffic_basis": "HBM bytes of one 2^28-base launch: the sum over its five kernels of the committed "
                                      "rocprofv3 FETCH_SIZE / WRITE_SIZE passes' mean per dispatch"},
        "decode_to_host": {"seconds": round(d2h_s, 4), "bases_per_s": round(n / d2h_s), "note": "PCIe-inclusive, pinned destination"},
        "check_full": {"seconds": round(cf_s, 4), "fasta_bytes": fasta_bytes, "equal": bool(ok), "hash": h},
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    if not ok:
        sys.exit(1)


def bench_fetch(args, d, gen):
    """Config 3: the mid cohort at q16k. 65,536 fetch(assembly, contig, start, 5000) with uniform valid coordinates as
    one batched windows call, the per-call fetch latency (synchronous, 1000 calls), and sample(1024, W) for a sweep of
    W, with the reference CPU decoder on the batch."""
    import numpy as np
    import torch
    import panvram_amd
    from oracle import oracle as O
    t = time.time()
    c = panvram_amd.Cohort.open(d, device="cuda:0", dataset="q16k")
    t_open = time.time() - t
    rng = np.random.default_rng(args.seed)
    L = 5000
    ctg = [(a, k, ln, off) for a in range(len(c)) for k, (_, _, ln, off, _) in enumerate(c.contigs(a)) if ln >= L]
    nf = 65536
    pick = rng.integers(0, len(ctg), nf)
    a_np = np.array([ctg[i][0] for i in pick], dtype=np.int64)
    s_np = np.array([ctg[i][3] + rng.integers(0, ctg[i][2] - L + 1) for i in pick], dtype=np.int64)
    a_t, s_t = torch.from_numpy(a_np).cuda(), torch.from_numpy(s_np).cuda()
    for _ in range(3):
        c.windows(a_t, s_t, L, check=False)
    torch.cuda.synchronize()
    reps = max(3, args.steps // 100)
    c.kernel_events = []
    t = time.perf_counter()
    for _ in range(reps):
        x = c.windows(a_t, s_t, L, check=False)
    torch.cuda.synchronize()
    batch_s = (time.perf_counter() - t) / reps
    ev, c.kernel_events = c.kernel_events, None
    kms = _events_mean_ms(ev)
    # per-call fetch latency (synchronous, like the reference's one-call-at-a-time measurement)
    lat = []
    for i in range(1000):
        a, k, ln, off = ctg[int(pick[i])]
        st = int(s_np[i] - off)
        t = time.perf_counter()
        y = c.fetch(a, k, st, L)
        torch.cuda.synchronize()
        lat.append(time.perf_counter() - t)
    sweep = {}
    g = torch.Generator(device="cuda:0").manual_seed(args.seed)
    for W in (1024, 4096, 8192, 32768, 65536):
        for _ in range(5):
            c.sample(1024, W, generator=g, check=False)
        torch.cuda.synchronize()
        t = time.perf_counter()
        K = max(20, args.steps // 20)
        for _ in range(K):
            c.sample(1024, W, generator=g, check=False)
        torch.cuda.synchronize()
        el = time.perf_counter() - t
        sweep[str(W)] = {"windows_per_s": round(K * 1024 / el), "output_GBps": round(K * 1024 * W / el / 1e9, 2)}
    # spot check and CPU baseline on the batch
    paths = [c.info(i)["path"] for i in range(len(c))]
    R = O.RefDecoder.open(os.path.join(d, "reference.fa"), paths, threads=min(16, os.cpu_count() or 1))
    cpu, spot = None, None
    if R is not None:
        k = 2048
        y = R.windows(a_np[:k], s_np[:k], L, threads=min(16, os.cpu_count() or 1))
        spot = f"{int((x[:k].cpu().numpy() == y).all(axis=1).sum())}/{k} fetches == CPU decoder (reference)"
        if not args.no_cpu:
            T = min(16, os.cpu_count() or 1)
            t = time.perf_counter()
            R.windows(a_np, s_np, L, threads=T)
            el = time.perf_counter() - t
            cpu = {"value": round(nf / el), "unit": "fetches/s", "cores": T, "kind": "reference",
                   "sample": f"the same {nf} fetches, {T} threads"}
    out = {
        "metric": "fetches/s, 65536 x fetch(asm, contig, start, 5000) batched, mid cohort q16k (config 3)",
        "value": round(nf / batch_s), "unit": "fetches/s", "n_gpus": 1, "steps": reps, "warmup": 3,
        "ms_per_step": round(batch_s * 1e3, 3), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "u8", "data": "synthetic",
        "config": {"workload": "mid16: windows(n=65536, W=5000) at uniform valid contig coordinates", "assemblies": len(c),
                   "Q": c.block_size, "open_s": round(t_open, 1), "generate_s": gen["seconds"] if gen else None},
        "kernel_ms": round(kms, 4),
        "fetch_latency_ms": {"median": round(statistics.median(lat) * 1e3, 4), "p90": round(sorted(lat)[900] * 1e3, 4),
                             "note": "one synchronous fetch() per call, 1000 calls"},
        "w_sweep_n1024": sweep,
        "cpu_baseline": cpu,
        "spot_check": spot,
    }
    print(json.dumps(out), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=1000)
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--config", default="headline")
    ap.add_argument("--assemblies", type=int, default=None, help="override the preset's haplotype count")
    ap.add_argument("--n", type=int, default=1024)
    ap.add_argument("--W", type=int, default=8192)
    ap.add_argument("--large-n", type=int, default=65536)
    ap.add_argument("--data", default=None)
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--seed", type=int, default=20261005)
    ap.add_argument("--no-variants", action="store_true", help="skip the tokens/rc and large-n variants (profiling runs)")
    ap.add_argument("--hw-queues", type=int, default=24, choices=range(1, 33), metavar="1..32",
                    help="GPU_MAX_HW_QUEUES for this process (sample's stream ring: one stream per queue but the "
                         "caller's, at most 15)")
    ap.add_argument("--sample-streams", type=int, default=None,
                    help="size of sample's stream ring (default: one per hardware queue but the caller's; 0: the caller's stream)")
    ap.add_argument("--sample-wait", default="counter", choices=("event", "counter"),
                    help="how the caller's stream waits for the ring (counter: less host time per call; not under "
                         "rocprofv3 --pmc, which needs --sample-streams 0)")
    ap.add_argument("--light-decode", default="on", choices=("on", "off"),
                    help="decode short-payload blocks one lane per block before the windows kernel (on), or every block "
                         "in the windows kernel's wave decoder (off)")
    ap.add_argument("--calib-copy-mb", type=int, default=0,
                    help="before timing, one plain device-to-device copy of this many MiB (scales rocprof byte counters)")
    ap.add_argument("--sync-calls", type=int, default=200, help="calls of the synchronous (one call at a time) figure")
    ap.add_argument("--default-queues", type=int, default=4, metavar="Q",
                    help="hardware queues of the child run that reports the ring under HIP's default (0: no child run)")
    ap.add_argument("--ring-child", action="store_true", help=argparse.SUPPRESS)
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU (asked for {args.gpus}); windows and blocks are independent, so more GPUs would each run their own batches", file=sys.stderr)
        sys.exit(2)

    # HIP gives a process GPU_MAX_HW_QUEUES hardware queues (default 4) and `sample` overlaps consecutive calls on one
    # stream per queue besides the caller's; a serving or training process sets this before HIP starts, as here.
    os.environ["GPU_MAX_HW_QUEUES"] = str(args.hw_queues)
    import numpy as np
    import torch

    import panvram_amd
    from oracle import oracle as O

    d = data_dir(args)
    gen = ensure_cohort(args, d)
    if args.ring_child:
        return ring_child(args, d)
    default_q = None
    if args.config == "headline" and not args.no_variants and args.default_queues and args.default_queues != args.hw_queues:
        default_q = run_ring_child(args, d, args.default_queues)       # before this process's first GPU call
    if args.config == "full":
        return bench_full_stream(args, d, gen)
    if args.config == "mid16":
        return bench_fetch(args, d, gen)
    t = time.time()
    c = panvram_amd.Cohort.open(d, device="cuda:0", dataset="q4k")
    t_open = time.time() - t
    rb = c.resident_bytes()
    log(f"bench: opened {len(c)} assemblies in {t_open:.1f} s, resident {rb['total'] / 1e9:.3f} GB on {torch.cuda.get_device_name(0)}")
    n, W, K = args.n, args.W, args.steps
    g = torch.Generator(device="cuda:0").manual_seed(args.seed)

    def run(steps, **kw):
        for _ in range(steps):
            c.sample(n, W, generator=g, check=False, **kw)

    if args.calib_copy_mb:
        src = torch.ones(args.calib_copy_mb << 20, dtype=torch.uint8, device="cuda:0")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"bench: calibration copy of {args.calib_copy_mb} MiB done")
        del src, dst
    if args.sample_streams is not None:
        c.sample_streams = args.sample_streams
    c.sample_wait = args.sample_wait
    c.light_decode = args.light_decode == "on"
    run(args.warmup)
    c.sample(n, W, generator=g)                                      # status checked once before timing
    state = g.get_state()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    run(K)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    c.sample(n, W, generator=g)                                      # status checked after
    sec = t1 - t0
    value = K * n / sec
    # kernel times while calls overlap: a pass of its own over the same ring (not timed), HIP events bracketing one
    # launch in 8 (every launch in short runs), since each event pair adds two timestamp packets to its stream
    c.kernel_events_every = 8 if K >= 64 else 1
    c.kernel_events = []
    run(min(K, 400))
    torch.cuda.synchronize()
    ev, c.kernel_events = c.kernel_events, None
    front_ov, kms_ov = _split_ms(ev)
    log(f"bench: {K} x sample({n}, {W}): {sec * 1e3 / K:.3f} ms/step, {value:,.0f} windows/s; overlapped launches: decode kernel "
        f"{front_ov * 1e3:.1f} us, windows kernel {kms_ov * 1e3:.1f} us mean")
    # Roofline pass: the same workload, one launch at a time on the caller's stream (no ring), HIP events on every
    # launch, so that a kernel's time is its own and not the time it shares the GPU with up to ~7 other launches.
    # (In a rocprofv3 trace of this command these are the windows_kernel dispatches on the caller's stream.)
    ring = c.sample_streams
    c.sample_streams, c.kernel_events_every, c.kernel_events = 0, 1, []
    for _ in range(ROOF_LAUNCHES):
        c.sample(n, W, generator=g, check=False)
    torch.cuda.synchronize()
    evr, c.kernel_events = c.kernel_events, None
    c.sample_streams = ring
    front_ms, kms = _split_ms(evr)
    log(f"bench: roofline pass, {ROOF_LAUNCHES} launches one at a time: decode kernel {front_ms * 1e3:.1f} us, windows kernel {kms * 1e3:.1f} us")
    # the anchor's protocol: one call at a time, synced before and after, with the ring and on the caller's stream
    sync_ring = sync_per_call(c, n, W, g, args.sync_calls)
    c.sample_streams = 0
    sync_caller = sync_per_call(c, n, W, g, args.sync_calls)
    c.sample_streams = ring
    log(f"bench: synchronous calls (median of {args.sync_calls}): ring {sync_ring['windows_per_s']:,} windows/s "
        f"({sync_ring['median_ms']} ms), caller's stream {sync_caller['windows_per_s']:,} ({sync_caller['median_ms']} ms)")

    # coordinates of the first timed batches (generator replayed) -> algorithmic bytes, spot check, CPU baseline
    g.set_state(state)
    nb_batches = 4 if n <= 8192 else 1
    batches = [c.sample(n, W, generator=g, return_coords=True) for _ in range(nb_batches)]
    coords = []
    for x, co in batches:
        co = co.cpu().numpy()
        st_ = np.array([c.contigs(int(a))[int(ci)][3] + int(s) for a, ci, s, _ in co], dtype=np.int64)
        coords.append((x.cpu().numpy(), co[:, 0].astype(np.int64), st_))
    off_host = c._array("off").cpu().numpy().view(np.uint32)
    asm_rec = c._array("asm").cpu().numpy().reshape(-1, 8)
    paths = [c.info(i)["path"] for i in range(len(c))]
    refpath = os.path.join(d, "reference.fa")
    t = time.time()
    R = O.RefDecoder.open(refpath, paths, threads=min(16, os.cpu_count() or 1))
    kind = "reference"
    if R is None:
        kind = "port"
        ref_np = O.reference_bases(refpath)
        arcs = [O.Archive(p) for p in paths]
        refbytes = lambda a, b: arcs[a].refbytes(ref_np, b)
        cpu_windows_at = lambda a, s, w, T: O.windows(arcs, ref_np, a, s, w, threads=T)
    else:
        refbytes = lambda a, b: R.refbytes(a, b)
        cpu_windows_at = lambda a, s, w, T: R.windows(a, s, w, threads=T)
    cpu_windows = lambda a, s, T: cpu_windows_at(a, s, W, T)
    log(f"bench: CPU decoder ({kind}) opened in {time.time() - t:.1f} s")
    rb_cache = {}

    def rbytes(a, b):
        k = (int(a), int(b))
        if k not in rb_cache:
            rb_cache[k] = refbytes(*k)
        return rb_cache[k]
    parts = [b_parts(c, off_host, asm_rec, list(zip(a.tolist(), s.tolist())), W, rbytes) for _, a, s in coords]
    pay_b, model_b, ref_b, out_b = (statistics.mean(p[i] for p in parts) for i in range(4))
    per_launch = pay_b + model_b + ref_b + out_b
    # per kernel: the decode kernel reads the covering blocks' payloads and table entries, the touched assemblies'
    # models and the draws (8 B a window); the windows kernel reads the reference bytes the copies need and writes the
    # rows
    alg = {"decode": pay_b + model_b + 8 * n, "windows": ref_b + out_b}
    # the decode kernel's latency bound: one call of each of the first batch's three longest covering blocks alone
    # (its serial rANS chain, then a replay of one block), HIP events around the call
    crit = []
    Q = c.block_size
    # (not in profiling runs, whose per-kernel means must be the workload's alone)
    for pl, a_, b_ in ([] if args.no_variants else longest_blocks(c, off_host, asm_rec, zip(coords[0][1].tolist(), coords[0][2].tolist()), W)):
        blen = min(Q, c.info(a_)["bases"] - b_ * Q)
        wa, ws = torch.tensor([a_], device="cuda:0"), torch.tensor([b_ * Q], device="cuda:0")
        c.windows(wa, ws, blen)                                     # status checked
        c.kernel_events = []
        for _ in range(10):
            c.windows(wa, ws, blen, check=False)
        torch.cuda.synchronize()
        evc, c.kernel_events = c.kernel_events, None
        crit.append((statistics.mean(e[0].elapsed_time(e[2]) for e in evc), pl))
    crit_ms, crit_pay = max(crit) if crit else (None, None)
    if crit:
        log(f"bench: longest block alone ({crit_pay} payload bytes): {crit_ms * 1e3:.1f} us per call; decode kernel {front_ms * 1e3:.1f} us")
    # spot check: the first timed batch against the CPU decoder
    T = min(16, os.cpu_count() or 1)
    x0, a0, s0 = coords[0]
    y0 = cpu_windows(a0, s0, T)
    equal = int(sum(np.array_equal(x0[i], y0[i]) for i in range(n)))
    log(f"bench: spot check {equal}/{n} windows == CPU decoder; algorithmic bytes per launch {per_launch / 1e6:.2f} MB")

    cpu = None
    if not args.no_cpu:
        def cpu_rate(threads, budget):
            reps, t_ = 0, time.perf_counter()
            while True:
                _, a, s = coords[reps % len(coords)]
                cpu_windows(a, s, threads)
                reps += 1
                el = time.perf_counter() - t_
                if el >= budget:
                    return reps * n / el, reps
        v_all, r_all = cpu_rate(T, args.cpu_seconds)
        v_one, r_one = cpu_rate(1, max(2.0, args.cpu_seconds / 4))
        model = next((ln.split(":", 1)[1].strip() for ln in open("/proc/cpuinfo") if ln.startswith("model name")), "unknown")
        cpu = {"value": round(v_all), "unit": "windows/s", "cores": T, "kind": kind, "cpu_model": model,
               "host_cores": len(os.sched_getaffinity(0)),
               "sample": f"{r_all} batches of {n} x {W} (the timed workload's first batches, generator replayed), {T} threads",
               "one_thread": {"value": round(v_one), "sample": f"{r_one} batches, 1 thread"}}
        log(f"bench: CPU decoder {v_all:,.0f} windows/s on {T} threads, {v_one:,.0f} on 1")

    # variants: tokens + rc, and a large batch
    variants = {}
    bad_variant = False
    if args.no_variants:
        args.large_n = 0
    else:
        run(args.warmup, tokens=True, reverse_complement=0.5)           # the GPU idled through the CPU baseline
        c.kernel_events = []
        torch.cuda.synchronize()
        t = time.perf_counter()
        run(K, tokens=True, reverse_complement=0.5)
        torch.cuda.synchronize()
        evt, c.kernel_events = c.kernel_events, None
        variants["tokens_rc0.5"] = {"windows_per_s": round(K * n / (time.perf_counter() - t)),
                                    "decode_kernel_ms": round(_split_ms(evt)[0], 4), "kernel_ms": round(_split_ms(evt)[1], 4)}
        # BASELINE config 2's loop body: tokens, reverse_complement=0.5, return_coords=True, timed as the main loop
        # (no events), one batch checked against the CPU decoder at its returned coordinates and strands
        run(args.warmup, tokens=True, reverse_complement=0.5, return_coords=True)
        torch.cuda.synchronize()
        t = time.perf_counter()
        run(K, tokens=True, reverse_complement=0.5, return_coords=True)
        torch.cuda.synchronize()
        v2 = K * n / (time.perf_counter() - t)
        x2, co2 = c.sample(n, W, generator=g, tokens=True, reverse_complement=0.5, return_coords=True)
        co2 = co2.cpu().numpy()
        st2 = np.array([c.contigs(int(a))[int(ci)][3] + int(s) for a, ci, s, _ in co2], dtype=np.int64)
        T2 = min(16, os.cpu_count() or 1)
        if R is not None:
            y2 = R.windows(co2[:, 0].astype(np.int64), st2, W, rc=co2[:, 3].astype(np.uint8), tokens=True, threads=T2)
        else:
            y2 = O.windows(arcs, ref_np, co2[:, 0].astype(np.int64), st2, W, rc=co2[:, 3].astype(np.uint8), tokens=True, threads=T2)
        eq2 = int((x2.cpu().numpy() == y2).all(axis=1).sum())
        variants["tokens_rc0.5_coords"] = {"windows_per_s": round(v2), "spot_check": f"{eq2}/{n} windows == CPU decoder ({kind})"}
        if eq2 != n:
            bad_variant = True
    if not args.no_variants:
        # every block in the windows kernel (no one-lane-per-block light decoder), same workload
        c.light_decode = False
        run(args.warmup)
        c.kernel_events = []
        torch.cuda.synchronize()
        t = time.perf_counter()
        run(K)
        torch.cuda.synchronize()
        evw, c.kernel_events = c.kernel_events, None
        variants["wave_decoder_only"] = {"windows_per_s": round(K * n / (time.perf_counter() - t)),
                                         "decode_kernel_ms": round(_split_ms(evw)[0], 4), "kernel_ms": round(_split_ms(evw)[1], 4)}
        c.light_decode = args.light_decode == "on"
    nl = args.large_n
    if nl:
        try:
            # every stream of the ring, and the caller's stream, through a first call of this shape (work buffers)
            ring = c.sample_streams
            for _ in range(max(1, ring) + 2):
                c.sample(nl, W, generator=g)
            c.sample_streams = 0
            c.sample(nl, W, generator=g)
            c.sample_streams = ring
            torch.cuda.synchronize()
            reps = 20
            t = time.perf_counter()
            for _ in range(reps):
                c.sample(nl, W, generator=g, check=False)
            torch.cuda.synchronize()
            el = time.perf_counter() - t
            # kernel times as in the roofline pass: one launch at a time on the caller's stream, events on each
            c.sample_streams, c.kernel_events_every, c.kernel_events = 0, 1, []
            for _ in range(5):
                c.sample(nl, W, generator=g, check=False)
            torch.cuda.synchronize()
            evl, c.kernel_events = c.kernel_events, None
            # the whole call with events only at its start and end, so that it runs as an untimed call on the caller's
            # stream does: the replay of the light slots beside the heavy waves, then the heavy slots' replay
            c.kernel_events_split = False
            c.sample(nl, W, generator=g, check=False)
            torch.cuda.synchronize()
            c.kernel_events = []
            for _ in range(5):
                c.sample(nl, W, generator=g, check=False)
            torch.cuda.synchronize()
            evw, c.kernel_events = c.kernel_events, None
            c.kernel_events_split = True
            c.sample_streams = ring
            c.sample(nl, W, generator=g)                               # status checked
            fl, kl = _split_ms(evl)
            whole = _events_mean_ms(evw)
            # the batch's bytes scaled from the headline batch's (every assembly's model touched)
            large_bytes = (per_launch - model_b) * nl / n + MODEL_BYTES * len(c)
            variants[f"n{nl}"] = {"windows_per_s": round(reps * nl / el), "decode_kernel_ms": round(fl, 3), "kernel_ms": round(kl, 3),
                                  "windows_kernel_frac_est": round(alg["windows"] * nl / n / (kl * 1e-3) / HBM_PEAK, 4),
                                  "call_frac_est": round(large_bytes / ((fl + kl) * 1e-3) / HBM_PEAK, 4),
                                  "call_overlapped_ms": round(whole, 3),
                                  "call_overlapped_frac": round(large_bytes / (whole * 1e-3) / HBM_PEAK, 4),
                                  "aggregate_frac_est": round(large_bytes * reps / el / HBM_PEAK, 4)}
        except RuntimeError as e:          # out of memory on a small device
            variants[f"n{nl}"] = {"error": str(e)[:200]}
    if not args.no_variants:
        # the compact resident forms (2-bit reference + grouped block table) on the same workload
        try:
            t = time.time()
            cf = panvram_amd.Cohort.open(d, device="cuda:0", dataset="q4k", packed_reference=True, compact_blocks=True)
            t_of = time.time() - t
            g0, gf = (torch.Generator(device="cuda:0").manual_seed(args.seed + 1) for _ in range(2))
            same = all(torch.equal(c.sample(n, W, generator=g0), cf.sample(n, W, generator=gf)) for _ in range(4))
            for _ in range(args.warmup):
                cf.sample(n, W, generator=gf, check=False)
            cf.kernel_events, cf.kernel_events_every = [], 8
            torch.cuda.synchronize()
            t = time.perf_counter()
            for _ in range(K):
                cf.sample(n, W, generator=gf, check=False)
            torch.cuda.synchronize()
            el = time.perf_counter() - t
            evf, cf.kernel_events = cf.kernel_events, None
            cf.sample(n, W, generator=gf)                                # status checked after
            variants["packed_compact"] = {"windows_per_s": round(K * n / el),
                                          "decode_kernel_ms": round(_split_ms(evf)[0], 4), "kernel_ms": round(_split_ms(evf)[1], 4),
                                          "resident_GB": round(cf.resident_bytes()["total"] / 1e9, 3), "open_s": round(t_of, 1),
                                          "equal_to_default_form": bool(same)}
            del cf
        except RuntimeError as e:
            variants["packed_compact"] = {"error": str(e)[:200]}

    # fetch latency on this cohort, drawn as the reference's 558-assembly run draws it (scripts/cohort558.py:73-93):
    # assembly uniform, contig by length, length 1 + 2^(20 u) capped at the contig, start uniform; one synchronous
    # call each. Each result is copied to the host after its timed span and all are checked against the CPU decoder
    # after the loop, so that the GPU does not idle through a CPU decode between two timed calls. The status check
    # inside fetch() (its device sync) is wrapped to mark when the host had issued the call.
    rng = random.Random(20261005)
    lat, fbad, calls, outs, issued = [], 0, [], [], []
    check0 = c._check

    def check_marked(status):
        issued.append(time.perf_counter())
        return check0(status)
    c._check = check_marked
    import gc
    gc_spans = []                     # (start, end) of every garbage collection during the loop, perf_counter time

    def gc_probe(phase, info):
        if phase == "start":
            gc_spans.append([time.perf_counter(), None])
        elif gc_spans and gc_spans[-1][1] is None:
            gc_spans[-1][1] = time.perf_counter()
    gc.callbacks.append(gc_probe)
    spans = []
    for i in range(1000):
        a = rng.randrange(len(c))
        ctgs = c.contigs(a)
        p = rng.randrange(sum(r[2] for r in ctgs))
        ci = 0
        while p >= ctgs[ci][2]:
            p -= ctgs[ci][2]
            ci += 1
        nb = ctgs[ci][2]
        L = min(nb, 1 + int(2 ** (rng.random() * 20)))
        s = rng.randrange(nb - L + 1)
        r0 = torch.cuda.memory_reserved()
        torch.cuda.synchronize()
        t = time.perf_counter()
        z = c.fetch(a, ci, s, L)
        torch.cuda.synchronize()
        t1 = time.perf_counter()
        lat.append(t1 - t)
        spans.append((t, t1))
        calls.append((a, ci, s, L, torch.cuda.memory_reserved() - r0))
        outs.append(z.cpu().numpy())
        del z
    gc.callbacks.remove(gc_probe)
    c._check = check0
    for i, (a, ci, s, L, _) in enumerate(calls):
        y = cpu_windows_at(np.array([a], dtype=np.int64), np.array([c.contigs(a)[ci][3] + s], dtype=np.int64), L, T)
        fbad += int(not np.array_equal(outs[i], y[0]))
    del outs

    def gc_ms(i):                     # garbage collection inside call i's timed span
        t0_, t1_ = spans[i]
        return sum(max(0.0, min(t1_, e) - max(t0_, b)) for b, e in gc_spans if e is not None) * 1e3
    # the ten slowest calls again, one at a time, with HIP events around the launch: a call slow only the first time
    # (a new allocation, the work buffer growing) is fast here; one slow by its own work stays slow
    slow = sorted(range(len(lat)), key=lat.__getitem__, reverse=True)[:10]
    tail = []
    for i in slow:
        a, ci, s, L, grew = calls[i]
        c.kernel_events = []
        torch.cuda.synchronize()
        t = time.perf_counter()
        c.fetch(a, ci, s, L)
        torch.cuda.synchronize()
        again = time.perf_counter() - t
        evf, c.kernel_events = c.kernel_events, None
        b0 = (c.contigs(a)[ci][3] + s) // Q
        tail.append({"ms": round(lat[i] * 1e3, 3), "call": i, "length": L, "blocks": (c.contigs(a)[ci][3] + s + L - 1) // Q - b0 + 1,
                     "reserved_grew_MB": round(grew / 2**20, 1), "gc_ms": round(gc_ms(i), 3),
                     "issue_ms": round((issued[i] - spans[i][0]) * 1e3, 3), "wait_ms": round((spans[i][1] - issued[i]) * 1e3, 3),
                     "again_ms": round(again * 1e3, 3), "again_device_ms": round(evf[0][0].elapsed_time(evf[0][2]), 3)})
    # the same synchronous pattern with no decode: a one-element torch kernel, its value read back (as fetch() reads
    # its status word) and a device sync, 1000 times; its tail is the platform's own
    probe = torch.zeros(1, dtype=torch.int32, device="cuda:0")
    plat = []
    for _ in range(1000):
        torch.cuda.synchronize()
        t = time.perf_counter()
        probe.add_(1)
        int(probe.item())
        torch.cuda.synchronize()
        plat.append(time.perf_counter() - t)
    plat.sort()
    variants["fetch_latency"] = {"median_ms": round(statistics.median(lat) * 1e3, 4), "p90_ms": round(sorted(lat)[900] * 1e3, 4),
                                 "max_ms": round(max(lat) * 1e3, 3), "calls": len(lat),
                                 "check": f"{len(lat) - fbad}/{len(lat)} == CPU decoder ({kind})", "slowest": tail,
                                 "gc_runs": len(gc_spans),
                                 "platform_sync": {"median_ms": round(plat[500] * 1e3, 4), "p90_ms": round(plat[900] * 1e3, 4),
                                                   "p99_ms": round(plat[990] * 1e3, 4), "max_ms": round(plat[-1] * 1e3, 3),
                                                   "note": "1000 x (one-element torch kernel, .item(), device sync), no decode"},
                                 "note": "1000 synchronous fetch() calls, length 1 .. 2^20 log-uniform (the reference's C558 draw)"}

    # the kernels of a call (one at a time, the roofline pass), and the dominant one by time as the line's roofline
    traffic = measured_traffic(args, c)
    names = {"decode": f"front_kernel<{Q}>" if n * ((W + Q - 1) // Q + 1) <= 16384 else f"slot+heavy+light_decode+spill<{Q}>",
             "windows": f"windows_kernel<{Q}>"}
    times = {"decode": front_ms, "windows": kms}

    def kern(k):
        return {"kernel": names[k], "kernel_ms": round(times[k], 4), "algorithmic_bytes_per_launch": round(alg[k]),
                "achieved": round(alg[k] / (times[k] * 1e-3) / 1e9, 3), "frac": round(alg[k] / (times[k] * 1e-3) / HBM_PEAK, 6),
                "traffic": traffic.get(names[k])}
    dom = max(times, key=times.get)
    # the line's own figure: the whole call's algorithmic bytes over the dominant kernel's time; the per-kernel split
    # (each kernel's own bytes over its own time) is under `kernels`
    roofline = {"bound": "hbm", "achieved": round(per_launch / (times[dom] * 1e-3) / 1e9, 3), "peak": HBM_PEAK / 1e9, "unit": "GB/s",
                "frac": round(per_launch / (times[dom] * 1e-3) / HBM_PEAK, 5), "traffic": traffic.get(names[dom]),
                "kernel": names[dom], "kernel_ms": round(times[dom], 4), "algorithmic_bytes_per_launch": round(per_launch),
                "basis": "the whole call's algorithmic bytes (payloads + block table + models + draws + reference bytes copied "
                         "+ output) over the dominant kernel's mean time; traffic: that kernel's measured HBM bytes",
                "timing": f"{ROOF_LAUNCHES} launches one at a time on the caller's stream, HIP events on each",
                "kernels": {k: kern(k) for k in ("decode", "windows")},
                # the decode kernel is latency-bound: its serial rANS chains, not bytes, set its time
                "latency": {"longest_block_call_ms": round(crit_ms, 4), "longest_block_payload": crit_pay,
                            "decode_kernel_over_longest_block_call": round(front_ms / crit_ms, 3)} if crit else None,
                "call": {"ms": round(front_ms + kms, 4), "algorithmic_bytes_per_launch": round(per_launch),
                         "achieved": round(per_launch / ((front_ms + kms) * 1e-3) / 1e9, 2),
                         "frac": round(per_launch / ((front_ms + kms) * 1e-3) / HBM_PEAK, 5)},
                # the same kernels inside the timed loop, where up to ~7 launches share the GPU
                "overlapped_kernel_ms": round(kms_ov, 4), "overlapped_decode_kernel_ms": round(front_ov, 4),
                # launches overlap on the stream ring: the GPU as a whole moves bytes per launch x launches per s
                "aggregate_achieved": round(per_launch * K / sec / 1e9, 2),
                "aggregate_frac": round(per_launch * K / sec / HBM_PEAK, 5)}
    out = {
        "metric": METRIC, "value": round(value), "unit": "windows/s", "n_gpus": 1, "steps": K, "warmup": args.warmup,
        "ms_per_step": round(sec * 1e3 / K, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": round(value / PUBLISHED, 3) if args.config == "headline" and not args.assemblies else None,
        "dtype": "u8", "data": "synthetic",
        "config": {"workload": f"{args.config}: sample(n={n}, W={W}) uint8 over {len(c)} synthetic q{c.block_size // 1024}k haplotypes",
                   "assemblies": len(c), "n": n, "W": W, "Q": c.block_size, "bases": int(sum(c.info(i)["bases"] for i in range(len(c)))),
                   "resident_GB": round(rb["total"] / 1e9, 3), "open_s": round(t_open, 1), "generate_s": gen["seconds"] if gen else None,
                   "sample_streams": c.sample_streams, "hw_queues": int(os.environ["GPU_MAX_HW_QUEUES"]), "sample_wait": c.sample_wait},
        "roofline": roofline,
        "sync_per_call": sync_ring,
        "sync_per_call_caller_stream": sync_caller,
        "default_queues": default_q,
        "cpu_baseline": cpu,
        "variants": variants,
        "spot_check": f"{equal}/{n} windows of the first timed batch == CPU decoder ({kind})",
    }
    print(json.dumps(out), flush=True)
    if equal != n or fbad or bad_variant:
        sys.exit(1)


if __name__ == "__main__":
    main()
