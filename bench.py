#!/usr/bin/env python3
"""Decode-attention benchmark: ASTC-V split-K attention on one MI355X.

Workload (one step = one decode step of the whole batch): T=8192 keys per
sequence, batch 16, 9 query heads / 3 KV heads, head dim 64, FP16 K, V as an
ASTC RGBA 6x5 atlas (page 120) with per-token fp16 scale/offset, encoded at
quality 98 (the reference bridge's default, astc_kv/codec.py:116-117);
independent seeded K/V per sequence (K ~ N(0,1) with 4 channels x8,
V ~ N(0, 0.5), q ~ N(0,1)). The same workload encoded at quality 50 is timed
beside it (`quality_50`), and each atlas's block classes are reported
(`v_blocks`: table-path / compute-path fractions, partitions, weight levels,
endpoint modes), since the decode cost depends on them.

Inputs are resident in HBM. A pool of distinct copies of the KV set (> 512 MB
in total) is rotated across steps so that the 256 MB Infinity Cache cannot
hold the working set; every step is timed as one launch (split kernel with the
merge in its last workgroup per head) replayed from a HIP graph, with events
on the launch stream. `copy_ceiling` is a device-to-device copy timed the
same way (what the box sustains for read + write).

Prints one JSON line. `value` is the effective bandwidth: algorithmic bytes
of a step (K + ASTC blocks read + V scale/offset + q + out) / step time.
`roofline.achieved` is the same bytes over the same one-launch time.
`roofline.traffic` is the HBM traffic per launch that rocprofv3 measured
(FETCH_SIZE + WRITE_SIZE, scaled by a plain copy kernel of known size) for
this same workload, read from the committed profile summary whose workload
line matches.

`--fixture DIR` times the reference's own astcenc payload fixture instead,
repeated to --tokens keys as the reference's traffic controls are
(scripts/make_traffic_fixture.py:12-49), batch 1, at the host's tile and at
the reference's tile for that size, next to the reference's published M5 Pro
times for the same payloads (docs/research_v3_report.md:28-32).
`--ragged N` times a paged ragged batch with block tables.

`python bench.py --summarize KT FETCH WRITE` instead prints a markdown summary
of rocprofv3 CSV output directories (kernel trace with --stats, a FETCH_SIZE
pass, a WRITE_SIZE pass) of a bench run made with --copy-calibration-mb.
"""
from __future__ import annotations

import argparse
import csv
import glob
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "astc-kv_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

HBM_PEAK_GBS = 8000.0
PROFILES = ROOT / "profiles"
COPY_KERNEL = "neg_kernel"   # the calibration copy: torch.neg over float32 (reads N bytes, writes N bytes)


def log(msg: str):
    print(f"# {msg}", file=sys.stderr, flush=True)


def parse_args(argv=None):
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--batch", type=int, default=16)
    ap.add_argument("--tokens", type=int, default=8192)
    ap.add_argument("--query-heads", type=int, default=9)
    ap.add_argument("--kv-heads", type=int, default=3)
    ap.add_argument("--dim", type=int, default=64)
    ap.add_argument("--layout", default="rgba")
    ap.add_argument("--block", default="6x5")
    ap.add_argument("--page", type=int, default=120)
    ap.add_argument("--tile", type=int, default=0, help="tokens per split (0 = automatic)")
    ap.add_argument("--fp16-tile", type=int, default=0, help="tokens per split of the FP16 control (0 = automatic)")
    ap.add_argument("--quality", type=float, default=98.0, help="encoder effort for the synthetic V atlas")
    ap.add_argument("--compare-quality", type=float, default=50.0,
                    help="also time the same workload encoded at this quality (0: off)")
    ap.add_argument("--fixture", default=None,
                    help="time an astc-kv-probe-v1 fixture directory (e.g. tests/golden/t384) repeated to --tokens")
    ap.add_argument("--ref-tile", type=int, default=0,
                    help="fixture: the reference's tile for this size (0: its protocol's 32/64/256 at T384/2048/8192)")
    ap.add_argument("--copy-ceiling-mb", type=float, default=1024.0,
                    help="size of the device-to-device copy timed for the copy ceiling (0: off)")
    ap.add_argument("--pool-mb", type=float, default=600.0, help="minimum bytes of distinct KV sets rotated")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU baseline budget")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-graph", action="store_true")
    ap.add_argument("--copy-calibration-mb", type=float, default=0.0,
                    help="also run a plain copy kernel over this many MB (for rocprofv3 counter scaling)")
    ap.add_argument("--traffic", default=None,
                    help="profile summary holding the measured traffic (default: the summary under profiles/ "
                         "whose workload line names this workload)")
    ap.add_argument("--counters", nargs="+", metavar="PMC_DIR",
                    help="print a table of the PMC counters in these rocprofv3 --pmc output directories")
    ap.add_argument("--summarize", nargs=3, metavar=("KT", "FETCH", "WRITE"),
                    help="print a markdown summary of rocprofv3 CSV output directories and exit")
    ap.add_argument("--out", default="", help="also write the JSON line to this file")
    ap.add_argument("--cache", default="",
                    help="directory for the encoded V atlases / paged pools of these arguments (reused when present)")
    ap.add_argument("--no-resident", action="store_true", help="skip the single-set (cache-resident) timing")
    ap.add_argument("--k-dist", default="outlier", choices=["outlier", "t3"],
                    help="K ~ N(0,1) with 4 channels x8, or Student-t with 3 degrees of freedom")
    ap.add_argument("--ragged", type=int, default=0,
                    help="paged ragged batch of this many sequences (lengths uniform in "
                         "[--min-tokens, --tokens]) instead of the uniform batch")
    ap.add_argument("--min-tokens", type=int, default=512)
    ap.add_argument("--k-format", default="fp16", choices=["fp16", "u4g32"], help="K storage (paged batches)")
    ap.add_argument("--tail", action="store_true", help="paged: keep each sequence's partial last page as FP16 V")
    return ap.parse_args(argv)


def workload_name(a, quality=None) -> str:
    bx, by = a.block.split("x")
    kd = ", Student-t K" if a.k_dist == "t3" else ""
    return (f"decode attention T{a.tokens} batch {a.batch}, {a.query_heads}q/{a.kv_heads}kv, D{a.dim}{kd}, "
            f"FP16 K + ASTC {a.layout.upper()} {bx}x{by} V (page {a.page}, quality {a.quality if quality is None else quality:g})")


def _cache_path(a, what: str) -> Path | None:
    """Cache file of an encoded input: the arguments that fix it, hashed."""
    if not a.cache:
        return None
    import hashlib
    key = json.dumps([what, a.batch, a.tokens, a.query_heads, a.kv_heads, a.dim, a.layout, a.block, a.page,
                      a.k_dist, a.ragged, a.min_tokens, a.k_format, a.tail], sort_keys=True)
    return Path(a.cache) / f"{what}-{hashlib.sha256(key.encode()).hexdigest()[:16]}.npz"


def cached_atlas(a, v, quality):
    """build_atlas, or the atlas a previous run with the same arguments saved."""
    from astc_kv.atlas import Atlas, build_atlas
    bx, by = (int(x) for x in a.block.split("x"))
    path = _cache_path(a, f"atlas-q{quality:g}")
    if path is not None and path.exists():
        z = np.load(path)
        return Atlas(z["blocks"], z["scale"], z["offset"], a.tokens, a.dim, a.layout, bx, by, a.page)
    atlas = build_atlas(v, a.layout, (bx, by), a.page, quality)
    if path is not None:
        path.parent.mkdir(parents=True, exist_ok=True)
        np.savez(path, blocks=atlas.blocks, scale=atlas.scale, offset=atlas.offset)
    return atlas


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def copy_ceiling(torch, mb: float, reps: int = 20) -> dict | None:
    """Device-to-device copy of `mb` MB (read mb, write mb), timed with events
    on the current stream: the read + write rate the box sustains."""
    if mb <= 0:
        return None
    n = int(mb * 1e6) // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    stream = torch.cuda.current_stream()
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0.record(stream)
    for _ in range(reps):
        dst.copy_(src)
    t1.record(stream)
    torch.cuda.synchronize()
    ms = t0.elapsed_time(t1) / reps
    del src, dst
    gbs = 2 * n * 4 / (ms * 1e-3) / 1e9
    return {"GB/s": round(gbs, 1), "frac_of_peak": round(gbs / HBM_PEAK_GBS, 4), "bytes_moved": 2 * n * 4,
            "us": round(ms * 1e3, 2), "kernel": "torch copy_ (float32, device to device)"}


def byte_ratios(a, nbytes) -> dict:
    """Persistent K + V + V metadata bytes over FP16 K + FP16 V for this
    workload, and for the same shape with a scalar 6x6 V atlas (the
    reference's compact layout; its T8192 measurement is 3,981,312 /
    6,291,456 = 0.6328, docs/research_v4_report.md:71-75)."""
    fp16 = 2 * nbytes["k"]
    per_tok_scalar66 = -(-a.dim // 6) * 16 / 6
    b, h, t = a.batch, a.kv_heads, a.tokens
    scalar = nbytes["k"] + b * h * (-(-t // 6) * 6) * per_tok_scalar66 + nbytes["v_meta"]
    return {"kv_over_fp16": round((nbytes["k"] + nbytes["v_blocks"] + nbytes["v_meta"]) / fp16, 4),
            "v_over_fp16_v": round((nbytes["v_blocks"] + nbytes["v_meta"]) / nbytes["k"], 4),
            "scalar6x6_kv_over_fp16": round(scalar / fp16, 4)}


def make_inputs(a, rng_seed=20261201):
    b, hq, hkv, t, d = a.batch, a.query_heads, a.kv_heads, a.tokens, a.dim
    q = np.empty((b, hq, d), np.float32)
    k = np.empty((b, hkv, t, d), np.float16)
    v = np.empty((b, hkv, t, d), np.float32)
    for s in range(b):
        rng = np.random.default_rng(rng_seed + s)
        q[s] = rng.normal(size=(hq, d))
        if a.k_dist == "t3":
            ks = rng.standard_t(3, size=(hkv, t, d))
        else:
            ks = rng.normal(size=(hkv, t, d))
            ks[..., :4] *= 8.0
        k[s] = ks
        v[s] = rng.normal(0.0, 0.5, size=(hkv, t, d))
    return q, k, v


def step_bytes(a, atlas):
    """Algorithmic bytes of one decode step; `split` = what the split kernel must read."""
    b, hq, hkv, t, d = a.batch, a.query_heads, a.kv_heads, a.tokens, a.dim
    rows_read = -(-t // atlas.block_y)
    k_bytes = b * hkv * t * d * 2
    v_bytes = b * hkv * rows_read * atlas.cols * 16
    meta = b * hkv * t * 4
    q_bytes = b * hq * d * 4
    out_bytes = b * hq * d * 4
    return {"k": k_bytes, "v_blocks": v_bytes, "v_meta": meta, "q": q_bytes, "out": out_bytes,
            "split": k_bytes + v_bytes + meta + q_bytes,
            "step": k_bytes + v_bytes + meta + q_bytes + out_bytes}


def time_graph(torch, fn, steps, warmup, use_graph=True):
    """Average ms per call of fn() over `steps`, replayed from one HIP graph
    (falls back to eager launches). Returns (ms, mode)."""
    stream = torch.cuda.current_stream()
    for _ in range(max(warmup, 1)):
        fn(0)
    torch.cuda.synchronize()
    mode = "eager"
    graph = None
    if use_graph:
        try:
            s = torch.cuda.Stream()
            s.wait_stream(stream)
            with torch.cuda.stream(s):
                graph = torch.cuda.CUDAGraph()
                with torch.cuda.graph(graph, stream=s):
                    for i in range(steps):
                        fn(i)
            stream.wait_stream(s)
            graph.replay()
            torch.cuda.synchronize()
            mode = "hipgraph"
        except Exception as e:  # noqa: BLE001
            log(f"graph capture failed ({e}); timing eager launches")
            graph = None
    t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0.record(stream)
    if graph is not None:
        graph.replay()
    else:
        for i in range(steps):
            fn(i)
    t1.record(stream)
    torch.cuda.synchronize()
    return t0.elapsed_time(t1) / steps, mode


def cpu_baseline(q, k, v_restored, seconds):
    """The oracle's NumPy restatement of astc_kv/codec.py:253-267 over the whole
    batch (V already decoded, as in the reference's CPU path). Returns
    (median seconds per step with all cores, cores, median with 1 core, reps)."""
    from threadpoolctl import threadpool_limits

    from oracle import attention_ref as R
    kf = k.astype(np.float32)
    cores = len(os.sched_getaffinity(0))
    res = {}
    for n, budget in ((cores, seconds * 0.6), (1, seconds * 0.4)):
        with threadpool_limits(limits=n):
            for _ in range(3):
                R.decode_attention(q, kf, v_restored)
            times = []
            start = time.perf_counter()
            while (time.perf_counter() - start < budget and len(times) < 200) or len(times) < 5:
                t0 = time.perf_counter()
                R.decode_attention(q, kf, v_restored)
                times.append(time.perf_counter() - t0)
        res[n] = (float(np.median(times)), len(times))
    return res[cores][0], cores, res[1][0], res[cores][1]


def read_traffic(path, workload: str):
    """Traffic per split launch from a profile summary whose `workload:` line
    matches; with no path, the first such summary under profiles/."""
    if path is None:
        for cand in sorted(PROFILES.glob("*.md")):
            got = read_traffic(str(cand), workload)
            if got:
                return got
        return None
    p = Path(path)
    if not p.exists():
        return None
    fields = {}
    for line in p.read_text().splitlines():
        line = line.strip().lstrip("-* ").strip()
        if ":" in line:
            key, val = line.split(":", 1)
            fields[key.strip().strip("`")] = val.strip().strip("`")
    if fields.get("workload") != workload or "traffic_bytes_per_launch" not in fields:
        return None
    return {"bytes": int(fields["traffic_bytes_per_launch"]), "source": str(p.relative_to(ROOT))
            if p.is_relative_to(ROOT) else str(p)}


# --- rocprofv3 summary ----------------------------------------------------------------

def _short(name: str) -> str:
    name = name.replace("akv_hip::", "").replace("(anonymous namespace)::", "").replace("void ", "")
    return name[: name.index("(")] if "(" in name else name


def _counter_means(directory: str, counter: str):
    sums, counts = {}, {}
    for f in glob.glob(os.path.join(directory, "**", "*counter_collection.csv"), recursive=True):
        for r in csv.DictReader(open(f)):
            if r["Counter_Name"] != counter:
                continue
            k = _short(r["Kernel_Name"])
            sums[k] = sums.get(k, 0.0) + float(r["Counter_Value"])
            counts[k] = counts.get(k, 0) + 1
    return {k: sums[k] / counts[k] for k in sums}


def _is_split_kernel(name: str) -> bool:
    """astc_attn_kernel<D, NCH, G, DUMP, WIDE, SPREAD> with DUMP false (not the decode
    readback), or the paged kernel paged_attn_kernel<D, NCH, G, KU4>."""
    if name.startswith("paged_attn_kernel<"):
        return True
    if not name.startswith("astc_attn_kernel<"):
        return False
    args = [x.strip() for x in name[name.index("<") + 1:name.rindex(">")].split(",")]
    return len(args) >= 4 and args[3] == "false"


def summarize_counters(dirs, kernels=("astc_attn_kernel", "fp16_attn_kernel", "paged_attn_kernel")) -> str:
    """Markdown table of every PMC counter found under `dirs` (rocprofv3
    --pmc output), mean per dispatch, for the kernels whose names start with
    one of `kernels`."""
    sums, counts = {}, {}
    for d in dirs:
        for f in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            for r in csv.DictReader(open(f)):
                k = _short(r["Kernel_Name"])
                if not k.startswith(kernels):
                    continue
                key = (k, r["Counter_Name"])
                sums[key] = sums.get(key, 0.0) + float(r["Counter_Value"])
                counts[key] = counts.get(key, 0) + 1
    names = sorted({k for k, _ in sums})
    ctrs = sorted({c for _, c in sums})
    out = ["| counter | " + " | ".join(f"`{n}`" for n in names) + " |", "|---|" + "---|" * len(names)]
    for c in ctrs:
        vals = [f"{sums[(n, c)] / counts[(n, c)]:.4g}" if (n, c) in sums else "" for n in names]
        out.append(f"| {c} | " + " | ".join(vals) + " |")
    return "\n".join(out) + "\n"


def summarize(kt_dir: str, fetch_dir: str, write_dir: str, calib_mb: float, workload: str) -> str:
    rows = []
    for f in glob.glob(os.path.join(kt_dir, "**", "*kernel_stats.csv"), recursive=True):
        for r in csv.DictReader(open(f)):
            rows.append((_short(r["Name"]), int(r["Calls"]), float(r["AverageNs"]) / 1e3, float(r["MinNs"]) / 1e3,
                         float(r["MaxNs"]) / 1e3))
    fetch = _counter_means(fetch_dir, "FETCH_SIZE")
    write = _counter_means(write_dir, "WRITE_SIZE")
    out = ["| kernel | calls | avg µs | min µs | max µs | FETCH_SIZE KiB/dispatch | WRITE_SIZE KiB/dispatch |",
           "|---|---|---|---|---|---|---|"]
    for name, calls, avg, mn, mx in sorted(rows, key=lambda r: -r[1] * r[2]):
        out.append(f"| `{name}` | {calls} | {avg:.2f} | {mn:.2f} | {mx:.2f} | "
                   f"{fetch.get(name, float('nan')):.1f} | {write.get(name, float('nan')):.1f} |")
    text = "\n".join(out) + "\n"
    copy = [k for k in fetch if COPY_KERNEL in k]
    split = [k for k in fetch if _is_split_kernel(k)]
    if copy and calib_mb > 0:
        nbytes = calib_mb * 1e6
        ff = nbytes / (fetch[copy[0]] * 1024)
        wf = nbytes / (write.get(copy[0], float("nan")) * 1024)
        text += (f"\ncopy calibration (`{copy[0]}`, {calib_mb:g} MB read + {calib_mb:g} MB written): "
                 f"bytes per FETCH_SIZE byte = {ff:.4f}, bytes per WRITE_SIZE byte = {wf:.4f}\n")
        if split:
            fb = fetch[split[0]] * 1024 * ff
            wb = write.get(split[0], 0.0) * 1024 * wf
            text += (f"\n- workload: {workload}\n- kernel: `{split[0]}`\n- fetch_bytes_per_launch: {fb:.0f}\n"
                     f"- write_bytes_per_launch: {wb:.0f}\n- traffic_bytes_per_launch: {fb + wb:.0f}\n")
    return text


def copy_calibration(torch, mb: float):
    """A plain copy kernel of known size (mb MB read, mb MB written) for
    scaling the FETCH_SIZE / WRITE_SIZE counters."""
    n = int(mb * 1e6) // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    del src, dst


def ragged_workload_name(a) -> str:
    bx, by = a.block.split("x")
    return (f"paged decode attention, ragged batch of {a.ragged} (T uniform in [{a.min_tokens},{a.tokens}]), "
            f"{a.query_heads}q/{a.kv_heads}kv, D{a.dim}, {a.k_format} K + ASTC {a.layout.upper()} {bx}x{by} V "
            f"(page {a.page}{', FP16 tail' if a.tail else ''}, quality {a.quality:g}), block tables")


def seq_bytes(pk, i) -> int:
    """Algorithmic bytes a decode step reads for sequence i of a paged cache
    (the per-sequence terms of PagedKV.byte_counts)."""
    n, full, h, d = int(pk.seq_lens[i]), pk.full_tokens(i), pk.kv_heads, pk.dim
    k = h * n * (d * 2 if pk.k_format == "fp16" else d // 2 + (d // 32) * 4)
    return k + h * -(-full // pk.block_y) * pk.cols * 16 + h * full * 4 + h * (n - full) * d * 2


def cpu_leg_ragged(q, kv, seconds, sample_bytes, what):
    """The oracle's NumPy attention per sequence of a sample (K, V float32
    [Hkv, T, D] each), all host cores then one."""
    from threadpoolctl import threadpool_limits

    from oracle import attention_ref as R
    cores = len(os.sched_getaffinity(0))

    def once():
        for i, (k, v) in enumerate(kv):
            R.decode_attention(q[i:i + 1], k[None], v[None])

    res = {}
    for n, budget in ((cores, seconds * 0.6), (1, seconds * 0.4)):
        with threadpool_limits(limits=n):
            once()
            times = []
            start = time.perf_counter()
            while (time.perf_counter() - start < budget and len(times) < 200) or len(times) < 3:
                t0 = time.perf_counter()
                once()
                times.append(time.perf_counter() - t0)
        res[n] = (float(np.median(times)), len(times))
    sec, sec1 = res[cores][0], res[1][0]
    return {"value": round(sample_bytes / sec / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": "port",
            "cpu_model": cpu_model(),
            "sample": f"{what}: median of {res[cores][1]} passes of the oracle's NumPy attention "
                      f"(astc_kv/codec.py:253-267) per sequence on pre-decoded K and V, {sec * 1e6:.0f} us per pass "
                      f"on {cores} cores ({sec1 * 1e6:.0f} us on 1 core); GB/s over the sample's algorithmic bytes",
            "us_per_sample": round(sec * 1e6, 1), "us_per_sample_1core": round(sec1 * 1e6, 1),
            "sample_bytes": int(sample_bytes)}


def ragged_inputs(a):
    """The ragged batch's sequence lengths, paged pool and queries (seeded;
    from the --cache directory when a previous run saved them)."""
    from astc_kv.paged import PagedKV, build_paged
    bx, by = (int(x) for x in a.block.split("x"))
    rng = np.random.default_rng(20261202)
    lens = rng.integers(a.min_tokens, a.tokens + 1, size=a.ragged).tolist()
    log(f"building {a.ragged} paged sequences, {sum(lens)} tokens: {ragged_workload_name(a)}")
    t0 = time.perf_counter()
    path = _cache_path(a, f"paged-q{a.quality:g}")
    if path is not None and path.exists():
        z = np.load(path)
        pk = PagedKV(z["k_pages"], z["k_meta"] if "k_meta" in z else None, z["v_blocks"], z["v_scale"], z["v_offset"],
                     z["block_table"], z["seq_lens"], z["v_tail"] if "v_tail" in z else None, a.dim, a.layout, bx, by,
                     a.page, a.k_format)
        q = z["q"]
    else:
        k, v = [], []
        for t in lens:
            kk = rng.normal(size=(a.kv_heads, t, a.dim)).astype(np.float32)
            kk[..., :4] *= 8.0
            k.append(kk.astype(np.float16))
            v.append(rng.normal(0.0, 0.5, size=(a.kv_heads, t, a.dim)).astype(np.float32))
        pk = build_paged(k, v, a.layout, (bx, by), a.page, a.quality, a.k_format, a.tail, seed=7,
                         progress=lambda i, n: log(f"  encoded {i}/{n} sequences") if i % 8 == 0 or i == n else None)
        del k, v
        q = rng.normal(size=(a.ragged, a.query_heads, a.dim)).astype(np.float32)
        if path is not None:
            path.parent.mkdir(parents=True, exist_ok=True)
            np.savez(path, q=q, **{f: getattr(pk, f) for f in ("k_pages", "k_meta", "v_blocks", "v_scale",
                                                               "v_offset", "block_table", "seq_lens", "v_tail")
                                   if getattr(pk, f) is not None})
    return lens, pk, q, time.perf_counter() - t0


def main_ragged(a, torch, gpu):
    """A ragged batch in page pools with block tables (akv_hip_paged_decode_attention)."""
    from astc_kv.atlas import block_class_histogram
    from oracle import attention_ref as R
    from oracle.paged_ref import host_kv

    bx, by = (int(x) for x in a.block.split("x"))
    lens, pk, q, setup_s = ragged_inputs(a)
    cache = gpu.DevicePagedKV.from_host(pk)
    qt = torch.from_numpy(q).cuda()
    params = gpu.paged_params(cache, a.query_heads, a.tile or None)
    s = params.splits
    partial = torch.empty((a.ragged, a.query_heads, s, a.dim), dtype=torch.float32, device="cuda")
    stats = torch.empty((a.ragged, a.query_heads, s, 2), dtype=torch.float32, device="cuda")
    out = torch.empty((a.ragged, a.query_heads, a.dim), dtype=torch.float32, device="cuda")
    counts = pk.byte_counts()
    step_bytes_ = counts["total"] + 2 * a.ragged * a.query_heads * a.dim * 4

    def step(i):
        gpu.paged_decode_attention(qt, cache, params=params, partial=partial, stats=stats, out=out)

    if a.copy_calibration_mb > 0:
        copy_calibration(torch, a.copy_calibration_mb)
    traffic = read_traffic(a.traffic, ragged_workload_name(a))
    log(f"timing {a.steps} steps (tile {params.tile_tokens}, {s} splits max)")
    ms_step, mode = time_graph(torch, step, a.steps, a.warmup, not a.no_graph)

    ceiling = copy_ceiling(torch, a.copy_ceiling_mb)
    # Parity on the shortest and the longest sequence.
    step(0)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    sub = [int(np.argmin(lens)), int(np.argmax(lens))]
    max_err, parity = 0.0, True
    host = {}
    for i in sub:
        host[i] = host_kv(pk, i)
        ref = R.decode_attention(q[i:i + 1], host[i][0][None], host[i][1][None])[0]
        max_err = max(max_err, float(np.max(np.abs(got[i] - ref))))
        parity = parity and bool(np.allclose(got[i], ref, rtol=1e-3, atol=2e-3))

    cpu = None
    if not a.no_cpu:
        # A bounded sample: the first sequences of the batch up to about 64k
        # tokens, K and V pre-decoded on the host, one NumPy attention each.
        n_s, tok = 0, 0
        while n_s < len(lens) and (tok < 65536 or n_s == 0):
            tok += lens[n_s]
            n_s += 1
        log(f"timing the CPU baseline on {n_s} sequences ({tok} tokens)")
        kv = [host.get(i) or host_kv(pk, i) for i in range(n_s)]
        sample_bytes = sum(seq_bytes(pk, i) + 2 * a.query_heads * a.dim * 4 for i in range(n_s))
        cpu = cpu_leg_ragged(q[:n_s], kv, a.cpu_seconds, sample_bytes,
                             f"the first {n_s} sequences of the batch ({tok} of {sum(lens)} tokens)")
        del kv

    value = step_bytes_ / (ms_step * 1e-3) / 1e9
    line = {
        "metric": "µs per decode-attention step + effective KV GB/s (% HBM peak)",
        "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(ms_step, 6), "us_per_step": round(ms_step * 1e3, 3),
        "pct_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": f"{a.k_format} K / ASTC V (u16 texels), fp32 accumulate",
        "data": "synthetic (seeded Gaussian K/V/q), V encoded by this package's ASTC encoder",
        "config": {"workload": ragged_workload_name(a), "sequences": a.ragged, "tokens_total": int(sum(lens)),
                   "tokens_max": int(max(lens)), "query_heads": a.query_heads, "kv_heads": a.kv_heads,
                   "dim": a.dim, "layout": a.layout, "block": [bx, by], "page_tokens": a.page,
                   "k_format": a.k_format, "tail": a.tail, "tile_tokens": params.tile_tokens,
                   "splits_max": s, "timing": mode, "bytes_per_step": {**counts, "step": step_bytes_}},
        "roofline": {"bound": "hbm", "achieved": round(value, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(value / HBM_PEAK_GBS, 4), "traffic": traffic["bytes"] if traffic else None,
                     "traffic_source": traffic["source"] if traffic else None,
                     "kernel": "paged_attn_kernel (split + in-kernel merge)", "bytes_per_launch": step_bytes_,
                     "us_per_launch": round(ms_step * 1e3, 3)},
        "cpu_baseline": cpu,
        "v_blocks": block_class_histogram(pk.v_blocks[np.unique(np.concatenate(
            [pk.block_table[i, :-(-pk.full_tokens(i) // a.page)] for i in range(a.ragged)]))], bx, by, a.layout),
        "copy_ceiling": ceiling,
        "parity": {"sequences_checked": sub, "max_abs_err": max_err, "within_rtol1e-3_atol2e-3": parity},
        "setup_s": round(setup_s, 2),
    }
    emit(a, line)
    return 0 if parity else 1


def oracle_values(atlas, sub):
    """V of sequences `sub` restored on the host from the oracle's decode of
    their blocks (float32 [len(sub), Hkv, T, D])."""
    from astc_kv.atlas import Atlas
    from oracle import astc_oracle as O
    from oracle import attention_ref as R
    bx, by = atlas.block_x, atlas.block_y
    small = Atlas(atlas.blocks[sub], atlas.scale[sub], atlas.offset[sub], atlas.tokens, atlas.dim, atlas.layout,
                  bx, by, atlas.page_tokens)
    tex, _ = O.decode_blocks_fp16(small.blocks.reshape(-1, 16), bx, by)
    bb, hh, rr, cc = small.blocks.shape[:4]
    img = tex.reshape(bb, hh, rr, cc, by, bx, 4).transpose(0, 1, 2, 4, 3, 5, 6).reshape(bb, hh, rr * by, cc * bx, 4)
    img = img[:, :, : atlas.tokens].astype(np.float32)
    d = atlas.dim
    un = img[..., :d, 0] if atlas.layout == "scalar" else img[:, :, :, : d // 4].reshape(bb, hh, atlas.tokens, d)
    return R.restore_token(un, small.scale.astype(np.float32)[..., None], small.offset.astype(np.float32)[..., None])


def time_atlas(a, torch, gpu, qt, kt, dev, params, steps, warmup):
    """(pooled ms per step, resident ms per step, pool size) of the one-launch
    decode step over `dev`."""
    s = params.splits
    partial = torch.empty((a.batch, a.query_heads, s, a.dim), dtype=torch.float32, device="cuda")
    stats = torch.empty((a.batch, a.query_heads, s, 2), dtype=torch.float32, device="cuda")
    out = torch.empty((a.batch, a.query_heads, a.dim), dtype=torch.float32, device="cuda")
    set_bytes = kt.numel() * 2 + dev.nbytes() + qt.numel() * 4
    pool_n = max(1, int(np.ceil(a.pool_mb * 1e6 / set_bytes)))
    pool = [(kt, dev)] + [(kt.clone(), dev.clone()) for _ in range(pool_n - 1)]

    def step(i):
        kk, dd = pool[i % pool_n]
        gpu.decode_attention(qt, kk, dd, params=params, partial=partial, stats=stats, out=out)

    torch.cuda.synchronize()
    ms_step, mode = time_graph(torch, step, steps, warmup, not a.no_graph)
    # The same launches one by one (what a profiler's per-kernel average sees:
    # without graph replay consecutive launches do not overlap).
    ms_eager = time_graph(torch, step, steps, warmup, False)[0] if mode == "hipgraph" else ms_step

    def resident(i):
        gpu.decode_attention(qt, kt, dev, params=params, partial=partial, stats=stats, out=out)

    ms_resident = float("nan") if a.no_resident else time_graph(torch, resident, steps, warmup, not a.no_graph)[0]
    del pool
    return ms_step, ms_resident, pool_n, mode, ms_eager


def cpu_leg(q, k, v_rest, seconds, step_bytes_, what):
    """The oracle's NumPy attention timed on the host cores (all, then one)."""
    sec, cores, sec1, reps = cpu_baseline(q, k, v_rest, seconds)
    return {"value": round(step_bytes_ / sec / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": "port",
            "cpu_model": cpu_model(),
            "sample": f"{what}: median of {reps} steps of the oracle's NumPy attention (astc_kv/codec.py:253-267) "
                      f"on pre-decoded V, {sec * 1e6:.0f} us/step on {cores} cores ({sec1 * 1e6:.0f} us/step on "
                      f"1 core)",
            "us_per_step": round(sec * 1e6, 1), "us_per_step_1core": round(sec1 * 1e6, 1)}


def emit(a, line) -> None:
    text = json.dumps(line)
    print(text, flush=True)
    if a.out:
        Path(a.out).parent.mkdir(parents=True, exist_ok=True)
        Path(a.out).write_text(text + "\n")


REFERENCE_TILES = {384: 32, 2048: 64, 8192: 256}           # configs/address_v7_20261029.json
REFERENCE_M5PRO_US = {384: (7.842, 5.733), 2048: (16.014, 11.738), 8192: (39.659, 25.337)}   # v7 hoisted, own FP16


def fixture_workload_name(a, m) -> str:
    return (f"reference fixture {Path(a.fixture).name} ({m['encoder']['name']} {m['encoder']['version']} "
            f"quality {m['encoder']['quality']:g}, {m['layout']} ASTC {a.block}, page {a.page}) repeated to "
            f"T{a.tokens}, batch 1, {m['query_heads']}q/{m['kv_heads']}kv, D{m['head_dim']}, FP16 K")


def main_fixture(a, torch, gpu):
    """The reference's own astcenc payloads (an astc-kv-probe-v1 fixture),
    repeated to a.tokens keys, through the probe's correctness gates, then
    timed at the host's tile and at the reference's."""
    from astc_kv import probe
    from astc_kv.atlas import block_class_histogram
    fx = probe.load_fixture(Path(a.fixture) / "manifest.json")
    if a.tokens != fx["atlas"].tokens:
        fx = probe.repeat_tokens(fx, a.tokens)
    m = fx["manifest"]
    atlas = fx["atlas"]
    dev = gpu.DeviceAtlas.from_host(atlas)
    qt = torch.from_numpy(fx["q"]).cuda()
    kt = torch.from_numpy(fx["k"]).cuda()
    a.batch, a.query_heads, a.kv_heads, a.dim = 1, m["query_heads"], m["kv_heads"], m["head_dim"]
    a.layout, a.block, a.page = atlas.layout, f"{atlas.block_x}x{atlas.block_y}", atlas.page_tokens
    ref_tile = a.ref_tile or REFERENCE_TILES.get(a.tokens)
    # Gates first, as the reference's probe does (probe_gqa_v10.mm:704-784).
    params = gpu.make_params(dev, a.query_heads, a.tile or None)
    u = gpu.decode_values(dev, params.tile_tokens)
    v_restored = (u.float() * dev.scale.float()[..., None]) + dev.offset.float()[..., None]
    out = gpu.decode_attention(qt, kt, dev, params=params)
    out16 = gpu.fp16_attention(qt, kt, v_restored.half(), fused=False)
    torch.cuda.synchronize()
    passed, correctness = probe.gates(fx, v_restored.cpu().numpy(), out.cpu().numpy(), out16.cpu().numpy())
    if not passed:
        emit(a, probe.refusal(correctness))
        return 1
    nbytes = step_bytes(a, atlas)
    runs = {}
    for name, tile in (("host_tile", a.tile or None), ("reference_tile", ref_tile)):
        if tile is None and name == "reference_tile":
            continue
        p = gpu.make_params(dev, a.query_heads, tile)
        ms, ms_res, pool_n, mode, _ = time_atlas(a, torch, gpu, qt, kt, dev, p, a.steps, a.warmup)
        runs[name] = {"tile_tokens": p.tile_tokens, "splits": p.splits, "us_per_step": round(ms * 1e3, 3),
                      "us_per_step_resident": round(ms_res * 1e3, 3), "pool_sets": pool_n,
                      "GB/s": round(nbytes["step"] / (ms * 1e-3) / 1e9, 2)}
    fparams = gpu.fp16_params(1, a.kv_heads, a.query_heads, a.tokens, a.dim, ref_tile)
    v16 = v_restored.half()
    fpart = torch.empty((1, a.query_heads, fparams.splits, a.dim), dtype=torch.float32, device="cuda")
    fstat = torch.empty_like(fpart[..., :2])

    def fstep(i):
        gpu.fp16_attention(qt, kt, v16, params=fparams, partial=fpart, stats=fstat, out=out, fused=False)

    ms_fp16, _ = time_graph(torch, fstep, a.steps, a.warmup, not a.no_graph)
    best = min(runs.values(), key=lambda r: r["us_per_step"])
    ms_step = best["us_per_step"] * 1e-3
    value = nbytes["step"] / (ms_step * 1e-3) / 1e9
    published = REFERENCE_M5PRO_US.get(a.tokens)
    cpu = None
    if not a.no_cpu:
        cpu = cpu_leg(fx["q"], fx["k"], v_restored.cpu().numpy(), a.cpu_seconds, nbytes["step"],
                      f"the whole fixture step (batch 1, T{a.tokens})")
    line = {
        "metric": "µs per decode-attention step + effective KV GB/s (% HBM peak)",
        "value": round(value, 2), "unit": "GB/s", "n_gpus": 1, "steps": a.steps, "warmup": a.warmup,
        "ms_per_step": round(ms_step, 6), "us_per_step": best["us_per_step"],
        "pct_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp16 K / ASTC V (u16 texels), fp32 accumulate",
        "data": f"the reference's {m['model']} layer {m['layer']} capture, {m['encoder']['name']} "
                f"{m['encoder']['version']} payloads, repeated (synthetic traffic control, not quality evidence)",
        "config": {"workload": fixture_workload_name(a, m), "tokens": a.tokens, "source_tokens": m.get(
                   "source_tokens", a.tokens), "layout": a.layout, "block": [atlas.block_x, atlas.block_y],
                   "timing": "hipgraph" if not a.no_graph else "eager", "bytes_per_step": nbytes},
        "runs": runs,
        "roofline": {"bound": "hbm", "achieved": round(value, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(value / HBM_PEAK_GBS, 4), "traffic": None,
                     "kernel": "astc_attn_kernel (split + in-kernel merge, ASTC V)",
                     "bytes_per_launch": nbytes["step"], "us_per_launch": best["us_per_step"],
                     "note": "launch-latency bound at these sizes; the fraction is not meaningful below ~1 MB"},
        "fp16_control": {"us_per_step": round(ms_fp16 * 1e3, 3), "tile_tokens": fparams.tile_tokens},
        "reference_m5pro_us": None if published is None else {
            "astc_v7_hoisted": published[0], "fp16_own": published[1],
            "source": "docs/research_v3_report.md:28-32 (medians of session medians, warm, one resident cache)"},
        "v_blocks": block_class_histogram(atlas.blocks, atlas.block_x, atlas.block_y, atlas.layout),
        "correctness": correctness,
        "cpu_baseline": cpu,
    }
    emit(a, line)
    return 0


def main(argv=None):
    a = parse_args(argv)
    if a.summarize:
        print(summarize(*a.summarize, a.copy_calibration_mb,
                        ragged_workload_name(a) if a.ragged else workload_name(a)))
        return 0
    if a.counters:
        print(summarize_counters(a.counters))
        return 0
    if a.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {a.gpus} is not supported (run with --gpus 1)",
              file=sys.stderr)
        return 2
    import torch

    from astc_kv import gpu
    if a.fixture:
        return main_fixture(a, torch, gpu)
    if a.ragged:
        return main_ragged(a, torch, gpu)
    from astc_kv.atlas import block_class_histogram
    from oracle import astc_oracle as O
    from oracle import attention_ref as R

    bx, by = (int(x) for x in a.block.split("x"))
    log(f"encoding the V atlas: {workload_name(a)}")
    t_setup = time.perf_counter()
    q, k, v = make_inputs(a)
    atlas = cached_atlas(a, v, a.quality)
    setup_s = time.perf_counter() - t_setup
    atlas_cmp = None
    if a.compare_quality > 0 and a.compare_quality != a.quality:
        log(f"encoding the comparison atlas at quality {a.compare_quality:g}")
        atlas_cmp = cached_atlas(a, v, a.compare_quality)
    del v
    dev = gpu.DeviceAtlas.from_host(atlas)
    qt = torch.from_numpy(q).cuda()
    kt = torch.from_numpy(k).cuda()
    params = gpu.make_params(dev, a.query_heads, a.tile or None)
    nbytes = step_bytes(a, atlas)
    out = torch.empty((a.batch, a.query_heads, a.dim), dtype=torch.float32, device="cuda")

    if a.copy_calibration_mb > 0:
        copy_calibration(torch, a.copy_calibration_mb)

    log(f"timing {a.steps} steps (tile {params.tile_tokens}, {params.splits} splits)")
    ms_step, ms_resident, pool_n, mode, ms_eager = time_atlas(a, torch, gpu, qt, kt, dev, params, a.steps, a.warmup)

    cmp = None
    if atlas_cmp is not None:
        log(f"timing the quality {a.compare_quality:g} atlas")
        dev_c = gpu.DeviceAtlas.from_host(atlas_cmp)
        ms_c, ms_c_res, _, _, _ = time_atlas(a, torch, gpu, qt, kt, dev_c, params, a.steps, a.warmup)
        cmp = {"quality": a.compare_quality, "us_per_step": round(ms_c * 1e3, 3),
               "us_per_step_resident": round(ms_c_res * 1e3, 3),
               "GB/s": round(nbytes["step"] / (ms_c * 1e-3) / 1e9, 2),
               "frac": round(nbytes["step"] / (ms_c * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
               "v_blocks": block_class_histogram(atlas_cmp.blocks, bx, by, a.layout)}
        del dev_c

    # FP16 K/V control on the same workload (V = restored values rounded to fp16).
    log("timing the FP16-K/V control")
    u = gpu.decode_values(dev)
    v16 = (u.float() * dev.scale.float()[..., None] + dev.offset.float()[..., None]).half()
    del u
    fparams = gpu.fp16_params(a.batch, a.kv_heads, a.query_heads, a.tokens, a.dim, a.fp16_tile or None)
    fpool = [(kt, v16)] + [(kt.clone(), v16.clone()) for _ in range(max(1, int(np.ceil(
        a.pool_mb * 1e6 / (kt.numel() * 4)))) - 1)]
    fpart = torch.empty((a.batch, a.query_heads, fparams.splits, a.dim), dtype=torch.float32, device="cuda")
    fstat = torch.empty_like(fpart[..., :2])

    def fstep(i):
        kk, vv = fpool[i % len(fpool)]
        # Split + merge launches: the control's fastest form (its one-launch
        # merge pays an L2 write-back per workgroup for the release fence).
        gpu.fp16_attention(qt, kk, vv, params=fparams, partial=fpart, stats=fstat, out=out, fused=False)

    ms_fp16, _ = time_graph(torch, fstep, a.steps, a.warmup, not a.no_graph)
    fp16_bytes = nbytes["k"] * 2 + nbytes["q"] + nbytes["out"]
    del fpool, v16
    ceiling = copy_ceiling(torch, a.copy_ceiling_mb)

    # Correctness of the measured configuration on two sequences (oracle decode + NumPy attention).
    log("checking two sequences against the oracle")
    gpu.decode_attention(qt, kt, dev, params=params, out=out)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    sub = [0, a.batch - 1]
    vr = oracle_values(atlas, sub)
    ref = R.decode_attention(q[sub], k[sub].astype(np.float32), vr)
    max_err = float(np.max(np.abs(got[sub] - ref)))
    parity = bool(np.allclose(got[sub], ref, rtol=1e-3, atol=2e-3))

    cpu = None
    if not a.no_cpu:
        log("timing the CPU baseline (oracle decode + NumPy attention)")
        t0 = time.perf_counter()
        O.decode_blocks_fp16(atlas.blocks.reshape(-1, 16), bx, by)
        decode_s = time.perf_counter() - t0
        v_rest = oracle_values(atlas, list(range(a.batch)))
        cpu = cpu_leg(q, k, v_rest, a.cpu_seconds, nbytes["step"], f"full workload (batch {a.batch}, T{a.tokens})")
        cpu["sample"] += (f"; the oracle's single-threaded C ASTC decode of the whole atlas took "
                          f"{decode_s * 1e6:.0f} us more, not folded in")
        cpu["astc_decode_us_1core"] = round(decode_s * 1e6, 1)
        del v_rest

    value = nbytes["step"] / (ms_step * 1e-3) / 1e9
    traffic = read_traffic(a.traffic, workload_name(a))
    line = {
        "metric": "µs per decode-attention step + effective KV GB/s (% HBM peak) at T8192",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms_step, 6),
        "us_per_step": round(ms_step * 1e3, 3),
        "pct_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16 K / ASTC V (u16 texels), fp32 accumulate",
        "data": f"synthetic (seeded Gaussian K/V/q), V encoded by this package's ASTC encoder at quality "
                f"{a.quality:g}",
        "config": {"workload": workload_name(a),
                   "batch": a.batch, "tokens": a.tokens, "query_heads": a.query_heads, "kv_heads": a.kv_heads,
                   "dim": a.dim, "layout": a.layout, "block": [bx, by], "quality": a.quality,
                   "tile_tokens": params.tile_tokens, "splits": params.splits, "pool_sets": pool_n,
                   "timing": mode, "bytes_per_step": nbytes, "byte_ratios": byte_ratios(a, nbytes)},
        "roofline": {"bound": "hbm", "achieved": round(value, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(value / HBM_PEAK_GBS, 4),
                     "traffic": traffic["bytes"] if traffic else None,
                     "traffic_source": traffic["source"] if traffic else None,
                     "kernel": "astc_attn_kernel (split + in-kernel merge, ASTC V)",
                     "bytes_per_launch": nbytes["step"], "us_per_launch": round(ms_step * 1e3, 3),
                     "eager_us_per_launch": round(ms_eager * 1e3, 3)},
        "cpu_baseline": cpu,
        "v_blocks": block_class_histogram(atlas.blocks, bx, by, a.layout),
        "quality_50" if a.compare_quality == 50 else "quality_compare": cmp,
        "resident_single_set": None if a.no_resident else {
            "us_per_step": round(ms_resident * 1e3, 3), "GB/s": round(nbytes["step"] / (ms_resident * 1e-3) / 1e9, 2)},
        "fp16_control": {"us_per_step": round(ms_fp16 * 1e3, 3), "bytes_per_step": fp16_bytes,
                         "GB/s": round(fp16_bytes / (ms_fp16 * 1e-3) / 1e9, 2), "tile_tokens": fparams.tile_tokens,
                         "astc_speedup": round(ms_fp16 / ms_step, 4)},
        "copy_ceiling": ceiling,
        "parity": {"sequences_checked": sub, "max_abs_err": max_err, "within_rtol1e-3_atol2e-3": parity},
        "setup_s": round(setup_s, 2),
    }
    emit(a, line)
    return 0 if parity else 1


if __name__ == "__main__":
    sys.exit(main())
