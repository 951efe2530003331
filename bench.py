#!/usr/bin/env python3
"""Decode-attention benchmark: ASTC-V split-K attention on one MI355X.

Workload (one step = one decode step of the whole batch): T=8192 keys per
sequence, batch 16, 9 query heads / 3 KV heads, head dim 64, FP16 K, V as an
ASTC RGBA 6x5 atlas (page 120) with per-token fp16 scale/offset; independent
seeded K/V per sequence (K ~ N(0,1) with 4 channels x8, V ~ N(0, 0.5), q ~ N(0,1)).

Inputs are resident in HBM. A pool of distinct copies of the KV set (> 512 MB
in total) is rotated across steps so that the 256 MB Infinity Cache cannot
hold the working set; every step is timed as split + merge launches replayed
from a HIP graph, with events on the launch stream.

Prints one JSON line. `value` is the effective bandwidth: algorithmic bytes
of a step (K + ASTC blocks read + V scale/offset + q + out) / step time.
`roofline.achieved` is the split kernel's algorithmic bytes (K + ASTC blocks
+ V scale/offset + q) / its own launch time. `roofline.traffic` is the HBM
traffic per split launch that rocprofv3 measured (FETCH_SIZE + WRITE_SIZE,
scaled by a plain copy kernel of known size) for this same workload, read from
the committed profile summary when its workload line matches.

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
    ap.add_argument("--quality", type=float, default=50.0, help="encoder effort for the synthetic V atlas")
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
    ap.add_argument("--ragged", type=int, default=0,
                    help="paged ragged batch of this many sequences (lengths uniform in "
                         "[--min-tokens, --tokens]) instead of the uniform batch")
    ap.add_argument("--min-tokens", type=int, default=512)
    ap.add_argument("--k-format", default="fp16", choices=["fp16", "u4g32"], help="K storage (paged batches)")
    ap.add_argument("--tail", action="store_true", help="paged: keep each sequence's partial last page as FP16 V")
    return ap.parse_args(argv)


def workload_name(a) -> str:
    bx, by = a.block.split("x")
    return (f"decode attention T{a.tokens} batch {a.batch}, {a.query_heads}q/{a.kv_heads}kv, D{a.dim}, "
            f"FP16 K + ASTC {a.layout.upper()} {bx}x{by} V (page {a.page})")


def make_inputs(a, rng_seed=20261201):
    b, hq, hkv, t, d = a.batch, a.query_heads, a.kv_heads, a.tokens, a.dim
    q = np.empty((b, hq, d), np.float32)
    k = np.empty((b, hkv, t, d), np.float16)
    v = np.empty((b, hkv, t, d), np.float32)
    for s in range(b):
        rng = np.random.default_rng(rng_seed + s)
        q[s] = rng.normal(size=(hq, d))
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
    """astc_attn_kernel<D, NCH, G, DUMP, WIDE> with DUMP false (not the decode
    readback), or the paged kernel paged_attn_kernel<D, NCH, G, KU4>."""
    if name.startswith("paged_attn_kernel<"):
        return True
    if not name.startswith("astc_attn_kernel<"):
        return False
    args = [x.strip() for x in name[name.index("<") + 1:name.rindex(">")].split(",")]
    return len(args) >= 4 and args[3] == "false"


def summarize_counters(dirs, kernels=("astc_attn_kernel", "fp16_attn_kernel")) -> str:
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
            f"(page {a.page}{', FP16 tail' if a.tail else ''}), block tables")


def main_ragged(a, torch, gpu):
    """A ragged batch in page pools with block tables (akv_hip_paged_decode_attention)."""
    from astc_kv.paged import build_paged
    from oracle import astc_oracle as O
    from oracle import attention_ref as R

    bx, by = (int(x) for x in a.block.split("x"))
    rng = np.random.default_rng(20261202)
    lens = rng.integers(a.min_tokens, a.tokens + 1, size=a.ragged).tolist()
    log(f"building {a.ragged} paged sequences, {sum(lens)} tokens: {ragged_workload_name(a)}")
    t0 = time.perf_counter()
    k, v = [], []
    for t in lens:
        kk = rng.normal(size=(a.kv_heads, t, a.dim)).astype(np.float32)
        kk[..., :4] *= 8.0
        k.append(kk.astype(np.float16))
        v.append(rng.normal(0.0, 0.5, size=(a.kv_heads, t, a.dim)).astype(np.float32))
    pk = build_paged(k, v, a.layout, (bx, by), a.page, a.quality, a.k_format, a.tail, seed=7,
                     progress=lambda i, n: log(f"  encoded {i}/{n} sequences") if i % 8 == 0 or i == n else None)
    setup_s = time.perf_counter() - t0
    cache = gpu.DevicePagedKV.from_host(pk)
    q = rng.normal(size=(a.ragged, a.query_heads, a.dim)).astype(np.float32)
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

    # Parity on the shortest and the longest sequence.
    step(0)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    sub = [int(np.argmin(lens)), int(np.argmax(lens))]
    max_err, parity = 0.0, True
    for i in sub:
        t, P, h, d = lens[i], a.page, a.kv_heads, a.dim
        ids = pk.block_table[i, :-(-t // P)]
        if a.k_format == "fp16":
            ki = pk.k_pages[ids].transpose(1, 0, 2, 3).reshape(h, -1, d)[:, :t].astype(np.float32)
        else:
            kb = pk.k_pages[ids].transpose(1, 0, 2, 3).reshape(h, -1, d // 2)[:, :t]
            codes = np.stack([kb & 15, kb >> 4], -1).reshape(h, t, d // 32, 32).astype(np.float32)
            meta = pk.k_meta[ids].transpose(1, 0, 2, 3, 4).reshape(h, -1, d // 32, 2)[:, :t].astype(np.float32)
            ki = (codes * meta[..., 1:2] + meta[..., 0:1]).reshape(h, t, d)
        full = pk.full_tokens(i)
        parts = []
        if full:
            npg, rpp, cols = -(-full // P), P // by, pk.cols
            blocks = pk.v_blocks[ids[:npg]].transpose(1, 0, 2, 3, 4).reshape(h, npg * rpp, cols, 16)
            tex, _ = O.decode_blocks_fp16(np.ascontiguousarray(blocks).reshape(-1, 16), bx, by)
            img = tex.reshape(h, npg * rpp, cols, by, bx, 4).transpose(0, 1, 3, 2, 4, 5)
            img = img.reshape(h, npg * P, cols * bx, 4)[:, :full].astype(np.float32)
            u = img[..., :d, 0] if a.layout == "scalar" else img[:, :, : d // 4].reshape(h, full, d)
            sc = pk.v_scale[ids[:npg]].transpose(1, 0, 2).reshape(h, -1)[:, :full].astype(np.float32)
            of = pk.v_offset[ids[:npg]].transpose(1, 0, 2).reshape(h, -1)[:, :full].astype(np.float32)
            parts.append(R.restore_token(u, sc[..., None], of[..., None]))
        if full < t:
            parts.append(pk.v_tail[i, :, : t - full].astype(np.float32))
        ref = R.decode_attention(q[i:i + 1], ki[None], np.concatenate(parts, 1)[None])[0]
        max_err = max(max_err, float(np.max(np.abs(got[i] - ref))))
        parity = parity and bool(np.allclose(got[i], ref, rtol=1e-3, atol=2e-3))

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
        "cpu_baseline": None,
        "parity": {"sequences_checked": sub, "max_abs_err": max_err, "within_rtol1e-3_atol2e-3": parity},
        "setup_s": round(setup_s, 2),
    }
    text = json.dumps(line)
    print(text, flush=True)
    if a.out:
        Path(a.out).parent.mkdir(parents=True, exist_ok=True)
        Path(a.out).write_text(text + "\n")
    return 0 if parity else 1


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
    if a.ragged:
        return main_ragged(a, torch, gpu)
    from astc_kv.atlas import Atlas, build_atlas
    from oracle import astc_oracle as O
    from oracle import attention_ref as R

    bx, by = (int(x) for x in a.block.split("x"))
    log(f"encoding the V atlas: {workload_name(a)}")
    t_setup = time.perf_counter()
    q, k, v = make_inputs(a)
    atlas = build_atlas(v, a.layout, (bx, by), a.page, a.quality)
    setup_s = time.perf_counter() - t_setup
    dev = gpu.DeviceAtlas.from_host(atlas)
    qt = torch.from_numpy(q).cuda()
    kt = torch.from_numpy(k).cuda()
    params = gpu.make_params(dev, a.query_heads, a.tile or None)
    nbytes = step_bytes(a, atlas)
    set_bytes = kt.numel() * 2 + dev.nbytes() + qt.numel() * 4
    pool_n = max(1, int(np.ceil(a.pool_mb * 1e6 / set_bytes)))
    pool = [(kt, dev)] + [(kt.clone(), dev.clone()) for _ in range(pool_n - 1)]
    s = params.splits
    partial = torch.empty((a.batch, a.query_heads, s, a.dim), dtype=torch.float32, device="cuda")
    stats = torch.empty((a.batch, a.query_heads, s, 2), dtype=torch.float32, device="cuda")
    out = torch.empty((a.batch, a.query_heads, a.dim), dtype=torch.float32, device="cuda")

    if a.copy_calibration_mb > 0:
        copy_calibration(torch, a.copy_calibration_mb)

    # One launch per step: the split kernel with the merge done by the last
    # split workgroup of each (sequence, kv head).
    def step(i):
        kk, dd = pool[i % pool_n]
        gpu.decode_attention(qt, kk, dd, params=params, partial=partial, stats=stats, out=out)

    torch.cuda.synchronize()
    log(f"timing {a.steps} steps (tile {params.tile_tokens}, {s} splits, pool of {pool_n} KV sets)")
    ms_step, mode = time_graph(torch, step, a.steps, a.warmup, not a.no_graph)

    def resident(i):
        gpu.decode_attention(qt, kt, dev, params=params, partial=partial, stats=stats, out=out)

    ms_resident, _ = time_graph(torch, resident, a.steps, a.warmup, not a.no_graph)

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
    del fpool

    # Correctness of the measured configuration on two sequences (oracle decode + NumPy attention).
    log("checking two sequences against the oracle")
    step(0)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    sub = [0, a.batch - 1]
    small = Atlas(atlas.blocks[sub], atlas.scale[sub], atlas.offset[sub], a.tokens, a.dim, a.layout, bx, by, a.page)
    tex, _ = O.decode_blocks_fp16(small.blocks.reshape(-1, 16), bx, by)
    bb, hh, rr, cc = small.blocks.shape[:4]
    img = tex.reshape(bb, hh, rr, cc, by, bx, 4).transpose(0, 1, 2, 4, 3, 5, 6).reshape(bb, hh, rr * by, cc * bx, 4)
    img = img[:, :, : a.tokens].astype(np.float32)
    un = img[..., : a.dim, 0] if a.layout == "scalar" else img[:, :, :, : a.dim // 4].reshape(bb, hh, a.tokens, a.dim)
    vr = R.restore_token(un, small.scale.astype(np.float32)[..., None], small.offset.astype(np.float32)[..., None])
    ref = R.decode_attention(q[sub], k[sub].astype(np.float32), vr)
    max_err = float(np.max(np.abs(got[sub] - ref)))
    parity = bool(np.allclose(got[sub], ref, rtol=1e-3, atol=2e-3))

    cpu = None
    if not a.no_cpu:
        log("timing the CPU baseline (oracle decode + NumPy attention)")
        t0 = time.perf_counter()
        tex_all, _ = O.decode_blocks_fp16(atlas.blocks.reshape(-1, 16), bx, by)
        decode_s = time.perf_counter() - t0
        bb, hh, rr, cc = atlas.blocks.shape[:4]
        img = tex_all.reshape(bb, hh, rr, cc, by, bx, 4).transpose(0, 1, 2, 4, 3, 5, 6)
        img = img.reshape(bb, hh, rr * by, cc * bx, 4)[:, :, : a.tokens].astype(np.float32)
        un = img[..., : a.dim, 0] if a.layout == "scalar" else img[:, :, :, : a.dim // 4].reshape(
            bb, hh, a.tokens, a.dim)
        v_rest = R.restore_token(un, atlas.scale.astype(np.float32)[..., None],
                                 atlas.offset.astype(np.float32)[..., None])
        del tex_all, img, un
        sec, cores, sec1, reps = cpu_baseline(q, k, v_rest, a.cpu_seconds)
        cpu = {"value": round(nbytes["step"] / sec / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": "port",
               "sample": f"full workload (batch {a.batch}, T{a.tokens}): median of {reps} steps of the oracle's "
                         f"NumPy attention (astc_kv/codec.py:253-267) on pre-decoded V, {sec*1e6:.0f} us/step on "
                         f"{cores} cores ({sec1*1e6:.0f} us/step on 1 core); the oracle's single-threaded C ASTC "
                         f"decode of the whole atlas took {decode_s*1e6:.0f} us more, not folded in",
               "us_per_step": round(sec * 1e6, 1), "us_per_step_1core": round(sec1 * 1e6, 1),
               "astc_decode_us_1core": round(decode_s * 1e6, 1)}

    achieved = nbytes["step"] / (ms_step * 1e-3) / 1e9
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
        "data": "synthetic (seeded Gaussian K/V/q), V encoded by this package's ASTC encoder",
        "config": {"workload": workload_name(a),
                   "batch": a.batch, "tokens": a.tokens, "query_heads": a.query_heads, "kv_heads": a.kv_heads,
                   "dim": a.dim, "layout": a.layout, "block": [bx, by], "tile_tokens": params.tile_tokens,
                   "splits": params.splits, "pool_sets": pool_n, "timing": mode,
                   "bytes_per_step": nbytes},
        "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": traffic["bytes"] if traffic else None,
                     "traffic_source": traffic["source"] if traffic else None,
                     "kernel": "astc_attn_kernel (split + in-kernel merge, ASTC V)",
                     "bytes_per_launch": nbytes["step"], "us_per_launch": round(ms_step * 1e3, 3)},
        "cpu_baseline": cpu,
        "resident_single_set": {"us_per_step": round(ms_resident * 1e3, 3),
                                "GB/s": round(nbytes["step"] / (ms_resident * 1e-3) / 1e9, 2)},
        "fp16_control": {"us_per_step": round(ms_fp16 * 1e3, 3), "bytes_per_step": fp16_bytes,
                         "GB/s": round(fp16_bytes / (ms_fp16 * 1e-3) / 1e9, 2), "tile_tokens": fparams.tile_tokens,
                         "astc_speedup": round(ms_fp16 / ms_step, 4)},
        "parity": {"sequences_checked": sub, "max_abs_err": max_err, "within_rtol1e-3_atol2e-3": parity},
        "setup_s": round(setup_s, 2),
    }
    text = json.dumps(line)
    print(text, flush=True)
    if a.out:
        Path(a.out).parent.mkdir(parents=True, exist_ok=True)
        Path(a.out).write_text(text + "\n")
    return 0 if parity else 1


if __name__ == "__main__":
    sys.exit(main())
