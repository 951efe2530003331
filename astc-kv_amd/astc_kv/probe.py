"""Decode-attention probe over an `astc-kv-probe-v1` fixture, with the
reference's correctness gates run before anything is timed.

The reference's Metal host (metal/probe_gqa_v10.mm) reads a fixture manifest
(docs/metal_path.md:54-73), runs its kernels once, compares them with host
references and refuses to publish timings when a gate fails: it prints
{"status": "correctness_failed", "raw_samples": []} and exits non-zero
(probe_gqa_v10.mm:704-784). scripts/verify_metal_v4.py:24-45 checks that
refusal with three derived controls: a wrong offline decode (one value
+1000), a non-finite one and a missing one. This is the same protocol over
the HIP path:

* v_decode_gate  V restored from the GPU decode (akv_hip_decode_values, then
                 fl32(fl32(u * scale) + offset)) against the fixture's offline
                 decode (`v_decoded_file`): every value finite and within
                 scale/1024 + 8 ulp of float32 of it (probe_gqa_v10.mm:757-779);
                 `bit_exact` records whether they are identical. A compressed V
                 without an offline decode fails ("Missing offline decode
                 reference", :745-749).
* k_decode_gate  FP16 K against `k_decoded_file` when present: identical values.
* astc_decode_attention / fp16_control  the GPU step (one launch, merge in the
                 split kernel) and the FP16-K/V control against FP64 host
                 accumulation over the same values: finite, relative L2 <= 1e-4
                 (:719-725).

Only then are `rounds` x `iterations` steps timed with HIP events.
`python -m astc_kv.probe MANIFEST [--tile T] [--tokens T] [--rounds R] [--iterations N]`
prints one JSON object; the exit status is 0, 1 for a refusal and 2 for a
fixture this path does not run (the reference's v10 probe takes FP16 K and
token-normalised ASTC V only, :460-461).
"""
from __future__ import annotations

import argparse
import json
import sys
from pathlib import Path

import numpy as np

SCHEMA_OK = "astc-kv-hip-probe-v1"
SCHEMA_FAIL = "astc-kv-hip-probe-failure-v1"
REL_L2_GATE = 1e-4


class UnsupportedFixture(ValueError):
    pass


def load_fixture(manifest: Path) -> dict:
    """Arrays of an astc-kv-probe-v1 fixture (FP16 K, token-normalised ASTC V)."""
    from .atlas import atlas_from_manifest
    manifest = Path(manifest)
    d = manifest.parent
    m = json.loads(manifest.read_text())
    if m.get("format") != "astc-kv-probe-v1" or m.get("metadata_dtype") != "float16_le":
        raise UnsupportedFixture("expected an astc-kv-probe-v1 manifest with float16_le metadata")
    if m.get("k_storage") != "fp16" or m.get("v_storage") != "astc" or m.get("v_normalization") != "token":
        raise UnsupportedFixture("this probe runs FP16 K with token-normalised ASTC V")
    t, hq, hkv, dim = m["tokens"], m["query_heads"], m["kv_heads"], m["head_dim"]
    atlas, _ = atlas_from_manifest(d)
    fx = {"manifest": m, "atlas": atlas,
          "q": np.fromfile(d / m["query_file"], "<f4").reshape(1, hq, dim),
          "k": np.fromfile(d / m["k_file"], "<f2").reshape(1, hkv, t, dim),
          "v_decoded": None, "k_decoded": None}
    for side in ("v", "k"):
        name = m.get(f"{side}_decoded_file")
        if name:
            fx[f"{side}_decoded"] = np.fromfile(d / name, "<f4").reshape(1, hkv, t, dim)
    return fx


def repeat_tokens(fx: dict, tokens: int) -> dict:
    """The fixture repeated along the sequence to `tokens` keys, as the
    reference builds its traffic controls (scripts/make_traffic_fixture.py:
    12-49): token i of K, its offline decode, V's offline decode and V's
    scale/offset is source token i mod T; ASTC block row r is source row
    r mod (T / block height), for as many rows as `tokens` rounded up to whole
    pages; the query is unchanged. Bounded to 1..8192 tokens like the
    reference's. Timing on such a fixture measures shape and traffic only."""
    from .atlas import Atlas
    if not 1 <= tokens <= 8192:
        raise ValueError("repeated fixtures are bounded to 1..8192 tokens")
    a = fx["atlas"]
    t = a.tokens
    if t % a.block_y or a.rows != t // a.block_y:
        raise ValueError("the source fixture must hold whole block rows of its tokens")
    idx = np.arange(tokens) % t
    padded = -(-tokens // a.page_tokens) * a.page_tokens
    rows = np.arange(-(-padded // a.block_y)) % a.rows
    atlas = Atlas(np.ascontiguousarray(a.blocks[:, :, rows]), np.ascontiguousarray(a.scale[..., idx]),
                  np.ascontiguousarray(a.offset[..., idx]), tokens, a.dim, a.layout, a.block_x, a.block_y,
                  a.page_tokens)
    out = dict(fx, atlas=atlas, k=np.ascontiguousarray(fx["k"][:, :, idx]),
               manifest=dict(fx["manifest"], tokens=tokens, source_tokens=t))
    for side in ("v_decoded", "k_decoded"):
        if fx[side] is not None:
            out[side] = np.ascontiguousarray(fx[side][:, :, idx])
    return out


def attention_fp64(q, k, v):
    """One query token per head, every key visible, FP64 accumulation (the
    reference probe's host reference, probe_gqa_v10.mm:345-369). q [Hq, D],
    k, v [Hkv, T, D] -> [Hq, D]."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    hq, d = q.shape
    g = hq // k.shape[0]
    out = np.empty((hq, d))
    for h in range(hq):
        s = k[h // g] @ q[h] / np.sqrt(d)
        w = np.exp(s - s.max())
        out[h] = (w / w.sum()) @ v[h // g]
    return out


def _errors(reference, estimate) -> dict:
    a = np.asarray(reference, np.float64)
    b = np.asarray(estimate, np.float64)
    finite = bool(np.isfinite(b).all() and np.isfinite(a).all())
    if not finite:
        return {"finite": False}
    diff = b - a
    return {"finite": True, "max_abs": float(np.max(np.abs(diff))),
            "relative_l2": float(np.linalg.norm(diff) / max(np.linalg.norm(a), 1e-30)),
            "rmse": float(np.sqrt(np.mean(diff * diff)))}


def gates(fx: dict, v_restored: np.ndarray, out_astc: np.ndarray, out_fp16: np.ndarray | None) -> tuple[bool, dict]:
    """The correctness gates over the GPU results (V restored from the GPU
    decode, the ASTC step's output, the FP16 control's output), all float32
    [1, ...] arrays. Returns (passed, correctness record)."""
    atlas = fx["atlas"]
    c, passed = {}, True
    sw = fx["v_decoded"]
    if sw is None:
        c["v_decode_gate"] = {"passed": False, "reason": "Missing offline decode reference"}
        passed = False
    else:
        hw = np.asarray(v_restored, np.float32)
        e = _errors(sw, hw)
        c["v_gpu_vs_offline_decode"] = e
        scale = atlas.scale.astype(np.float64)[..., None]
        good = e["finite"] and bool(np.all(np.isfinite(scale)) and np.all(scale > 0))
        if good:
            roundoff = 8 * np.finfo(np.float32).eps * np.maximum(1.0, np.maximum(np.abs(hw), np.abs(sw)))
            good = bool(np.all(np.abs(hw.astype(np.float64) - sw) <= scale / 1024.0 + roundoff))
        c["v_decode_gate"] = {"passed": good, "criterion": "abs_delta <= scale/1024 + FP32_roundoff",
                              "bit_exact": bool(np.array_equal(hw.view(np.uint32), sw.view(np.uint32)))}
        passed = passed and good
    if fx["k_decoded"] is not None:
        e = _errors(fx["k_decoded"], fx["k"].astype(np.float32))
        good = e["finite"] and e["max_abs"] == 0.0
        c["k_fp16_vs_offline_values"] = e
        c["k_decode_gate"] = {"passed": good, "criterion": "exact FP16 values"}
        passed = passed and good
    q, k = fx["q"][0], fx["k"][0].astype(np.float64)
    for name, out, v in (("astc_decode_attention", out_astc, v_restored),
                         ("fp16_control", out_fp16, None if out_fp16 is None else
                          np.asarray(v_restored, np.float32).astype(np.float16))):
        if out is None:
            continue
        ref = attention_fp64(q, k, np.asarray(v, np.float64)[0])
        e = _errors(ref, np.asarray(out)[0])
        good = e["finite"] and e["relative_l2"] <= REL_L2_GATE
        c[name] = {"vs_same_values_cpu_fp64_accumulation": e, "passed_rtol_l2_1e_4": good}
        passed = passed and good
    return passed, c


def refusal(correctness: dict) -> dict:
    return {"schema": SCHEMA_FAIL, "status": "correctness_failed", "correctness": correctness, "raw_samples": []}


def run(manifest: Path, tile: int | None = None, rounds: int = 5, iterations: int = 20,
        tokens: int | None = None) -> tuple[int, dict]:
    """Gates, then timing; `tokens` repeats the fixture to that many keys
    first (repeat_tokens). Returns (exit status, JSON record)."""
    import torch

    from . import gpu
    try:
        fx = load_fixture(manifest)
    except UnsupportedFixture as e:
        return 2, {"schema": SCHEMA_FAIL, "status": "unsupported_fixture", "error": str(e), "raw_samples": []}
    if tokens:
        fx = repeat_tokens(fx, tokens)
    atlas = gpu.DeviceAtlas.from_host(fx["atlas"])
    qt = torch.from_numpy(fx["q"]).cuda()
    kt = torch.from_numpy(fx["k"]).cuda()
    hq = qt.shape[1]
    params = gpu.make_params(atlas, hq, tile)
    u = gpu.decode_values(atlas, params.tile_tokens)
    v_restored = (u.float() * atlas.scale.float()[..., None]) + atlas.offset.float()[..., None]
    out = gpu.decode_attention(qt, kt, atlas, params=params)
    out16 = gpu.fp16_attention(qt, kt, v_restored.half(), fused=False)
    torch.cuda.synchronize()
    passed, correctness = gates(fx, v_restored.cpu().numpy(), out.cpu().numpy(), out16.cpu().numpy())
    if not passed:
        return 1, refusal(correctness)
    s = params.splits
    partial = torch.empty((1, hq, s, fx["q"].shape[2]), dtype=torch.float32, device="cuda")
    stats = torch.empty((1, hq, s, 2), dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream()
    samples = []
    for _ in range(rounds):
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record(stream)
        for _ in range(iterations):
            gpu.decode_attention(qt, kt, atlas, params=params, partial=partial, stats=stats, out=out)
        t1.record(stream)
        t1.synchronize()
        samples.append(t0.elapsed_time(t1) * 1e3 / iterations)
    return 0, {"schema": SCHEMA_OK, "status": "ok", "correctness": correctness, "tokens": fx["atlas"].tokens,
               "tile_tokens": params.tile_tokens,
               "splits": params.splits, "raw_samples": samples, "median_us": float(np.median(samples)),
               "unit": "us per decode-attention step (one launch)"}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("manifest", type=Path)
    ap.add_argument("--tile", type=int, default=None, help="tokens per split (any positive count)")
    ap.add_argument("--rounds", type=int, default=5)
    ap.add_argument("--iterations", type=int, default=20)
    ap.add_argument("--tokens", type=int, default=None,
                    help="repeat the fixture's blocks to this many keys (1..8192) before running")
    a = ap.parse_args(argv)
    rc, record = run(a.manifest, a.tile, a.rounds, a.iterations, a.tokens)
    print(json.dumps(record, indent=1))
    if rc == 1:
        print("astc-kv probe: attention correctness gate failed; no timing result is published", file=sys.stderr)
    return rc


if __name__ == "__main__":
    sys.exit(main())
