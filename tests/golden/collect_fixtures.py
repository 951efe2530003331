#!/usr/bin/env python3
"""Copy the reference's archived ASTC data fixtures into tests/golden/.

Run in a container where the reference checkout is mounted (default
/root/reference). Only data files are copied: astcenc 5.7.0 payloads
(.astc/.bin), the reference's astcenc-decoded and restored tensors
(*_decoded.f32, *.npy), fp16 metadata and queries. For the block-geometry
captures the arrays of fixed_input.npz are extracted (numpy.load with
allow_pickle=False): the captured V prefix, its fp16 token offsets/scales and
the normalised, edge-padded scalar image the reference encoded
(scripts/probe_block_geometry.py:142-155). Writes PROVENANCE.json with the
SHA256 of every source file.

Sources (relative to the reference root):
  results/kernel_v2/fixtures_page/{t384,t391}         scalar 6x6, token-normalised V
  results/metal_fixtures/story_l17_kv_page6           scalar 6x6, page_channel K and V
  results/block_geometry_v2/<cap>/{variant}.{bin,npy}  raw payloads + restored V
  results/geometry_holdout_v2/<doc>/<layer>.bin        payloads without expected values
"""
from __future__ import annotations

import argparse
import hashlib
import json
import shutil
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent

PAGE_FILES = ["manifest.json", "q.f32", "k.f16", "k_decoded.f32", "v-h000.astc", "v-h001.astc", "v-h002.astc",
              "v_decoded.f32", "v_scale.f16", "v_offset.f16"]
KV_FILES = ["manifest.json", "q.f32"] + [f"{n}-h00{h}.astc" for n in "kv" for h in range(3)] + \
           [f"{n}_{s}" for n in "kv" for s in ("decoded.f32", "scale.f16", "offset.f16")]
GEOMETRY = {"records_l17": ["identity", "transpose", "random36"],
            "science_l5": ["identity", "transpose", "random36"]}
HOLDOUT = ["bread_notes/layer0_identity", "bread_notes/layer29_transpose",
           "coastal_letter/layer15_identity", "choir_rehearsal/layer7_transpose"]


def sha(p: Path) -> str:
    return hashlib.sha256(p.read_bytes()).hexdigest()


def main():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--reference", type=Path, default=Path("/root/reference"))
    args = ap.parse_args()
    res = args.reference / "results"
    prov = {}

    def copy(src: Path, dst: Path):
        dst.parent.mkdir(parents=True, exist_ok=True)
        shutil.copyfile(src, dst)
        prov[str(dst.relative_to(HERE))] = {"source": str(src.relative_to(args.reference)), "sha256": sha(src)}

    for t in ("t384", "t391"):
        for f in PAGE_FILES:
            copy(res / "kernel_v2/fixtures_page" / t / f, HERE / t / f)
    for f in KV_FILES:
        copy(res / "metal_fixtures/story_l17_kv_page6" / f, HERE / "kv_page6" / f)
    for cap, variants in GEOMETRY.items():
        src = res / "block_geometry_v2" / cap
        for v in variants:
            copy(src / f"{v}.bin", HERE / "geometry" / f"{cap}_{v}.bin")
            copy(src / f"{v}.npy", HERE / "geometry" / f"{cap}_{v}.npy")
        with np.load(src / "fixed_input.npz", allow_pickle=False) as z:
            dst = HERE / "geometry" / f"{cap}_ranges.npz"
            np.savez(dst, fp16_offsets=z["fp16_offsets"], fp16_scales=z["fp16_scales"])
            prov[str(dst.relative_to(HERE))] = {"source": str((src / "fixed_input.npz").relative_to(args.reference)),
                                                "sha256": sha(src / "fixed_input.npz"),
                                                "extracted": ["fp16_offsets", "fp16_scales"]}
            dst = HERE / "geometry" / f"{cap}_fixed_input.npz"
            keys = ["original_v_prefix", "normalized_padded", "fp16_offsets", "fp16_scales"]
            np.savez_compressed(dst, **{k: z[k] for k in keys})
            prov[str(dst.relative_to(HERE))] = {"source": str((src / "fixed_input.npz").relative_to(args.reference)),
                                                "sha256": sha(src / "fixed_input.npz"), "extracted": keys}
    for f in HOLDOUT:
        copy(res / "geometry_holdout_v2" / f"{f}.bin", HERE / "holdout" / (f.replace("/", "_") + ".bin"))
    (HERE / "PROVENANCE.json").write_text(json.dumps(prov, indent=1, sort_keys=True) + "\n")


if __name__ == "__main__":
    main()
