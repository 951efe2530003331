#!/usr/bin/env python3
"""Scores this package's ASTC encoder against astcenc 5.7.0 on the inputs the
reference ships, and writes tests/golden/encoder_quality.json.

The reference's block-geometry study (scripts/probe_block_geometry.py:129-210)
saved, for 24 (capture, layer) pairs, the token-normalised, edge-padded V
prefix it encoded (results/block_geometry_v2/<pair>/fixed_input.npz:
normalized_padded [3, 288, 66], original_v_prefix, fp16 offsets/scales) and
recorded astcenc's errors for the unpermuted layout (rows.jsonl, variant
"identity"): `normalized_padded_error_sse`, the squared error of the decoded
normalized image (6x6 blocks, quality 98, scalar value in R, G and B with
alpha 1), and `tensor_error_sse`, the squared error of the restored V
(decoded * scale + offset, then the padding dropped) against the original.
This script encodes the same images the same way with akv_encode at quality
98 and at the encoder's other presets, decodes them with akv_decode, and
computes both errors with the same formulas. It reads /root/reference, so it
runs in the build container only; the JSON it writes is the record.
"""
from __future__ import annotations

import json
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT / "astc-kv_amd"))
REF = Path("/root/reference/results/block_geometry_v2")


def sse(a) -> float:
    return float(np.sum(np.square(a, dtype=np.float64)))


def main() -> int:
    from astc_kv.codec import AstcEncoder
    rows = {(r["capture"], r["layer"]): r for r in map(json.loads, open(REF / "rows.jsonl"))
            if r["variant"] == "identity"}
    qualities = (98.0, 60.0, 10.0)
    encoders = {q: AstcEncoder((6, 6), q) for q in qualities}
    out = []
    for (cap, layer), r in sorted(rows.items()):
        z = np.load(REF / f"{cap}_l{layer}" / "fixed_input.npz", allow_pickle=False)
        scalar, x = z["normalized_padded"].astype(np.float32), z["original_v_prefix"].astype(np.float32)
        off, scale = z["fp16_offsets"].astype(np.float32), z["fp16_scales"].astype(np.float32)
        dim = x.shape[2]
        rec = {"capture": cap, "layer": layer, "astcenc_q98": {
            "normalized_padded_error_sse": r["normalized_padded_error_sse"],
            "tensor_error_sse": r["tensor_error_sse"], "tensor_reference_sse": r["tensor_reference_sse"]}}
        for q, enc in encoders.items():
            t0 = time.perf_counter()
            dec = []
            for img in scalar:
                image = np.ones(img.shape + (4,), np.float32)
                image[..., :3] = img[..., None]
                _, back, _ = enc.roundtrip(image)
                dec.append(back[..., 0])
            dec = np.stack(dec).astype(np.float64)
            restored = (dec[:, :, :dim].astype(np.float32) * scale + off).astype(np.float64)
            rec[f"this_q{q:g}"] = {"normalized_padded_error_sse": sse(dec - scalar),
                                   "tensor_error_sse": sse(restored - x), "encode_s": time.perf_counter() - t0}
        out.append(rec)
        a, b = rec["astcenc_q98"]["normalized_padded_error_sse"], rec["this_q98"]["normalized_padded_error_sse"]
        print(f"{cap} l{layer}: astcenc q98 {a:.2f}, this q98 {b:.2f} ({b / a:.2f}x)", flush=True)
    for enc in encoders.values():
        enc.close()
    summary = {}
    for key in ["astcenc_q98"] + [f"this_q{q:g}" for q in qualities]:
        summary[key] = {f: float(sum(rec[key][f] for rec in out)) for f in ("normalized_padded_error_sse",
                                                                             "tensor_error_sse")}
    result = {"source": "results/block_geometry_v2 (rows.jsonl identity rows; <pair>/fixed_input.npz)",
              "block": [6, 6], "layout": "scalar value in RGB, alpha 1", "pairs": out, "totals": summary}
    (Path(__file__).with_name("encoder_quality.json")).write_text(json.dumps(result, indent=1) + "\n")
    for k, v in summary.items():
        print(k, {f: round(x, 2) for f, x in v.items()})
    return 0


if __name__ == "__main__":
    sys.exit(main())
