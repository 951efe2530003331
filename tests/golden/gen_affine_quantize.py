#!/usr/bin/env python3
"""Write golden vectors of the reference's affine_quantize (astc_kv/codec.py:218-250).

Run in a container where the reference checkout is mounted (default
/root/reference): it imports the reference module astc_kv.codec there (which
needs only NumPy at import time; nothing else of the reference runs) and
records, for seeded inputs, the float32 reconstruction and byte counts that
affine_quantize returns. The GPU box never runs this; the tests read the
committed affine_quantize.npz.

Inputs (all float32, [H, T, D]):
  heavy   Student-t (3 dof) values, the heavy-tailed K of the c4/c5 workloads;
  ties    groups whose range makes the scale exactly 1 or 1/2 and whose values
          sit on half steps, so that (x - o) / s lands exactly halfway between
          two codes (np.rint rounds half to even; a round-half-up quantiser
          gives other codes);
  flat    constant groups (scale floored at 2^-24) and groups spanning signs
          and fp16 magnitudes up to 6e4.
Configurations: 4-bit token groups of 32 (the paged K format), 2-bit token
groups of 64, 8-bit token groups of 64, 4-bit channel groups of 32, 8-bit
channel groups of 96 (scripts/evaluate_hybrid.py:48).
"""
from __future__ import annotations

import argparse
import hashlib
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
CONFIGS = [(4, "token", 32), (2, "token", 64), (8, "token", 64), (4, "channel", 32), (8, "channel", 96)]


def inputs():
    rng = np.random.default_rng(20261202)
    heavy = rng.standard_t(3, size=(2, 96, 128)).astype(np.float32)
    # Half-step ties: within each group of 32 channels, min 0 and max 15 (scale
    # 15/15 = 1) or max 7.5 (scale 0.5), values k + 1/2 steps in between.
    ties = np.empty((2, 96, 128), np.float32)
    for h in range(2):
        for t in range(96):
            for g in range(4):
                step = 1.0 if (t + g) % 2 == 0 else 0.5
                v = (rng.integers(0, 15, 32) + 0.5) * step
                v[0], v[1] = 0.0, 15 * step
                ties[h, t, 32 * g:32 * g + 32] = rng.permutation(v)
    flat = np.clip(rng.normal(size=(2, 96, 128)) * 1.5e4, -6e4, 6e4).astype(np.float32)
    flat[:, ::3] = np.float32(1.25)                     # constant rows: every group flat
    flat[1, 1::3, :64] = -np.abs(flat[1, 1::3, :64])    # negative groups
    return {"heavy": heavy, "ties": ties, "flat": flat}


def main():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--reference", type=Path, default=Path("/root/reference"))
    args = ap.parse_args()
    sys.path.insert(0, str(args.reference))
    from astc_kv import codec as ref   # the reference module itself

    src = args.reference / "astc_kv" / "codec.py"
    arrays, meta = {}, {"source": "astc_kv/codec.py", "sha256": hashlib.sha256(src.read_bytes()).hexdigest(),
                        "function": "affine_quantize", "cases": []}
    for name, x in inputs().items():
        arrays[f"{name}__x"] = x
        for bits, axis, group in CONFIGS:
            dec, counts = ref.affine_quantize(x, bits, axis, group)
            key = f"{name}__{bits}_{axis}_{group}"
            arrays[key] = np.asarray(dec, np.float32)
            meta["cases"].append({"input": name, "bits": bits, "axis": axis, "group": group, "key": key,
                                  "counts": {k: int(v) for k, v in counts.items()}})
    np.savez_compressed(HERE / "affine_quantize.npz", **arrays)
    (HERE / "affine_quantize.json").write_text(json.dumps(meta, indent=1) + "\n")
    print(f"wrote {len(meta['cases'])} cases")


if __name__ == "__main__":
    main()
