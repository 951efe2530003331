"""ORACLE — test infrastructure only (tests/, __graft_entry__.smoke(), bench.py's
parity check and CPU-baseline leg). Never imported by the product package.

Host reconstruction of one sequence of a paged KV cache, read back through the
pages its block-table row names: FP16 K, or 4-bit group-32 K restored as
code * scale + zero in float32 (astc_kv/codec.py:248, the reference's
affine dequantisation), and V restored from the oracle's decode of the page
blocks (oracle/astc_oracle.c) as u * scale + offset in float32
(astc_kv/codec.py:206), followed by the sequence's FP16 tail.
"""
from __future__ import annotations

import numpy as np

from oracle import astc_oracle as O
from oracle import attention_ref as R


def host_kv(pk, i):
    """K and V of sequence i of a PagedKV as float32 [Hkv, T, D]."""
    t, P, h, d = int(pk.seq_lens[i]), pk.page_tokens, pk.kv_heads, pk.dim
    ids = pk.block_table[i, :-(-t // P)]
    if pk.k_format == "fp16":
        k = pk.k_pages[ids].transpose(1, 0, 2, 3).reshape(h, -1, d)[:, :t].astype(np.float32)
    else:
        b = pk.k_pages[ids].transpose(1, 0, 2, 3).reshape(h, -1, d // 2)[:, :t]
        codes = np.stack([b & 15, b >> 4], -1).reshape(h, t, d // 32, 32).astype(np.float32)
        meta = pk.k_meta[ids].transpose(1, 0, 2, 3, 4).reshape(h, -1, d // 32, 2)[:, :t].astype(np.float32)
        k = (codes * meta[..., 1:2] + meta[..., 0:1]).reshape(h, t, d)
    full = pk.full_tokens(i)
    parts = []
    if full:
        npg = -(-full // P)
        rpp, cols, bx, by = P // pk.block_y, pk.cols, pk.block_x, pk.block_y
        blocks = pk.v_blocks[ids[:npg]].transpose(1, 0, 2, 3, 4).reshape(h, npg * rpp, cols, 16)
        tex, _ = O.decode_blocks_fp16(np.ascontiguousarray(blocks).reshape(-1, 16), bx, by)
        img = tex.reshape(h, npg * rpp, cols, by, bx, 4).transpose(0, 1, 3, 2, 4, 5)
        img = img.reshape(h, npg * P, cols * bx, 4)[:, :full].astype(np.float32)
        u = img[..., :d, 0] if pk.layout == "scalar" else img[:, :, : d // 4].reshape(h, full, d)
        s = pk.v_scale[ids[:npg]].transpose(1, 0, 2).reshape(h, -1)[:, :full].astype(np.float32)
        o = pk.v_offset[ids[:npg]].transpose(1, 0, 2).reshape(h, -1)[:, :full].astype(np.float32)
        parts.append(R.restore_token(u, s[..., None], o[..., None]))
    if full < t:
        parts.append(pk.v_tail[i, :, : t - full].astype(np.float32))
    return k, np.concatenate(parts, axis=1)
