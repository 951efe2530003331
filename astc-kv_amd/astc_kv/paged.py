"""Paged, ragged KV caches for the paged decode-attention kernel.

A page holds `page_tokens` tokens of every KV head: K (FP16, or 4-bit codes
in groups of 32 channels with an fp16 (offset, scale) pair per group, the
reference's affine_quantize(axis="token", group=32), astc_kv/codec.py:218-250)
and V as ASTC blocks with per-token fp16 scale/offset (the atlas of
astc_kv.atlas, cut into pages). Each sequence owns a row of a block table
listing its pages; pages are scattered through the pool. With `tail=True`
the tokens past a sequence's last full page keep exact FP16 V in a per-sequence
tail page (the fresh tail the reference plans, docs/representation_v0.1.md:84-95),
their K in an ordinary page. The layouts are those of
akv_hip_paged_decode_attention (include/astc_kv_hip.h).
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import codec
from .atlas import build_atlas, texel_columns


@dataclass
class PagedKV:
    k_pages: np.ndarray            # fp16 [NP, Hkv, P, D] or uint8 codes [NP, Hkv, P, D/2]
    k_meta: np.ndarray | None      # fp16 [NP, Hkv, P, D/32, 2]: (offset, scale) per 32 channels
    v_blocks: np.ndarray           # uint8 [NP, Hkv, P/by, cols, 16]
    v_scale: np.ndarray            # fp16 [NP, Hkv, P]
    v_offset: np.ndarray           # fp16 [NP, Hkv, P]
    block_table: np.ndarray        # int32 [B, max_pages]
    seq_lens: np.ndarray           # int32 [B]
    v_tail: np.ndarray | None      # fp16 [B, Hkv, P, D]
    dim: int
    layout: str
    block_x: int
    block_y: int
    page_tokens: int
    k_format: str                  # "fp16" or "u4g32"

    @property
    def batch(self) -> int:
        return int(self.seq_lens.shape[0])

    @property
    def kv_heads(self) -> int:
        return int(self.k_pages.shape[1])

    @property
    def cols(self) -> int:
        return int(self.v_blocks.shape[3])

    def full_tokens(self, i: int) -> int:
        """Tokens of sequence i whose V is ASTC-encoded (the rest is the tail)."""
        n = int(self.seq_lens[i])
        return n - n % self.page_tokens if self.v_tail is not None else n

    def byte_counts(self) -> dict:
        """Logical bytes a decode step reads: K (codes + metadata), the V blocks
        of the encoded tokens' block rows, V scale/offset, and the FP16 tail."""
        d, p, by = self.dim, self.page_tokens, self.block_y
        kb = vb = meta = tail = 0
        for i, n in enumerate(self.seq_lens.tolist()):
            full = self.full_tokens(i)
            kb += self.kv_heads * n * (d * 2 if self.k_format == "fp16" else d // 2 + (d // 32) * 4)
            vb += self.kv_heads * -(-full // by) * self.cols * 16
            meta += self.kv_heads * full * 4
            tail += self.kv_heads * (n - full) * d * 2
        return {"k": kb, "v_blocks": vb, "v_meta": meta, "v_tail": tail, "total": kb + vb + meta + tail}


def build_paged(k_seqs, v_seqs, layout: str = "scalar", block=(6, 6), page_tokens: int = 96,
                quality: float = 50, k_format: str = "fp16", tail: bool = True, seed: int = 0,
                threads: int | None = None, progress=None, reserve_tokens: int = 0) -> PagedKV:
    """k_seqs, v_seqs: per sequence [Hkv, T_i, D] (K fp16 or float, V float).
    Pages are assigned in a seeded random order; each sequence gets pages for
    T_i + reserve_tokens tokens (the ones past T_i empty, for appends).
    progress(i, n), if given, is called after each sequence."""
    bx, by = codec._footprint(block)
    if page_tokens % 16 or page_tokens % by:
        raise ValueError("page_tokens must be a multiple of 16 and of the block height")
    if k_format not in ("fp16", "u4g32"):
        raise ValueError("k_format must be 'fp16' or 'u4g32'")
    if len(k_seqs) != len(v_seqs) or not k_seqs:
        raise ValueError("need matching, non-empty K and V sequence lists")
    h, _, d = np.shape(v_seqs[0])
    if k_format == "u4g32" and d % 32:
        raise ValueError("4-bit K needs a multiple of 32 channels")
    P = page_tokens
    lens = [int(np.shape(v)[1]) for v in v_seqs]
    if min(lens) < 1:
        raise ValueError("empty sequence")
    if reserve_tokens < 0:
        raise ValueError("reserve_tokens must be >= 0")
    pages = [-(-(t + reserve_tokens) // P) for t in lens]
    total = sum(pages)
    perm = np.random.default_rng(seed).permutation(total).astype(np.int32)
    rpp = P // by
    cols = -(-texel_columns(d, layout) // bx)
    if k_format == "fp16":
        k_pages = np.zeros((total, h, P, d), np.float16)
        k_meta = None
    else:
        k_pages = np.zeros((total, h, P, d // 2), np.uint8)
        k_meta = np.zeros((total, h, P, d // 32, 2), np.float16)
    v_blocks = np.zeros((total, h, rpp, cols, 16), np.uint8)
    v_scale = np.zeros((total, h, P), np.float16)
    v_offset = np.zeros((total, h, P), np.float16)
    table = np.zeros((len(lens), max(pages)), np.int32)
    v_tail = np.zeros((len(lens), h, P, d), np.float16) if tail else None
    first = 0
    for i, (k, v, t) in enumerate(zip(k_seqs, v_seqs, lens)):
        k = np.asarray(k)
        v = np.asarray(v, np.float32)
        if k.shape != (h, t, d) or v.shape != (h, t, d):
            raise ValueError(f"sequence {i}: K and V must both be [Hkv, T, D]")
        ids = perm[first:first + pages[i]]
        first += pages[i]
        table[i, :pages[i]] = ids
        # K pages (the last one zero-padded).
        if k_format == "fp16":
            kk = k.astype(np.float16)
        else:
            _, _, _, packed, off, sc = codec.affine_quantize_codes(k.astype(np.float32), 4, "token", 32)
            kk = packed.reshape(h, t, d // 2)
            meta = np.concatenate([off, sc], axis=-1).astype(np.float16)     # [h, t, d/32, 2]
        for j, pid in enumerate(ids[:-(-t // P)]):
            n = min(P, t - j * P)
            k_pages[pid, :, :n] = kk[:, j * P:j * P + n]
            if k_meta is not None:
                k_meta[pid, :, :n] = meta[:, j * P:j * P + n]
        # V: encoded pages; with a tail, the partial last page stays FP16.
        full = t - t % P if tail else t
        if tail and full < t:
            v_tail[i, :, :t - full] = v[:, full:].astype(np.float16)
        if full:
            enc = -(-full // P) * P
            vv = np.pad(v[:, :full], ((0, 0), (0, enc - full), (0, 0)), mode="edge")
            at = build_atlas(vv[None], layout, (bx, by), P, quality, threads)
            for j in range(enc // P):
                pid = ids[j]
                v_blocks[pid] = at.blocks[0, :, j * rpp:(j + 1) * rpp]
                v_scale[pid] = at.scale[0, :, j * P:(j + 1) * P]
                v_offset[pid] = at.offset[0, :, j * P:(j + 1) * P]
        if progress is not None:
            progress(i + 1, len(lens))
    return PagedKV(k_pages, k_meta, v_blocks, v_scale, v_offset, table, np.asarray(lens, np.int32), v_tail, d,
                   layout, bx, by, P, k_format)
