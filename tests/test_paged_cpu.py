"""Paged, ragged cache builder (astc_kv.paged): every token of every sequence
lands in the page its block-table row names, K as given (FP16) or as the 4-bit
codes and fp16 (offset, scale) pairs of affine_quantize(axis="token", group=32)
(astc_kv/codec.py:218-250), V blocks identical to the contiguous atlas of the
same sequence, and the FP16 tail. CPU only."""
import numpy as np
import pytest

from astc_kv import codec
from astc_kv.atlas import build_atlas
from astc_kv.paged import build_paged


def _seqs(rng, lens, h=2, d=64):
    k = [rng.normal(size=(h, t, d)).astype(np.float16) for t in lens]
    v = [rng.normal(0, 0.5, size=(h, t, d)).astype(np.float32) for t in lens]
    return k, v


@pytest.mark.parametrize("k_format,tail", [("fp16", True), ("u4g32", False)])
def test_pages_hold_each_sequence(k_format, tail):
    rng = np.random.default_rng(3)
    lens = [100, 96, 250, 17]
    k, v = _seqs(rng, lens)
    P = 48
    pk = build_paged(k, v, "rgba", (4, 4), P, quality=10, k_format=k_format, tail=tail, seed=9)
    used = np.concatenate([pk.block_table[i, :-(-t // P)] for i, t in enumerate(lens)])
    assert sorted(used.tolist()) == list(range(pk.k_pages.shape[0]))          # each page once
    for i, t in enumerate(lens):
        ids = pk.block_table[i, :-(-t // P)]
        if k_format == "fp16":
            got = pk.k_pages[ids].transpose(1, 0, 2, 3).reshape(2, -1, 64)[:, :t]
            assert np.array_equal(got, k[i])
        else:
            _, _, codes, packed, off, sc = codec.affine_quantize_codes(k[i].astype(np.float32), 4, "token", 32)
            got = pk.k_pages[ids].transpose(1, 0, 2, 3).reshape(2, -1, 32)[:, :t]
            assert np.array_equal(got, packed.reshape(2, t, 32))
            lo, hi = got & 15, got >> 4                                          # low nibble = even channel
            unpacked = np.stack([lo, hi], -1).reshape(2, t, 64)
            assert np.array_equal(unpacked, codes.reshape(2, t, 64))
            meta = pk.k_meta[ids].transpose(1, 0, 2, 3, 4).reshape(2, -1, 2, 2)[:, :t]
            assert np.array_equal(meta[..., 0], off[..., 0]) and np.array_equal(meta[..., 1], sc[..., 0])
        full = pk.full_tokens(i)
        assert full == (t - t % P if tail else t)
        if full:
            at = build_atlas(np.pad(v[i][:, :full], ((0, 0), (0, -(-full // P) * P - full), (0, 0)), mode="edge")[None],
                             "rgba", (4, 4), P, 10)
            rows = -(-full // P) * (P // 4)
            got_b = pk.v_blocks[ids[:-(-full // P)]].transpose(1, 0, 2, 3, 4).reshape(2, -1, 4, 16)[:, :rows]
            assert np.array_equal(got_b, at.blocks[0])
            got_s = pk.v_scale[ids[:-(-full // P)]].transpose(1, 0, 2).reshape(2, -1)[:, :full]
            assert np.array_equal(got_s, at.scale[0, :, :full])
        if tail and full < t:
            assert np.array_equal(pk.v_tail[i, :, :t - full], v[i][:, full:].astype(np.float16))
    counts = pk.byte_counts()
    assert counts["total"] == counts["k"] + counts["v_blocks"] + counts["v_meta"] + counts["v_tail"]


def test_rejects_bad_pages():
    rng = np.random.default_rng(0)
    k, v = _seqs(rng, [40])
    with pytest.raises(ValueError):
        build_paged(k, v, "rgba", (6, 5), 40)          # not a multiple of 16
    with pytest.raises(ValueError):
        build_paged(k, v, "rgba", (6, 5), 48)          # not a multiple of the block height


@pytest.mark.parametrize("layout,block", [("rgba", (6, 5)), ("scalar", (6, 6))])
def test_pagewise_encoding_equals_whole_sequence(layout, block):
    # The append path encodes each completed page on its own (from the FP16
    # tail) and copies the blocks into the pool; that equals encoding the whole
    # sequence because a page is whole block rows and normalization is per token.
    rng = np.random.default_rng(5)
    P = 120 if block == (6, 5) else 96
    v = rng.normal(0, 0.5, size=(2, 3 * P, 64)).astype(np.float16).astype(np.float32)
    whole = build_atlas(v[None], layout, block, P, 20)
    pages = build_atlas(v.reshape(2, 3, P, 64).transpose(1, 0, 2, 3), layout, block, P, 20)
    rpp = P // block[1]
    for j in range(3):
        assert np.array_equal(pages.blocks[j], whole.blocks[0, :, j * rpp:(j + 1) * rpp])
        assert np.array_equal(pages.scale[j], whole.scale[0, :, j * P:(j + 1) * P])
        assert np.array_equal(pages.offset[j], whole.offset[0, :, j * P:(j + 1) * P])


def test_reserved_pages_for_appends():
    rng = np.random.default_rng(2)
    lens = [50, 96, 97]
    k, v = _seqs(rng, lens)
    P = 48
    pk = build_paged(k, v, "rgba", (4, 4), P, quality=10, tail=True, seed=1, reserve_tokens=60)
    pages = [-(-(t + 60) // P) for t in lens]
    assert pk.block_table.shape == (3, max(pages)) and pk.k_pages.shape[0] == sum(pages)
    used = np.concatenate([pk.block_table[i, :n] for i, n in enumerate(pages)])
    assert sorted(used.tolist()) == list(range(sum(pages)))
    for i, t in enumerate(lens):                       # reserved pages stay empty
        empty = pk.block_table[i, -(-t // P):pages[i]]
        assert not pk.k_pages[empty].any() and not pk.v_blocks[empty].any()
    with pytest.raises(ValueError):
        build_paged(k, v, "rgba", (4, 4), P, reserve_tokens=-1)
