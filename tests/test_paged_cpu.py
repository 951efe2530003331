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
