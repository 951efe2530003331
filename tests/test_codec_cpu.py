"""CPU tests of the drop-in Python API (astc_kv.codec), the product CPU codec
(libakv_astc.so) against the oracle, and the atlas / host planning helpers.

The first group restates the reference's own numeric tests
(tests/test_numeric.py:17-74) against this package's codec.py: the transforms
with the lossy codec replaced by an identity round trip, payload and metadata
byte accounting, the incomplete-page rule, fp16 metadata bounds, GQA attention
against a scalar FP64 loop, a constant image through the real codec, and the
quantiser's byte counts."""
import ctypes as ct
from unittest.mock import patch

import numpy as np
import pytest

from astc_kv import codec
from astc_kv.atlas import Atlas, build_atlas, texel_columns
from oracle import astc_oracle as O
from oracle import attention_ref as R


class IdentityAstc:
    """Stand-in for AstcEncoder whose round trip is lossless (square blocks)."""

    def __init__(self, block, *args):
        self.block = block

    def close(self):
        pass

    def roundtrip(self, im):
        h, w, _ = im.shape
        b = self.block[0] if isinstance(self.block, tuple) else self.block
        return bytes(-(-h // b) * -(-w // b) * 16), im.copy(), 0.0


def test_transforms_and_permutation_inverses():
    x = np.random.default_rng(42).normal(size=(3, 288, 64)).astype("f4")
    configs = [{"layout": "scalar", "block": b, "normalization": "page_channel"} for b in (4, 6, 8)]
    configs += [{"layout": "rgba", "block": 4, "normalization": "page_channel"},
                {"layout": "scalar", "block": 6, "normalization": "token"},
                {"layout": "scalar", "block": 6, "normalization": "block_min", "profile": "hdr"}]
    configs += [dict(layout="scalar", block=6, normalization="page_channel", permutation=p)
                for p in ("tokens_within_page", "channels")]
    with patch("astc_kv.codec.AstcEncoder", IdentityAstc):
        for cfg in configs:
            y = codec.encode_tensor(x, cfg)
            np.testing.assert_allclose(y.decoded, x, rtol=2e-6, atol=2e-6, err_msg=str(cfg))


def test_payload_and_metadata_padding():
    with patch("astc_kv.codec.AstcEncoder", IdentityAstc):
        x = np.zeros((3, 288, 64), np.float32)
        p = codec.encode_tensor(x, dict(layout="scalar", block=6, normalization="page_channel"))
        assert p.width == 66
        assert p.byte_counts["astc_blocks_including_edge_padding"] == 3 * 48 * 11 * 16
        assert p.logical_bytes == 3 * 288 * 64 * 4 // 8
        assert len(p.astc_file(0)) == 16 + 48 * 11 * 16
        t = codec.encode_tensor(x, dict(layout="scalar", block=6, normalization="token"))
        assert t.bits_per_scalar == pytest.approx(4 + 1 / 6)


def test_no_future_in_incomplete_page():
    with pytest.raises(ValueError):
        codec.encode_tensor(np.zeros((1, 97, 64), "f4"), dict(layout="scalar", block=6, normalization="token"))


def test_metadata_bounds():
    x = np.concatenate([np.linspace(-500, 500, 10001), [0, 2 ** -27, -2 ** -27, 1.0004]]).astype("f4")
    assert np.all(codec.fp16_floor(x).astype("f4") <= x)
    assert np.all(codec.fp16_ceil(x).astype("f4") >= x)
    # Tightness: no float16 lies strictly between the bound and x.
    lo = codec.fp16_floor(x)
    assert np.all(np.nextafter(lo, np.float16(np.inf)).astype("f4") > x)


def test_gqa_causal_against_scalar_oracle():
    rng = np.random.default_rng(17)
    q = rng.normal(size=(6, 2, 8)).astype("f4")
    k = rng.normal(size=(2, 7, 8)).astype("f4")
    v = rng.normal(size=k.shape).astype("f4")
    positions = np.array([3, 6])
    got, p = codec.attention(q, k, v, positions)
    ref = np.zeros_like(got)
    for h in range(6):
        for i, t in enumerate(positions):
            scores = k[h // 3, : t + 1].astype("f8") @ q[h, i].astype("f8") / np.sqrt(8)
            w = np.exp(scores - scores.max())
            w /= w.sum()
            ref[h, i] = w @ v[h // 3, : t + 1]
    np.testing.assert_allclose(got, ref, rtol=2e-6, atol=2e-6)
    assert np.all(p[:, 0, 4:] == 0)


@pytest.mark.parametrize("normalization", ["page_channel", "token"])
def test_real_astc_constants(normalization):
    x = np.full((1, 96, 64), 3.75, np.float32)
    y = codec.encode_tensor(x, dict(layout="scalar", block=6, normalization=normalization), quality=10)
    np.testing.assert_allclose(y.decoded, x, atol=1e-5)


def test_hdr_profile_is_rejected_by_the_ldr_codec():
    x = np.full((1, 96, 64), 3.75, np.float32)
    with pytest.raises(RuntimeError):
        codec.encode_tensor(x, dict(layout="scalar", block=6, normalization="block_min", profile="hdr"),
                            quality=10)


def test_quantizer_counts():
    x = np.random.default_rng(4).normal(size=(3, 288, 64)).astype("f4")
    for bits in (2, 4, 8):
        decoded, counts = codec.affine_quantize(x, bits)
        assert sum(counts.values()) * 8 / x.size == bits + 0.5
        assert np.isfinite(decoded).all()


@pytest.mark.parametrize("bits,axis,group", [(4, "token", 32), (2, "token", 64), (8, "channel", 96)])
def test_quantizer_codes_match_oracle_and_invariants(bits, axis, group):
    x = np.random.default_rng(bits).standard_t(3, size=(2, 192, 128)).astype("f4")
    dec, counts, codes, packed, offset, scale = codec.affine_quantize_codes(x, bits, axis, group)
    ref = R.affine_quantize(x, bits, axis, group)
    rdec, rcodes = ref[0], ref[2]
    np.testing.assert_array_equal(codes.ravel(), rcodes.ravel())
    np.testing.assert_array_equal(dec, rdec)
    assert codes.max() <= (1 << bits) - 1
    # Reconstruction error within half a step of the group's scale.
    step = np.broadcast_to(scale.astype(np.float32), codes.shape).reshape(x.shape)
    assert np.all(np.abs(dec - x) <= step / 2 * (1 + 1e-6))
    # Packing: code i of each run of 8/bits sits at bit (i mod 8/bits) * bits.
    per = 8 // bits
    flat = codes.ravel()
    unpacked = ((packed[:, None] >> (np.arange(per, dtype=np.uint8) * bits)) & ((1 << bits) - 1)).ravel()
    np.testing.assert_array_equal(unpacked[: flat.size], flat)


def test_affine_quantize_matches_reference_vectors(golden):
    """The product quantiser against outputs of the reference's own
    affine_quantize (tests/golden/gen_affine_quantize.py), ties included."""
    import json
    meta = json.loads((golden / "affine_quantize.json").read_text())
    with np.load(golden / "affine_quantize.npz", allow_pickle=False) as z:
        for c in meta["cases"]:
            dec, counts = codec.affine_quantize(z[c["input"] + "__x"], c["bits"], c["axis"], c["group"])
            assert np.array_equal(dec.view(np.uint32), z[c["key"]].view(np.uint32)), c["key"]
            assert counts == c["counts"]


@pytest.mark.parametrize("cap", ["records_l17", "science_l5"])
def test_normalisation_and_packing_match_reference_capture(golden, cap):
    """codec.encode_tensor's token normalisation and scalar packing
    (codec.py:162-166, :181-187) and atlas.normalize_tokens on a captured V
    prefix reproduce the reference's fp16 offsets/scales and padded image."""
    from astc_kv.atlas import normalize_tokens
    with np.load(golden / "geometry" / f"{cap}_fixed_input.npz", allow_pickle=False) as z:
        x, padded, off, sc = z["original_v_prefix"], z["normalized_padded"], z["fp16_offsets"], z["fp16_scales"]
    heads, tokens, dim = x.shape
    u, o, s = codec._range_normalize(x, "token", heads, tokens, dim, 66, 6, 6, 96)
    assert np.array_equal(o.view(np.uint16), off.view(np.uint16))
    assert np.array_equal(s.view(np.uint16), sc.view(np.uint16))
    image = codec.pack_images(np.clip(u, 0, 1), "scalar", 66)
    assert np.array_equal(image[..., 0].view(np.uint32), padded.view(np.uint32))
    assert np.all(image[..., 0] == image[..., 1]) and np.all(image[..., 3] == 1)
    u2, o2, s2 = normalize_tokens(x)
    assert np.array_equal(o2.view(np.uint16), off[..., 0].view(np.uint16))
    assert np.array_equal(s2.view(np.uint16), sc[..., 0].view(np.uint16))
    assert np.array_equal(u2.view(np.uint32), padded[..., :dim].view(np.uint32))
    # The byte accounting of the same encode (reference row: 25344 + 1728 + 1728).
    with patch("astc_kv.codec.AstcEncoder", IdentityAstc):
        t = codec.encode_tensor(x, dict(layout="scalar", block=6, normalization="token"))
    assert t.byte_counts == {"astc_blocks_including_edge_padding": 25344, "fp16_offsets": 1728,
                             "fp16_scales": 1728, "permutation_map": 0}


# --- the product CPU codec against the oracle ------------------------------------

def product_decode(blocks, bx, by):
    lib = codec.load_codec_library()
    blocks = np.ascontiguousarray(blocks, np.uint8).reshape(-1, 16)
    out = np.empty((len(blocks), by, bx, 4), np.uint16)
    kinds = np.empty(len(blocks), np.int32)
    rc = lib.akv_decode_blocks_fp16(bx, by, blocks.ctypes.data, len(blocks), out.ctypes.data, kinds.ctypes.data)
    assert rc == 0
    return out, kinds


def test_product_decoder_matches_oracle_on_reference_fixture(golden):
    raw = (golden / "t384" / "v-h000.astc").read_bytes()
    hdr = O.read_astc_file(raw)
    blocks = np.frombuffer(hdr["payload"], np.uint8).reshape(-1, 16)
    got, kinds = product_decode(blocks, hdr["bx"], hdr["by"])
    ref, rkinds = O.decode_blocks_fp16(blocks, hdr["bx"], hdr["by"])
    np.testing.assert_array_equal(got, ref.view(np.uint16))
    np.testing.assert_array_equal(kinds, rkinds)


@pytest.mark.parametrize("bx,by", [(4, 4), (5, 4), (6, 5), (6, 6), (8, 5), (8, 8)])
def test_product_decoder_matches_oracle_on_random_blocks(bx, by):
    blocks = np.random.default_rng(bx * 16 + by).integers(0, 256, size=(20000, 16), dtype=np.uint8)
    got, kinds = product_decode(blocks, bx, by)
    ref, rkinds = O.decode_blocks_fp16(blocks, bx, by)
    np.testing.assert_array_equal(got, ref.view(np.uint16))
    np.testing.assert_array_equal(kinds, rkinds)


@pytest.mark.parametrize("bx,by,quality", [(4, 4, 50), (6, 5, 10), (6, 5, 50), (6, 5, 98), (6, 6, 70), (8, 8, 50)])
def test_encoder_round_trip(bx, by, quality):
    """Own encoder output decodes identically in the oracle and the product
    decoder, and reconstructs smooth and noisy tiles within a loose bound."""
    rng = np.random.default_rng(quality)
    n = 256
    yy, xx = np.meshgrid(np.linspace(0, 1, by), np.linspace(0, 1, bx), indexing="ij")
    smooth = (0.2 + 0.3 * yy[None, ..., None] + 0.4 * xx[None, ..., None] * rng.random((n, 1, 1, 4)))
    noisy = np.clip(rng.normal(0.5, 0.15, size=(n, by, bx, 4)), 0, 1)
    texels = np.concatenate([smooth, noisy]).astype(np.float32)
    enc = codec.AstcEncoder((bx, by), quality)
    try:
        blocks = enc.encode_blocks(texels)
    finally:
        enc.close()
    got, _ = product_decode(blocks, bx, by)
    ref, kinds = O.decode_blocks_fp16(blocks, bx, by)
    np.testing.assert_array_equal(got, ref.view(np.uint16))
    assert np.all(kinds != 2), "encoder emitted an error block"
    dec = ref.astype(np.float32)
    assert np.abs(dec[:n] - texels[:n]).mean() < 0.08
    assert np.sqrt(((dec[n:] - texels[n:]) ** 2).mean()) < 0.15


# --- atlas and host planning --------------------------------------------------------

@pytest.mark.parametrize("layout,block,d", [("rgba", (6, 5), 64), ("rgba", (4, 4), 128), ("scalar", (6, 6), 64)])
def test_atlas_layout_and_restore(layout, block, d):
    v = np.random.default_rng(3).normal(0, 0.5, size=(2, 2, 250, d)).astype(np.float32)
    page = {(6, 5): 120, (4, 4): 128, (6, 6): 96}[block]
    at = build_atlas(v, layout, block, page, quality=50)
    bx, by = block
    t_pad = -(-250 // page) * page
    assert at.blocks.shape == (2, 2, t_pad // by, -(-texel_columns(d, layout) // bx), 16)
    assert at.scale.shape == at.offset.shape == (2, 2, 250)
    # Oracle decode of the atlas, restored with the token affine, tracks v.
    tex, kinds = O.decode_blocks_fp16(at.blocks.reshape(-1, 16), bx, by)
    assert np.all(kinds != 2)
    bb, hh, rr, cc = at.blocks.shape[:4]
    img = tex.reshape(bb, hh, rr, cc, by, bx, 4).transpose(0, 1, 2, 4, 3, 5, 6).reshape(bb, hh, rr * by, cc * bx, 4)
    img = img[:, :, :250].astype(np.float32)
    u = img[..., :d, 0] if layout == "scalar" else img[:, :, :, : d // 4].reshape(bb, hh, 250, d)
    np.testing.assert_array_equal(u, at.normalized())
    rec = R.restore_token(u, at.scale.astype(np.float32)[..., None], at.offset.astype(np.float32)[..., None])
    # i.i.d. Gaussian V at 1.2-3.7 bits per value is coded coarsely: a
    # sanity bound on the mean error relative to each token's range only.
    span = at.scale.astype(np.float32)[..., None]
    assert np.abs(rec - v).mean() < 0.2 * span.mean()
    # Byte accounting: blocks + two fp16 per token.
    counts = at.byte_counts()
    assert counts["astc_blocks"] == at.blocks.size
    assert counts["fp16_scales"] == counts["fp16_offsets"] == 2 * 2 * 250 * 2


def test_default_tiles():
    from astc_kv.gpu import default_tile, fp16_params, tile_for_splits
    # c3 (48 sequence x kv-head pairs, 256-token chunks): 16 splits = 768
    # workgroups, one round of 3 per CU on 256 CUs (two rounds of one-chunk
    # splits cost 2 x (256 + 64) > 512 + 64): two whole chunks per split.
    t = default_tile(16, 3, 8192, 256, 16)
    assert t == 512 and 48 * -(-8192 // t) == 768
    # 4x4 (160-token chunks): one full round of 16 splits.
    t = default_tile(16, 3, 8192, 160, 16)
    assert t % 16 == 0 and t == 512 and 48 * -(-8192 // t) == 768
    # 64 pairs of 32768 tokens in 80-token chunks (> 32 rounds): several
    # chunks per split.
    t = default_tile(8, 8, 32768, 80, 4)
    assert t % 80 == 0 and 80 < t <= 16 * 80
    # c4 (64 pairs, 128-token chunks, two workgroups per CU): 16 splits of
    # 2048 tokens, two full rounds on 256 CUs.
    t = default_tile(8, 8, 32768, 128, 16, groups_per_cu=2)
    assert t == 2048 and 64 * -(-32768 // t) == 2 * 512
    # Tiny workloads: split for parallelism, in whole tiles, never above a
    # chunk, at most 32 splits per sequence.
    t = default_tile(1, 3, 384, 256, 16)
    assert t == 16 and -(-384 // t) == 24
    t = default_tile(1, 3, 2048, 128, 16)
    assert t == 64 and -(-2048 // t) == 32
    # T8192 at batch 1 (192 one-chunk workgroups of 128 tokens): the chunk
    # caps the split; more splits (tile 64: 29.7 us) or fewer (tile 256:
    # 35.0 us) measured slower on the reference's payload than 128 (24.4 us).
    t = default_tile(1, 3, 8192, 128, 16)
    assert t == 128 and -(-8192 // t) == 64
    assert tile_for_splits(2048, 8, 6, 64) == 256 and -(-2048 // 256) == 8
    p = fp16_params(16, 3, 9, 8192, 64)
    assert p.tile_tokens == 512 and p.splits == 16


@pytest.mark.parametrize("bx,by", [(4, 4), (6, 5), (6, 6), (8, 8)])
def test_block_classes_against_oracle_kinds_and_spec_fields(bx, by):
    """akv_block_classes: the kind of every block equals the oracle decoder's
    (void extents valid and invalid included), and each normal block's fields
    equal those the spec-written parser reads from it."""
    import astc_spec as S
    from astc_kv.atlas import block_class_histogram
    from test_oracle_reductions import constructed_blocks
    rng = np.random.default_rng(bx * 31 + by)
    rand = rng.integers(0, 256, size=(20000, 16), dtype=np.uint8)
    rand[:1000, 0] = 0xFC
    rand[:1000, 1] = (rand[:1000, 1] & 0xF0) | rng.choice([0x0D, 0x0F], size=1000).astype(np.uint8)
    rand[:200, 8:] = 0xFF   # all-ones extents
    blocks = np.concatenate([np.array(constructed_blocks(bx, by), np.uint8).reshape(-1, 16), rand])
    lib = codec.load_codec_library()
    cls = np.empty(len(blocks), np.uint32)
    assert lib.akv_block_classes(bx, by, blocks.ctypes.data, len(blocks), cls.ctypes.data) == 0
    _, kinds = O.decode_blocks_fp16(blocks, bx, by)
    np.testing.assert_array_equal(cls & 3, kinds)
    assert np.count_nonzero(kinds == 0) > 400 and np.count_nonzero(kinds == 1) > 100
    for raw, c in zip(blocks[kinds == 0], cls[kinds == 0]):
        b = S.parse_block(bytes(raw))
        shared = len(b.cems) == 1 or (raw[2] >> 7 | (raw[3] & 1) << 1) == 0   # bits 23-24
        expect = ((len(b.cems) - 1) << 2 | b.dual << 4 | int((b.w, b.h) == (bx, by)) << 5 |
                  S.LEVELS[b.wrange] << 6 | b.cems[0] << 12 | int(shared) << 16)
        assert int(c) == expect, (raw.tolist(), hex(int(c)), hex(expect))
    h = block_class_histogram(blocks, bx, by, "rgba")
    assert h["blocks"] == len(blocks)
    assert abs(h["table_path"] + h["compute_path"] + h["void_extent"] + h["error"] - 1) < 1e-3
    assert abs(sum(h["partitions"].values()) - np.mean(kinds == 0)) < 1e-3


@pytest.mark.parametrize("pair", [("records", 17), ("science", 5)])
def test_encoder_quality_against_astcenc_record(golden, pair):
    """Own encoder at quality 98 on the reference's captured, normalised V
    (fixed_input.npz of scripts/probe_block_geometry.py:142-155): the error
    tests/golden/encoder_quality.py recorded is reproduced, and stays within
    1.15x of astcenc 5.7.0's recorded quality-98 error on the same image."""
    import json
    cap, layer = pair
    rec = next(r for r in json.loads((golden / "encoder_quality.json").read_text())["pairs"]
               if r["capture"] == cap and r["layer"] == layer)
    z = np.load(golden / "geometry" / f"{cap}_l{layer}_fixed_input.npz")
    scalar = z["normalized_padded"].astype(np.float32)
    enc = codec.AstcEncoder((6, 6), 98)
    try:
        dec = []
        for img in scalar:
            image = np.ones(img.shape + (4,), np.float32)
            image[..., :3] = img[..., None]
            dec.append(enc.roundtrip(image)[1][..., 0])
    finally:
        enc.close()
    err = float(np.sum(np.square(np.stack(dec).astype(np.float64) - scalar)))
    assert err == pytest.approx(rec["this_q98"]["normalized_padded_error_sse"], rel=1e-9)
    assert err <= 1.15 * rec["astcenc_q98"]["normalized_padded_error_sse"]
