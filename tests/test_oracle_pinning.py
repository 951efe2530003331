"""Pins the oracle before anything is compared against it.

* Against the reference's archived astcenc 5.7.0 outputs (tests/golden, copied by
  tests/golden/collect_fixtures.py): decoded texels u must recompose the
  reference's restored tensors bit-exactly as fl32(fl32(u*s)+o)
  (astc_kv/codec.py:206, :203).
* Against closed forms for what the data leave open: the trit and quint block
  codes are bijections onto all digit tuples, unquantised levels are evenly
  spaced with exact end points, bit counts of integer sequences, void-extent
  colours and the UNORM16 -> FP16 truncation rule.
"""
import itertools
import json

import numpy as np
import pytest

from oracle import astc_oracle as O
from oracle import attention_ref as R

SEED_RANDOM36 = 20261028  # configs/block_geometry_v2.json "seed"


def _geometry_maps():
    g = np.arange(36).reshape(6, 6)
    return {"identity": g.ravel(), "transpose": g.T.ravel(),
            "random36": np.random.default_rng(SEED_RANDOM36).permutation(36)}


def _join_blocks(a, tokens, width, block=6):
    return a.reshape(len(a), tokens // block, width // block, block, block).transpose(0, 1, 3, 2, 4).reshape(
        len(a), tokens, width)


@pytest.mark.parametrize("name,T", [("t384", 384), ("t391", 391)])
def test_token_fixture_bit_exact(golden, name, T):
    d = golden / name
    m = json.loads((d / "manifest.json").read_text())
    assert m["encoder"]["version"] == "5.7.0" and m["v_normalization"] == "token"
    vd = np.fromfile(d / "v_decoded.f32", "<f4").reshape(3, T, 64)
    s = np.fromfile(d / "v_scale.f16", "<f2").reshape(3, T, 1)
    o = np.fromfile(d / "v_offset.f16", "<f2").reshape(3, T, 1)
    for h in range(3):
        f = O.read_astc_file((d / f"v-h{h:03d}.astc").read_bytes())
        assert (f["bx"], f["by"], f["width"]) == (6, 6, 66)
        img = O.decode_image(f["payload"], 6, 6, f["width"], f["height"])
        u = img[:T, :64, 0]
        assert np.all(u.astype(np.float16).astype(np.float32) == u), "decoded texels must be FP16 values"
        rec = R.restore_token(u, s[h], o[h])
        assert np.array_equal(rec.view(np.uint32), vd[h].view(np.uint32))


def test_page_channel_fixture_bit_exact(golden):
    d = golden / "kv_page6"
    for side in "kv":
        dec = np.fromfile(d / f"{side}_decoded.f32", "<f4").reshape(3, 384, 64)
        s = np.fromfile(d / f"{side}_scale.f16", "<f2").reshape(3, 4, 64)
        o = np.fromfile(d / f"{side}_offset.f16", "<f2").reshape(3, 4, 64)
        u = np.stack([O.decode_image(O.read_astc_file((d / f"{side}-h{h:03d}.astc").read_bytes())["payload"],
                                     6, 6, 66, 384)[:, :64, 0] for h in range(3)])
        rec = R.restore_page_channel(u, s, o, 96)
        assert np.array_equal(rec.view(np.uint32), dec.view(np.uint32)), side


@pytest.mark.parametrize("cap", ["records_l17", "science_l5"])
@pytest.mark.parametrize("variant", ["identity", "transpose", "random36"])
def test_geometry_fixture_bit_exact(golden, cap, variant):
    g = golden / "geometry"
    raw = np.fromfile(g / f"{cap}_{variant}.bin", np.uint8).reshape(-1, 16)
    expected = np.load(g / f"{cap}_{variant}.npy", allow_pickle=False)
    with np.load(g / f"{cap}_ranges.npz", allow_pickle=False) as z:
        s, o = z["fp16_scales"], z["fp16_offsets"]
    tex, kinds = O.decode_blocks_fp16(raw, 6, 6)
    assert np.all(kinds == 0)
    u = tex[..., 0].astype(np.float32).reshape(3, -1, 36)
    u = u[..., np.argsort(_geometry_maps()[variant])]     # undo the in-block map
    restored = _join_blocks(u, 288, 66)[:, :, :64]
    rec = R.restore_token(restored, s, o)
    assert np.array_equal(rec.view(np.uint32), expected.view(np.uint32))


def test_holdout_payloads_decode_to_valid_fp16(golden):
    for f in sorted((golden / "holdout").glob("*.bin")):
        raw = np.fromfile(f, np.uint8).reshape(-1, 16)
        tex, kinds = O.decode_blocks_fp16(raw, 6, 6)
        assert np.all(kinds == 0), f.name
        v = tex.astype(np.float32)
        assert np.all((v >= 0) & (v <= 1)) and np.all(v[..., 3] == 1.0)
        assert np.all(v[..., 0] == v[..., 1]) and np.all(v[..., 1] == v[..., 2])


def test_trit_and_quint_codes_are_onto():
    tuples = {tuple(O.decode_trits(T)) for T in range(256)}
    assert tuples == set(itertools.product(range(3), repeat=5))
    assert O.decode_trits(0) == [0] * 5
    qt = {tuple(O.decode_quints(Q)) for Q in range(128)}
    assert qt == set(itertools.product(range(5), repeat=3))
    assert O.decode_quints(0) == [0] * 3


def test_unquantised_levels_evenly_spaced():
    for r, levels in enumerate(O.LEVELS):
        if r >= 4:  # colour ranges start at 6 levels
            vals = sorted(O.unquant_color(r, v) for v in range(levels))
            ideal = np.round(np.arange(levels) * 255 / (levels - 1))
            assert vals[0] == 0 and vals[-1] == 255
            assert np.max(np.abs(np.array(vals) - ideal)) <= 1, (levels, vals)
        if r <= 11:  # weight ranges up to 32 levels
            w = sorted(O.unquant_weight(r, v) for v in range(levels))
            ideal = np.round(np.arange(levels) * 64 / (levels - 1))
            assert w[0] == 0 and w[-1] == 64
            assert np.max(np.abs(np.array(w) - ideal)) <= 1, (levels, w)


def test_unquant_known_orderings():
    # A weight range's odd ISE value mirrors the even one below it: w(v^1) = 64 - w(v)
    # for trit/quint ranges with at least one plain bit.
    for r in (4, 6, 7, 9, 10):
        for v in range(0, O.LEVELS[r], 2):
            assert O.unquant_weight(r, v) + O.unquant_weight(r, v + 1) == 64
        for v in range(0, O.LEVELS[r], 2):
            if r >= 4:
                assert O.unquant_color(r, v) + O.unquant_color(r, v + 1) == 255


def test_ise_bit_counts_closed_form():
    for r, levels in enumerate(O.LEVELS):
        for n in range(1, 65):
            bits = int(np.log2(levels & -levels))
            if levels % 3 == 0:
                expect = n * bits + -(-8 * n // 5)
            elif levels % 5 == 0:
                expect = n * bits + -(-7 * n // 3)
            else:
                expect = n * bits
            assert O.ise_bits(n, r) == expect


def test_unorm16_to_fp16_rule():
    for c in range(65536):
        h = np.uint16(O.unorm16_to_fp16(c)).view(np.float16)
        if c == 0xFFFF:
            assert h == 1.0
            continue
        exact = c / 65536.0
        assert float(h) <= exact
        nxt = np.nextafter(h, np.float16(2))
        assert float(nxt) > exact, c


def test_void_extent_blocks():
    rng = np.random.default_rng(3)
    for _ in range(200):
        rgba = rng.integers(0, 65536, 4)
        blk = bytearray(16)
        word = 0x1FC | (0 << 9) | (3 << 10) | (((1 << 52) - 1) << 12)
        blk[:8] = word.to_bytes(8, "little")
        for c in range(4):
            blk[8 + 2 * c: 10 + 2 * c] = int(rgba[c]).to_bytes(2, "little")
        tex, kind = O.decode_block_unorm16(bytes(blk), 6, 5)
        assert kind == 1 and np.all(tex == rgba[None, None, :])


def test_partition_small_block_doubles_coordinates():
    # Blocks with fewer than 31 texels evaluate the hash at doubled coordinates.
    for seed in range(0, 1024, 37):
        for pc in (2, 3, 4):
            for x in range(4):
                for y in range(4):
                    assert O.select_partition(seed, x, y, 0, pc, True) == O.select_partition(
                        seed, 2 * x, 2 * y, 0, pc, False)


def test_block_mode_header_examples():
    # probe_block_geometry.py:88-89 header examples: mode 291 with 2 partitions
    # decodes as a normal block (not void extent), 0x1FC as a void extent.
    blk = bytes([0x23, 0x09]) + bytes(14)
    _, kind = O.decode_block_unorm16(blk, 6, 6)
    assert kind in (0, 2)
    blk = bytes([0xFC, 0x01]) + bytes(14)
    _, kind = O.decode_block_unorm16(blk, 6, 6)
    assert kind in (1, 2)


@pytest.mark.parametrize("cap", ["records_l17", "science_l5"])
def test_token_normalisation_matches_reference_capture(golden, cap):
    """The reference's own normalisation of two captured V prefixes
    (scripts/probe_block_geometry.py:142-146, the code of codec.py:162-166):
    fp16 offsets and scales and the clipped, edge-padded scalar image, bit for
    bit, from the captured float32 values."""
    with np.load(golden / "geometry" / f"{cap}_fixed_input.npz", allow_pickle=False) as z:
        x, padded, off, sc = z["original_v_prefix"], z["normalized_padded"], z["fp16_offsets"], z["fp16_scales"]
    u, o, s = R.normalize_token(x)
    assert np.array_equal(o.view(np.uint16), off.view(np.uint16))
    assert np.array_equal(s.view(np.uint16), sc.view(np.uint16))
    mine = np.pad(u, ((0, 0), (0, 0), (0, padded.shape[-1] - u.shape[-1])), mode="edge")
    assert np.array_equal(mine.view(np.uint32), padded.view(np.uint32))


def test_affine_quantize_matches_reference_vectors(golden):
    """affine_quantize outputs written by the reference module itself
    (tests/golden/gen_affine_quantize.py): 5 configurations x 3 inputs,
    including exact half-step ties (round half to even)."""
    meta = json.loads((golden / "affine_quantize.json").read_text())
    with np.load(golden / "affine_quantize.npz", allow_pickle=False) as z:
        for c in meta["cases"]:
            dec, counts, *_ = R.affine_quantize(z[c["input"] + "__x"], c["bits"], c["axis"], c["group"])
            assert np.array_equal(dec.view(np.uint32), z[c["key"]].view(np.uint32)), c["key"]
            assert counts == c["counts"]
