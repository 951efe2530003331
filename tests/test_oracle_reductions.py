"""Pins the oracle's decode of the ASTC features the reference's astcenc
payloads never contain by reducing each to the astcenc-pinned path.

The archived payloads (tests/golden, astcenc 5.7.0 at quality 98) hold only
6x6 luminance blocks: endpoint mode 0 (and three class-0/1 blocks), 1-4
partitions, six weight grids. test_oracle_pinning.py pins the oracle's decode
of every one of them bit for bit. Here:

* the block writer of tests/astc_spec.py (written from the specification) is
  pinned first: the fields it parses from every archived block write back to
  a block with the same fields and the same decoded texels;
* every archived block's endpoint pairs are re-expressed in the other LDR
  endpoint modes: luminance base+offset (1), luminance+alpha (4, 5), RGB and
  RGBA direct (8, 12) unswapped and swapped with blue contraction, RGB(A)
  base+offset with bit transfer (9, 13) in both orders, RGB base+scale (6,
  10), and partitions mixing endpoint classes (extra mode bits below the
  weights). Each such block must decode to exactly the astcenc texels of the
  block it came from; a plausible mistake in any of these modes (a swapped
  pair, a missing blue contraction, a wrong bit transfer, a misplaced mode
  bit) changes the texels;
* endpoints swapped with mirrored weights (w -> 64 - w) decode identically;
* per-channel separability: an RGBA block with four different endpoint pairs
  decodes, channel by channel, to the luminance blocks of those pairs;
* dual plane: a block whose two weight planes are equal decodes like the
  single-plane block, and with different planes the selected channel follows
  the second plane only;
* footprints 4x4 .. 12x12 with identity weight grids map texel (x, y) to
  weight y * bx + x (one-hot weights), and reduced grids reproduce their
  corner weights at the corner texels, constant grids give constant texels
  and weights that grow along x never shrink along x.

The colour channel each endpoint value feeds (R from values 0/1, G from 2/3,
B from 4/5, A from 6/7) is the specification's table; luminance data cannot
distinguish channels, so that assignment is pinned by the specification text
only.
"""
from __future__ import annotations

from functools import lru_cache

import numpy as np
import pytest

import astc_spec as S
from oracle import astc_oracle as O


@lru_cache(maxsize=None)
def fixture_blocks():
    from conftest import GOLDEN
    g = GOLDEN
    raw = [np.frombuffer(O.read_astc_file(p.read_bytes())["payload"], np.uint8) for p in sorted(g.glob("t*/*.astc"))]
    raw += [np.frombuffer(O.read_astc_file(p.read_bytes())["payload"], np.uint8)
            for p in sorted(g.glob("kv_page6/*.astc"))]
    raw += [np.fromfile(p, np.uint8) for p in sorted(g.glob("geometry/*.bin"))]
    raw += [np.fromfile(p, np.uint8) for p in sorted(g.glob("holdout/*.bin"))]
    return np.unique(np.concatenate(raw).reshape(-1, 16), axis=0)


@lru_cache(maxsize=None)
def parsed_fixtures():
    out = []
    for b in fixture_blocks():
        f = S.parse_block(bytes(b))
        assert f is not None
        out.append((bytes(b), f))
    return out


def decode(blocks, bx=6, by=6):
    tex, kinds = O.decode_blocks_fp16(np.frombuffer(b"".join(blocks), np.uint8).reshape(-1, 16), bx, by)
    return tex.view(np.uint16), kinds


@lru_cache(maxsize=None)
def unq_colour(r):
    return [O.unquant_color(r, q) for q in range(S.LEVELS[r])]


@lru_cache(maxsize=None)
def _q_index(r):
    out = {}
    for q, byte in enumerate(unq_colour(r)):
        out.setdefault(byte, q)
    return out


def q_of(r, byte):
    """An ISE value of colour range r that unquantises to `byte`, or None."""
    return _q_index(r).get(int(byte))


def test_writer_matches_archived_blocks():
    blocks = [b for b, _ in parsed_fixtures()]
    rebuilt, same_bytes = [], 0
    for b, f in parsed_fixtures():
        w = S.write_block(S.Block(f.w, f.h, f.wrange, list(f.weights), list(f.cems), list(f.colours), f.seed,
                                  f.dual, f.ccs))
        g = S.parse_block(w)
        assert (g.w, g.h, g.wrange, g.weights, g.cems, g.colours, g.seed, g.crange) == \
               (f.w, f.h, f.wrange, f.weights, f.cems, f.colours, f.seed, f.crange)
        rebuilt.append(w)
        same_bytes += w == b
    a, _ = decode(blocks)
    c, _ = decode(rebuilt)
    assert np.array_equal(a, c)
    assert same_bytes >= 0.7 * len(blocks)   # the rest differ only in duplicate trit/quint codes
    # The spec's trit/quint decoding restated here agrees with the oracle's.
    assert all(S.trit_decode(T) == O.decode_trits(T) for T in range(256))
    assert all(S.quint_decode(Q) == O.decode_quints(Q) for Q in range(128))


# --- endpoint-mode reductions ---------------------------------------------------

def _bt_pair(base, off, r):
    """ISE values (b, o) whose bit transfer gives base `base` and signed 6-bit
    offset `off`: base = (b >> 1) | (o & 0x80), off = sext6((o >> 1) & 0x3F)."""
    if not -32 <= off <= 31:
        return None
    for lo in (0, 1):
        vb = q_of(r, ((base & 0x7F) << 1) | lo)
        if vb is None:
            continue
        for lo2 in (0, 1):
            vo = q_of(r, (base & 0x80) | ((off & 0x3F) << 1) | lo2)
            if vo is not None:
                return vb, vo
    return None


def _bt_alpha255(r):
    """Bit-transfer alpha values giving 255 at both ends: base 255 and any
    offset in [0, 31] (the sum clamps to 255)."""
    for off in range(32):
        got = _bt_pair(255, off, r)
        if got is not None:
            return got
    return None


def _scale_pair(A, B, r):
    """(base, scale) ISE values with base = B and (B * scale) >> 8 = A."""
    vb = q_of(r, B)
    if vb is None:
        return None
    for s, byte in enumerate(unq_colour(r)):
        if (B * byte) >> 8 == A:
            return vb, s
    return None


def _values(kind, A, B, r):
    """ISE values of one partition's endpoints in mode `kind` that decode to the
    luminance pair e0 = A, e1 = B with alpha 255, or None."""
    q = lambda x: q_of(r, x)  # noqa: E731
    if kind == "cem1":
        if not 0 <= B - A <= 63:
            return None
        v1 = q((A & 0xC0) | (B - A))
        for lo in range(4):
            v0 = q(((A & 0x3F) << 2) | lo)
            if v0 is not None and v1 is not None:
                return [v0, v1]
        return None
    if kind == "cem4":
        out = [q(A), q(B), q(255), q(255)]
    elif kind == "cem5":
        lum, alpha = _bt_pair(A, B - A, r), _bt_alpha255(r)
        return None if lum is None or alpha is None else [*lum, *alpha]
    elif kind in ("cem6", "cem10"):
        if A > B:
            return None
        bs = _scale_pair(A, B, r)
        if bs is None:
            return None
        out = [bs[0], bs[0], bs[0], bs[1]] + ([q(255), q(255)] if kind == "cem10" else [])
    elif kind in ("cem8", "cem12"):
        if B < A:
            return None
        out = [q(A), q(B)] * 3 + ([q(255), q(255)] if kind == "cem12" else [])
    elif kind in ("cem8s", "cem12s"):   # sum of e1 < sum of e0: swapped, blue-contracted
        if not A < B:
            return None
        out = [q(B), q(A)] * 3 + ([q(255), q(255)] if kind == "cem12s" else [])
    elif kind in ("cem9", "cem13"):
        p = _bt_pair(A, B - A, r)
        if p is None or B < A:
            return None
        out = list(p) * 3
        if kind == "cem13":
            a = _bt_alpha255(r)
            out = None if a is None else out + list(a)
    elif kind in ("cem9s", "cem13s"):   # negative offsets: swapped, blue-contracted
        p = _bt_pair(B, A - B, r)
        if p is None or not A < B:
            return None
        out = list(p) * 3
        if kind == "cem13s":
            a = _bt_alpha255(r)
            out = None if a is None else out + list(a)
    else:
        raise ValueError(kind)
    return None if out is None or any(v is None for v in out) else out


KINDS = {"cem1": 1, "cem4": 4, "cem5": 5, "cem6": 6, "cem8": 8, "cem8s": 8, "cem9": 9, "cem9s": 9, "cem10": 10,
         "cem12": 12, "cem12s": 12, "cem13": 13, "cem13s": 13}
# Partitions alternating between two endpoint classes (per-partition mode bits).
MIXED = {"mixed01": ("cem1", "cem4"), "mixed12": ("cem4", "cem8"), "mixed23": ("cem9", "cem13"),
         "mixed_all": ("cem5", "cem8s")}


def _reexpress(f, kinds, rng=None):
    """Block f (endpoint mode 0 in every partition) with partition p's endpoints
    in mode kinds[p % len(kinds)]: (source block, re-expressed block) or None
    when the values do not fit or cannot reach the same endpoints.

    With rng, each partition first gets new endpoints drawn so that the mode
    can express them (base+offset modes need |e1 - e0| <= 31, which token-
    normalised data never has; direct modes need e1 >= e0 in every partition
    and values the lower colour range holds): the source block is then f with
    those endpoints, still a mode-0 block on f's mode, weights and
    partitions."""
    if any(c != 0 for c in f.cems):
        return None
    levels = unq_colour(f.crange)
    ends = [(levels[f.colours[2 * p]], levels[f.colours[2 * p + 1]]) for p in range(f.parts)]
    cems = [KINDS[kinds[p % len(kinds)]] for p in range(f.parts)]
    if max(cems) // 4 - min(cems) // 4 > 1:
        return None
    g = S.Block(f.w, f.h, f.wrange, list(f.weights), cems, [0] * sum(2 * ((c >> 2) + 1) for c in cems), f.seed)
    r = S.colour_range(len(g.colours), S.colour_bits_available(g))
    if r < 0:
        return None
    src_bytes = None
    if rng is not None:
        src_levels = set(levels)
        new = []
        for p in range(f.parts):
            pairs = [pr for pr in reachable(kinds[p % len(kinds)], r)
                     if pr[0] in src_levels and pr[1] in src_levels]
            if not pairs:
                return None
            new.append(pairs[int(rng.integers(len(pairs)))])
        ends = new
        src_bytes = S.write_block(S.Block(f.w, f.h, f.wrange, list(f.weights), list(f.cems),
                                          [levels.index(x) for pr in ends for x in pr], f.seed))
    vals = []
    for p, (A, B) in enumerate(ends):
        v = _values(kinds[p % len(kinds)], A, B, r)
        if v is None:
            return None
        vals += v
    g.colours = vals
    return src_bytes, S.write_block(g)


@lru_cache(maxsize=None)
def reachable(kind, r):
    """Luminance endpoint pairs (e0, e1), e0 != e1, that mode `kind` can express
    exactly in colour range r."""
    return [(A, B) for A in range(256) for B in range(256) if A != B and _values(kind, A, B, r) is not None]


@lru_cache(maxsize=None)
def endpoint_mode_blocks(name):
    """(source blocks, the same blocks re-expressed in endpoint mode(s) `name`)."""
    kinds = MIXED.get(name, (name,))
    rng = np.random.default_rng(sum(map(ord, name)))
    src, built, exact = [], [], 0
    for b, f in parsed_fixtures():
        got = _reexpress(f, kinds)
        if got is not None:
            exact += 1
        elif len(built) < 250 + exact:
            got = _reexpress(f, kinds, rng)
        if got is not None:
            src.append(got[0] or b)
            built.append(got[1])
    return src, built


@pytest.mark.parametrize("name", list(KINDS) + list(MIXED))
def test_endpoint_modes_reduce_to_luminance(name):
    """Archived blocks re-expressed with their own endpoints where the mode can
    hold them, and with drawn endpoints on the same mode, weights and
    partitions otherwise (at least 200 blocks per mode)."""
    kinds = MIXED.get(name, (name,))
    src, built = endpoint_mode_blocks(name)
    assert len(built) >= 200, f"{name}: only {len(built)} blocks"
    # The re-expressed blocks really use the intended modes.
    for w in built[:50]:
        g = S.parse_block(w)
        assert g.cems == [KINDS[kinds[p % len(kinds)]] for p in range(g.parts)]
    a, ka = decode(src)
    c, kc = decode(built)
    assert np.all(ka == 0) and np.all(kc == 0)
    bad = np.flatnonzero((a != c).any(axis=(1, 2, 3)))
    assert bad.size == 0, f"{name}: {bad.size} of {len(built)} blocks differ"


def _mirror_weights(f):
    levels = S.LEVELS[f.wrange]
    w = [O.unquant_weight(f.wrange, q) for q in range(levels)]
    mirror = {q: w.index(64 - w[q]) for q in range(levels)}
    return [mirror[q] for q in f.weights]


def test_swapped_endpoints_with_mirrored_weights():
    """Swapping every partition's endpoints and mirroring the weights (w ->
    64 - w) leaves the texels unchanged on identity grids (6x6 weights on 6x6
    texels). On reduced grids the infill rounds half up, (sum + 8) >> 4, which
    is not symmetric under the mirror, so they are left out."""
    src, built = [], []
    for b, f in parsed_fixtures():
        if f.cems != [0] * f.parts or (f.w, f.h) != (6, 6):
            continue
        cols = list(f.colours)
        for p in range(f.parts):
            cols[2 * p], cols[2 * p + 1] = cols[2 * p + 1], cols[2 * p]
        built.append(S.write_block(S.Block(f.w, f.h, f.wrange, _mirror_weights(f), list(f.cems), cols, f.seed)))
        src.append(b)
    a, _ = decode(src)
    c, _ = decode(built)
    assert len(built) > 1000 and np.array_equal(a, c)


def _lum_block(f, A, B):
    """Single-partition luminance block with f's grid and weights and endpoints
    (A, B) (colour range 20 when it fits, else None)."""
    g = S.Block(f.w, f.h, f.wrange, list(f.weights), [0], [0, 0])
    r = S.colour_range(2, S.colour_bits_available(g))
    if q_of(r, A) is None or q_of(r, B) is None:
        return None
    g.colours = [q_of(r, A), q_of(r, B)]
    return S.write_block(g)


def test_rgba_channels_are_separable():
    """An RGBA-direct block with four endpoint pairs decodes, channel by channel,
    like the luminance blocks of those pairs (astcenc-pinned path)."""
    rng = np.random.default_rng(12)
    done = 0
    for b, f in parsed_fixtures():
        if f.parts != 1 or done >= 200:
            continue
        g = S.Block(f.w, f.h, f.wrange, list(f.weights), [12], [0] * 8)
        r = S.colour_range(8, S.colour_bits_available(g))
        if r < 0:
            continue
        levels = unq_colour(r)
        # Four pairs with e1 >= e0 in every channel (no swap): sums agree.
        pairs = [tuple(sorted(rng.choice(levels, 2))) for _ in range(4)]
        lum = [_lum_block(f, A, B) for A, B in pairs]
        if any(x is None for x in lum):
            continue
        g.colours = [levels.index(x) for pr in pairs[:3] for x in pr] + [levels.index(x) for x in pairs[3]]
        rgba, _ = decode([S.write_block(g)])
        ref, _ = decode(lum)
        for ch in range(4):
            assert np.array_equal(rgba[0, ..., ch], ref[ch, ..., 0]), (ch, pairs)
        done += 1
    assert done >= 100


@lru_cache(maxsize=None)
def channel_blocks(cem):
    """(blocks of endpoint mode `cem` with random values, 4 luminance blocks
    per block holding its channels' endpoint pairs, count of swap-boundary ties)."""
    rng = np.random.default_rng(100 + cem)
    nv = 2 * ((cem >> 2) + 1)
    built, lum, ties = [], [], 0
    for _, f in parsed_fixtures():
        if f.parts != 1 or len(built) >= 1500:
            continue
        g = S.Block(f.w, f.h, f.wrange, list(f.weights), [cem], [0] * nv)
        r = S.colour_range(nv, S.colour_bits_available(g))
        if r < 0:
            continue
        L = S.LEVELS[r]
        q = rng.integers(0, L, nv).tolist()
        if cem in (8, 12) and len(built) % 3 == 0:   # equal sums: v1 = v2, v3 = v4, v5 = v0
            q[1], q[3], q[5] = q[2], q[4], q[0]
        if cem in (9, 13) and len(built) % 3 == 0:   # offsets summing to zero: all three zero
            q[1] = q[3] = q[5] = q_of(r, 0)
        vals = [unq_colour(r)[x] for x in q]
        e0, e1 = S.spec_endpoints(cem, vals)
        refs = [_lum_block(f, e0[ch], e1[ch]) for ch in range(4)]
        if any(x is None for x in refs):
            continue
        if cem in (8, 12) and vals[1] + vals[3] + vals[5] == vals[0] + vals[2] + vals[4]:
            ties += 1
        if cem in (9, 13) and sum(S._bit_transfer(vals[2 * c + 1], vals[2 * c])[0] for c in range(3)) == 0:
            ties += 1
        g.colours = q
        built.append(S.write_block(g))
        lum += refs
    return built, lum, ties


@pytest.mark.parametrize("cem", [1, 4, 5, 6, 8, 9, 10, 12, 13])
def test_endpoint_modes_channel_by_channel(cem):
    """Random colour values in every LDR endpoint mode on the archived blocks'
    modes and weights: each channel decodes like the luminance (mode 0) block
    of that channel's endpoint pair, e0 -> e1 as the specification derives it
    (tests/astc_spec.spec_endpoints: swap on the sums with blue contraction,
    bit transfer, scale, alpha pairs). This is where channel routing, the
    swap condition at equal sums (values chosen so that ties occur), blue
    contraction and the alpha values are checked; the grey reductions above
    cannot see them."""
    built, lum, ties = channel_blocks(cem)
    assert len(built) >= 250
    if cem in (8, 9, 12, 13):
        assert ties >= 5, ties
    got, kinds = decode(built)
    ref, _ = decode(lum)
    assert np.all(kinds == 0)
    ref = ref.reshape(len(built), 4, 6, 6, 4)
    for ch in range(4):
        bad = np.flatnonzero((got[..., ch] != ref[:, ch, ..., 0]).any(axis=(1, 2)))
        assert bad.size == 0, f"mode {cem} channel {ch}: {bad.size} of {len(built)} blocks differ"


# --- dual plane -------------------------------------------------------------------

def _dual_cases():
    """Single-partition archived blocks whose weight grid doubled still fits a
    dual-plane mode (grids of at most 32 weights, ranges of 2-4 levels)."""
    for b, f in parsed_fixtures():
        if f.parts == 1 and f.w * f.h <= 32 and S.ise_bits(2 * f.w * f.h, f.wrange) <= 96:
            yield b, f
    # Constructed ones on the archived grids too (few archived blocks qualify).
    rng = np.random.default_rng(5)
    for (w, h) in ((6, 4), (4, 6), (6, 5), (5, 6), (5, 5)):
        for wr in (0, 1, 2):
            if S.ise_bits(2 * w * h, wr) > 96:
                continue
            for _ in range(20):
                f = S.Block(w, h, wr, rng.integers(0, S.LEVELS[wr], w * h).tolist(), [0], [0, 0])
                f.crange = S.colour_range(2, S.colour_bits_available(f))
                f.colours = rng.integers(0, S.LEVELS[f.crange], 2).tolist()
                yield S.write_block(f), f


@lru_cache(maxsize=None)
def dual_blocks():
    """(single-plane blocks, the same as dual-plane blocks with equal planes)."""
    src, built = [], []
    for b, f in _dual_cases():
        ends = (unq_colour(f.crange)[f.colours[0]], unq_colour(f.crange)[f.colours[1]])
        for ccs in range(4):
            g = S.Block(f.w, f.h, f.wrange, [x for q in f.weights for x in (q, q)], [0], [0, 0], dual=1, ccs=ccs)
            r = S.colour_range(2, S.colour_bits_available(g))
            if r < 0 or q_of(r, ends[0]) is None or q_of(r, ends[1]) is None:
                continue
            g.colours = [q_of(r, ends[0]), q_of(r, ends[1])]
            built.append(S.write_block(g))
            src.append(b)
    return src, built


def test_dual_plane_equal_planes_is_single_plane():
    src, built = dual_blocks()
    a, _ = decode(src)
    c, kc = decode(built)
    assert len(built) >= 100 and np.all(kc == 0)
    assert np.array_equal(a, c)


def test_dual_plane_selected_channel_follows_plane_two():
    rng = np.random.default_rng(9)
    n = 0
    for b, f in _dual_cases():
        if n >= 150:
            break
        w2 = rng.integers(0, S.LEVELS[f.wrange], f.w * f.h).tolist()
        ccs = int(rng.integers(0, 3))          # R, G or B: luminance alpha is constant
        g = S.Block(f.w, f.h, f.wrange, [x for pair in zip(f.weights, w2) for x in pair], [4], [0] * 4, dual=1,
                    ccs=ccs)
        r = S.colour_range(4, S.colour_bits_available(g))
        if r < 0:
            continue
        A, B = sorted(rng.choice(unq_colour(r), 2))
        g.colours = [q_of(r, A), q_of(r, B), q_of(r, 255), q_of(r, 255)]
        one = _lum_block(f, A, B)
        two = _lum_block(S.Block(f.w, f.h, f.wrange, w2, [0], [0, 0]), A, B)
        if one is None or two is None:
            continue
        dual, kind = decode([S.write_block(g)])
        ref, _ = decode([one, two])
        assert kind[0] == 0
        for ch in range(4):
            expect = ref[1] if ch == ccs else ref[0]
            assert np.array_equal(dual[0, ..., ch], expect[..., ch]), (ch, ccs)
        n += 1
    assert n >= 100


# --- footprints and weight grids ---------------------------------------------------

# Footprints of at most 64 texels (the decoders' limit).
FOOTPRINTS = [(4, 4), (5, 4), (5, 5), (6, 5), (6, 6), (8, 5), (8, 6), (8, 8), (10, 5), (10, 6)]


def _grid_block(w, h, wr, weights, A=0, B=255):
    g = S.Block(w, h, wr, list(weights), [0], [0, 0])
    r = S.colour_range(2, S.colour_bits_available(g))
    g.colours = [q_of(r, A), q_of(r, B)]
    return S.write_block(g)


@pytest.mark.parametrize("bx,by", FOOTPRINTS)
def test_identity_grid_maps_texel_to_weight(bx, by):
    """One-hot weights on a grid the size of the block: exactly texel (x, y) =
    weight y*bx + x decodes to 1.0, every other texel to 0."""
    # The smallest plain weight range whose sequence fills the 24 bits a mode needs.
    wr = next(r for r in (0, 2, 5, 8) if 24 <= S.ise_bits(bx * by, r) <= 96)
    hot = S.LEVELS[wr] - 1
    blocks = []
    for i in range(bx * by):
        wts = [0] * (bx * by)
        wts[i] = hot
        blocks.append(_grid_block(bx, by, wr, wts))
    tex, kinds = decode(blocks, bx, by)
    assert np.all(kinds == 0)
    one, zero = np.uint16(0x3C00), np.uint16(0)
    for i in range(bx * by):
        expect = np.full((by, bx), zero)
        expect[i // bx, i % bx] = one
        assert np.array_equal(tex[i, ..., 0], expect), (bx, by, i)


def _modes_for(bx, by):
    """Reduced (gw, gh) grids with a plain weight range that fit a mode."""
    out = []
    for gw in range(2, bx + 1):
        for gh in range(2, by + 1):
            if (gw, gh) == (bx, by):
                continue
            for wr in (2, 5, 8, 11):      # 4, 8, 16, 32 levels (plain bits)
                try:
                    S.encode_mode(gw, gh, 0, wr)
                except ValueError:
                    continue
                out.append((gw, gh, wr))
                break
    return out


def _texel_weights(tex):
    """Unquantised weight of each texel of a block with endpoints (0, 255):
    C = (65535 w + 32) >> 6, whose FP16 value identifies w (w = 0..64)."""
    table = {O.unorm16_to_fp16((65535 * w + 32) >> 6): w for w in range(65)}
    return np.vectorize(table.__getitem__)(tex)


@pytest.mark.parametrize("bx,by", FOOTPRINTS)
def test_reduced_grids_corners_constant_and_monotone(bx, by):
    rng = np.random.default_rng(bx * 13 + by)
    modes = _modes_for(bx, by)
    assert modes
    for gw, gh, wr in modes:
        L = S.LEVELS[wr]
        unq = [O.unquant_weight(wr, q) for q in range(L)]
        rand = rng.integers(0, L, gw * gh).tolist()
        const = [int(rng.integers(0, L))] * (gw * gh)
        ramp = [min(L - 1, (x * (L - 1)) // max(gw - 1, 1)) for y in range(gh) for x in range(gw)]
        tex, kinds = decode([_grid_block(gw, gh, wr, w) for w in (rand, const, ramp)], bx, by)
        assert np.all(kinds == 0)
        tw = _texel_weights(tex[..., 0])
        g = np.array([unq[q] for q in rand]).reshape(gh, gw)
        corners = [(0, 0), (0, bx - 1), (by - 1, 0), (by - 1, bx - 1)]
        gcorn = [(0, 0), (0, gw - 1), (gh - 1, 0), (gh - 1, gw - 1)]
        for (ty, tx), (gy, gx) in zip(corners, gcorn):
            assert tw[0, ty, tx] == g[gy, gx], (bx, by, gw, gh, ty, tx)
        assert np.all(tw[1] == unq[const[0]])
        assert np.all(np.diff(tw[2], axis=1) >= 0) and np.all(tw[2][:, 0] == 0) and np.all(tw[2][:, -1] == 64)
        assert np.all(tw[2] == tw[2][:1])      # a ramp along x is constant along y


def constructed_blocks(bx, by):
    """Every block these tests build for footprint bx x by, as uint8 [n, 16]
    (6x6: endpoint-mode reductions, per-channel modes, dual plane; all
    footprints: identity and reduced weight grids), for the GPU decoders."""
    out = []
    if (bx, by) == (6, 6):
        for name in list(KINDS) + list(MIXED):
            out += endpoint_mode_blocks(name)[1]
        for cem in (1, 4, 5, 6, 8, 9, 10, 12, 13):
            out += channel_blocks(cem)[0]
        out += dual_blocks()[1]
    wr = next(r for r in (0, 2, 5, 8) if 24 <= S.ise_bits(bx * by, r) <= 96)
    for i in range(bx * by):
        wts = [0] * (bx * by)
        wts[i] = S.LEVELS[wr] - 1
        out.append(_grid_block(bx, by, wr, wts))
    rng = np.random.default_rng(bx * 31 + by)
    for gw, gh, r in _modes_for(bx, by):
        cr = S.colour_range(2, S.colour_bits_available(S.Block(gw, gh, r, [0] * gw * gh, [0], [0, 0])))
        for _ in range(4):
            A, B = sorted(int(x) for x in rng.choice(unq_colour(cr), 2))
            out.append(_grid_block(gw, gh, r, rng.integers(0, S.LEVELS[r], gw * gh).tolist(), A, B))
    return np.frombuffer(b"".join(out), np.uint8).reshape(-1, 16)
