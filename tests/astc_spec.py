"""ASTC block fields <-> 128-bit blocks, written from the Khronos Data Format
Specification (ASTC chapter) for the tests: a parser and a writer of 2D LDR
blocks (block mode, partitions, colour endpoint modes, integer sequences of
colour values and weights, dual plane).

Test infrastructure only. It is kept separate from the oracle's C decoder
(oracle/astc_oracle.c) so that the reduction tests can build blocks the
reference's archived astcenc payloads never contain (RGB/RGBA endpoint
modes, dual plane, other footprints) and compare the oracle's decode of
them with its decode of the astcenc-pinned blocks they are derived from.
The writer is itself pinned: parsing every archived astcenc block and writing
the fields back gives the same fields and a block that decodes to the same
texels (tests/test_oracle_reductions.py); the bytes differ only where a trit
or quint group has two packed codes for the same digits.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from functools import lru_cache

# Levels of the 21 integer-sequence ranges (spec: "Integer Sequence Encoding").
LEVELS = [2, 3, 4, 5, 6, 8, 10, 12, 16, 20, 24, 32, 40, 48, 64, 80, 96, 128, 160, 192, 256]


def ise_params(r: int):
    """(plain bits, trit, quint) of range r."""
    n = LEVELS[r]
    if n % 3 == 0:
        return (n // 3).bit_length() - 1, True, False
    if n % 5 == 0:
        return (n // 5).bit_length() - 1, False, True
    return n.bit_length() - 1, False, False


def ise_bits(count: int, r: int) -> int:
    b, t, q = ise_params(r)
    return count * b + (-(-8 * count // 5) if t else 0) + (-(-7 * count // 3) if q else 0)


def _bit(v, i):
    return (v >> i) & 1


def trit_decode(T: int):
    """Five trits of the 8-bit packed value T (spec's trit decoding procedure)."""
    if (T >> 2) & 7 == 7:
        C = (((T >> 5) & 7) << 2) | (T & 3)
        t4 = t3 = 2
    else:
        C = T & 31
        if (T >> 5) & 3 == 3:
            t4, t3 = 2, _bit(T, 7)
        else:
            t4, t3 = _bit(T, 7), (T >> 5) & 3
    if C & 3 == 3:
        t2, t1 = 2, _bit(C, 4)
        t0 = (_bit(C, 3) << 1) | (_bit(C, 2) & (1 - _bit(C, 3)))
    elif (C >> 2) & 3 == 3:
        t2, t1, t0 = 2, 2, C & 3
    else:
        t2, t1 = _bit(C, 4), (C >> 2) & 3
        t0 = (_bit(C, 1) << 1) | (_bit(C, 0) & (1 - _bit(C, 1)))
    return [t0, t1, t2, t3, t4]


def quint_decode(Q: int):
    """Three quints of the 7-bit packed value Q (spec's quint decoding procedure)."""
    if (Q >> 1) & 3 == 3 and (Q >> 5) & 3 == 0:
        q2 = (_bit(Q, 0) << 2) | ((_bit(Q, 4) & (1 - _bit(Q, 0))) << 1) | (_bit(Q, 3) & (1 - _bit(Q, 0)))
        return [4, 4, q2]
    if (Q >> 1) & 3 == 3:
        q2 = 4
        C = (((Q >> 3) & 3) << 3) | ((~(Q >> 5) & 3) << 1) | _bit(Q, 0)
    else:
        q2 = (Q >> 5) & 3
        C = Q & 31
    if C & 7 == 5:
        q1, q0 = 4, (C >> 3) & 3
    else:
        q1, q0 = (C >> 3) & 3, C & 7
    return [q0, q1, q2]


TRIT_ENCODE = {}
for _T in range(256):
    TRIT_ENCODE.setdefault(tuple(trit_decode(_T)), _T)
QUINT_ENCODE = {}
for _Q in range(128):
    QUINT_ENCODE.setdefault(tuple(quint_decode(_Q)), _Q)


def ise_encode(values, r: int):
    """Bits (LSB first) of the integer sequence of `values` in range r."""
    b, t, q = ise_params(r)
    bits = []

    def put(v, n):
        bits.extend((v >> i) & 1 for i in range(n))

    vals = list(values)
    if t:
        for g in range(0, len(vals), 5):
            grp = vals[g:g + 5] + [0] * (5 - len(vals[g:g + 5]))
            T = TRIT_ENCODE[tuple(v >> b for v in grp)]
            m = [v & ((1 << b) - 1) for v in grp]
            seq = [(m[0], b), (T & 3, 2), (m[1], b), ((T >> 2) & 3, 2), (m[2], b), ((T >> 4) & 1, 1),
                   (m[3], b), ((T >> 5) & 3, 2), (m[4], b), ((T >> 7) & 1, 1)]
            for v, n in seq:
                put(v, n)
        return bits[:ise_bits(len(vals), r)]
    if q:
        for g in range(0, len(vals), 3):
            grp = vals[g:g + 3] + [0] * (3 - len(vals[g:g + 3]))
            Q = QUINT_ENCODE[tuple(v >> b for v in grp)]
            m = [v & ((1 << b) - 1) for v in grp]
            for v, n in [(m[0], b), (Q & 7, 3), (m[1], b), ((Q >> 3) & 3, 2), (m[2], b), ((Q >> 5) & 3, 2)]:
                put(v, n)
        return bits[:ise_bits(len(vals), r)]
    for v in vals:
        put(v, b)
    return bits


def ise_decode(bits, count: int, r: int):
    """Inverse of ise_encode (bits past the list read as zero)."""
    b, t, q = ise_params(r)
    pos = 0

    def take(n):
        nonlocal pos
        v = 0
        for i in range(n):
            if pos + i < len(bits):
                v |= bits[pos + i] << i
        pos += n
        return v

    out = []
    if t:
        while len(out) < count:
            m0 = take(b); T = take(2)
            m1 = take(b); T |= take(2) << 2
            m2 = take(b); T |= take(1) << 4
            m3 = take(b); T |= take(2) << 5
            m4 = take(b); T |= take(1) << 7
            tr = trit_decode(T)
            out += [(tr[i] << b) | m for i, m in enumerate((m0, m1, m2, m3, m4))]
    elif q:
        while len(out) < count:
            m0 = take(b); Q = take(3)
            m1 = take(b); Q |= take(2) << 3
            m2 = take(b); Q |= take(2) << 5
            qu = quint_decode(Q)
            out += [(qu[i] << b) | m for i, m in enumerate((m0, m1, m2))]
    else:
        out = [take(b) for _ in range(count)]
    return out[:count]


def decode_mode(m: int):
    """2D block mode -> (grid w, grid h, dual plane, weight range) or None for
    reserved modes and void extent (spec: "Block Mode" layout tables)."""
    if m & 0x1FF == 0x1FC:
        return None
    R = _bit(m, 4)
    H, D = _bit(m, 9), _bit(m, 10)
    A = (m >> 5) & 3
    if m & 3:
        R |= (m & 3) << 1
        B = (m >> 7) & 3
        k = (m >> 2) & 3
        if k == 0:
            w, h = B + 4, A + 2
        elif k == 1:
            w, h = B + 8, A + 2
        elif k == 2:
            w, h = A + 2, B + 8
        elif _bit(m, 8):
            w, h = (B & 1) + 2, A + 2
        else:
            w, h = A + 2, (B & 1) + 6
    else:
        if (m >> 2) & 3 == 0:
            return None
        R |= ((m >> 2) & 3) << 1
        k = (m >> 7) & 3
        if k == 0:
            w, h = 12, A + 2
        elif k == 1:
            w, h = A + 2, 12
        elif k == 2:
            w, h = A + 6, ((m >> 9) & 3) + 6
            D = H = 0
        elif A == 0:
            w, h = 6, 10
        elif A == 1:
            w, h = 10, 6
        else:
            return None
    wr = (R - 2) + 6 * H
    count = w * h * (D + 1)
    if count > 64 or not 24 <= ise_bits(count, wr) <= 96:
        return None
    return w, h, D, wr


@lru_cache(maxsize=None)
def encode_mode(w: int, h: int, dual: int, wrange: int) -> int:
    for m in range(2048):
        if decode_mode(m) == (w, h, dual, wrange):
            return m
    raise ValueError(f"no block mode for grid {w}x{h} dual={dual} range={wrange}")


def colour_range(nvalues: int, avail: int) -> int:
    """Highest range whose sequence of nvalues fits avail bits (-1: none of 6+ levels)."""
    if nvalues > 18:
        return -1
    for r in range(20, 3, -1):
        if ise_bits(nvalues, r) <= avail:
            return r
    return -1


@dataclass
class Block:
    w: int                      # weight grid
    h: int
    wrange: int
    weights: list               # ISE values, grid order, planes interleaved when dual
    cems: list                  # one per partition
    colours: list               # ISE values of the colour range (2 per endpoint pair)
    seed: int = 0               # partition pattern index (partitions > 1)
    dual: int = 0
    ccs: int = 0                # colour component of plane 1 (dual plane)
    crange: int = field(default=-1)   # filled by write/parse

    @property
    def parts(self) -> int:
        return len(self.cems)


def _put(bits, pos, n, v):
    for i in range(n):
        bits[pos + i] = (v >> i) & 1


def _get(bits, pos, n):
    return sum(bits[pos + i] << i for i in range(n))


def _cem_fields(cems):
    """(6-bit selector at bit 23, extra bits below the weights, count) for
    more than one partition."""
    if len(set(cems)) == 1:
        return cems[0] << 2, 0, 0
    classes = [c >> 2 for c in cems]
    base = min(classes)
    if max(classes) - base > 1:
        raise ValueError("partition endpoint modes must share a class or neighbour classes")
    sel = base + 1
    n = len(cems)
    for p, c in enumerate(cems):
        sel |= (c >> 2) - base << (2 + p)
    for p, c in enumerate(cems):
        sel |= (c & 3) << (2 + n + 2 * p)
    extra = 3 * n - 4
    return sel & 0x3F, sel >> 6, extra


def write_block(b: Block) -> bytes:
    bits = [0] * 128
    count = b.w * b.h * (b.dual + 1)
    if len(b.weights) != count:
        raise ValueError("weight count does not match the grid")
    mode = encode_mode(b.w, b.h, b.dual, b.wrange)
    _put(bits, 0, 11, mode)
    _put(bits, 11, 2, b.parts - 1)
    extra_v, extra_n = 0, 0
    if b.parts == 1:
        _put(bits, 13, 4, b.cems[0])
        cstart = 17
    else:
        _put(bits, 13, 10, b.seed)
        sel, extra_v, extra_n = _cem_fields(b.cems)
        _put(bits, 23, 6, sel)
        cstart = 29
    wbits = ise_encode(b.weights, b.wrange)
    for i, v in enumerate(wbits):
        bits[127 - i] = v
    below = 128 - len(wbits)
    below -= extra_n
    _put(bits, below, extra_n, extra_v)
    if b.dual:
        below -= 2
        _put(bits, below, 2, b.ccs)
    nv = sum(2 * ((c >> 2) + 1) for c in b.cems)
    if len(b.colours) != nv:
        raise ValueError(f"{nv} colour values expected")
    b.crange = colour_range(nv, below - cstart)
    if b.crange < 0:
        raise ValueError("colour values do not fit")
    if max(b.colours) >= LEVELS[b.crange]:
        raise ValueError(f"colour value out of range {b.crange}")
    for i, v in enumerate(ise_encode(b.colours, b.crange)):
        bits[cstart + i] = v
    return bytes(_get(bits, 8 * i, 8) for i in range(16))


def parse_block(raw: bytes) -> Block | None:
    """Fields of a normal block (None for void extent or reserved encodings)."""
    bits = [(raw[i >> 3] >> (i & 7)) & 1 for i in range(128)]
    md = decode_mode(_get(bits, 0, 11))
    if md is None:
        return None
    w, h, dual, wr = md
    parts = _get(bits, 11, 2) + 1
    count = w * h * (dual + 1)
    nw = ise_bits(count, wr)
    weights = ise_decode([bits[127 - i] for i in range(nw)], count, wr)
    below = 128 - nw
    seed = 0
    if parts == 1:
        cems = [_get(bits, 13, 4)]
        cstart = 17
    else:
        seed = _get(bits, 13, 10)
        sel = _get(bits, 23, 6)
        cstart = 29
        if sel & 3 == 0:
            cems = [sel >> 2] * parts
        else:
            extra = 3 * parts - 4
            below -= extra
            sel |= _get(bits, below, extra) << 6
            base = (sel & 3) - 1
            cems = [((base + ((sel >> (2 + p)) & 1)) << 2) | ((sel >> (2 + parts + 2 * p)) & 3) for p in range(parts)]
    ccs = 0
    if dual:
        below -= 2
        ccs = _get(bits, below, 2)
    nv = sum(2 * ((c >> 2) + 1) for c in cems)
    cr = colour_range(nv, below - cstart)
    if cr < 0:
        return None
    colours = ise_decode(bits[cstart:cstart + ise_bits(nv, cr)], nv, cr)
    blk = Block(w, h, wr, weights, cems, colours, seed, dual, ccs)
    blk.crange = cr
    return blk


def colour_bits_available(b: Block) -> int:
    """Bits between the colour data's start and the bits below the weights
    (extra endpoint-mode bits, dual-plane selector) for block fields b."""
    count = b.w * b.h * (b.dual + 1)
    below = 128 - ise_bits(count, b.wrange)
    if b.parts > 1 and len(set(b.cems)) > 1:
        below -= 3 * b.parts - 4
    if b.dual:
        below -= 2
    return below - (17 if b.parts == 1 else 29)


def _bit_transfer(a: int, b: int):
    """Spec's bit transfer for base+offset modes: (offset a, base b) ->
    (signed 6-bit offset, base)."""
    b = (b >> 1) | (a & 0x80)
    a = (a >> 1) & 0x3F
    return (a - 0x40 if a & 0x20 else a), b


def _clamp(v):
    return max(0, min(255, v))


def spec_endpoints(cem: int, v):
    """LDR endpoint pair (e0, e1), RGBA bytes each, of endpoint mode `cem` from
    its unquantised colour values v (spec: "LDR Endpoint Decoding"); None for
    HDR modes."""
    if cem == 0:
        return [v[0]] * 3 + [255], [v[1]] * 3 + [255]
    if cem == 1:
        l0 = (v[0] >> 2) | (v[1] & 0xC0)
        l1 = min(l0 + (v[1] & 0x3F), 255)
        return [l0] * 3 + [255], [l1] * 3 + [255]
    if cem == 4:
        return [v[0]] * 3 + [v[2]], [v[1]] * 3 + [v[3]]
    if cem == 5:
        d, l0 = _bit_transfer(v[1], v[0])
        da, a0 = _bit_transfer(v[3], v[2])
        return [l0] * 3 + [a0], [_clamp(l0 + d)] * 3 + [_clamp(a0 + da)]
    if cem in (6, 10):
        s = v[3]
        a0, a1 = (v[4], v[5]) if cem == 10 else (255, 255)
        return [(v[0] * s) >> 8, (v[1] * s) >> 8, (v[2] * s) >> 8, a0], [v[0], v[1], v[2], a1]
    if cem in (8, 12):
        a0, a1 = (v[6], v[7]) if cem == 12 else (255, 255)
        if v[1] + v[3] + v[5] >= v[0] + v[2] + v[4]:
            return [v[0], v[2], v[4], a0], [v[1], v[3], v[5], a1]
        # Swapped, with blue contraction: r = (r + b) >> 1, g = (g + b) >> 1.
        return ([(v[1] + v[5]) >> 1, (v[3] + v[5]) >> 1, v[5], a1],
                [(v[0] + v[4]) >> 1, (v[2] + v[4]) >> 1, v[4], a0])
    if cem in (9, 13):
        pairs = [_bit_transfer(v[2 * c + 1], v[2 * c]) for c in range(3)]
        if cem == 13:
            pairs.append(_bit_transfer(v[7], v[6]))
        else:
            pairs.append((0, 255))
        base = [b for _, b in pairs]
        summed = [b + d for d, b in pairs]
        if sum(d for d, _ in pairs[:3]) >= 0:
            e0, e1 = base, summed
        else:
            e0 = [(summed[0] + summed[2]) >> 1, (summed[1] + summed[2]) >> 1, summed[2], summed[3]]
            e1 = [(base[0] + base[2]) >> 1, (base[1] + base[2]) >> 1, base[2], base[3]]
        return [_clamp(x) for x in e0], [_clamp(x) for x in e1]
    return None
