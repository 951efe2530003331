/*
 * ORACLE — test infrastructure only. Nothing in the product links, loads or
 * calls this file; only tests/, __graft_entry__.smoke() and bench.py's CPU
 * baseline leg use it, and only to check results or as the timed CPU baseline.
 *
 * CPU restatement of ASTC LDR block decoding as performed by Arm astcenc 5.7.0
 * (ARM-software/astc-encoder, tag 5.7.0, Apache-2.0), the codec the reference
 * binds in astc_kv/bridge.cpp:27-35 (akv_decode -> astcenc_decompress_image)
 * and calls from astc_kv/codec.py:56. astcenc's source is not vendored in the
 * reference (.gitignore:6,34; fetched by scripts/download_dependencies.py:37),
 * so this is written from the published Khronos Data Format Specification,
 * ASTC chapter, not from astcenc's code. It deliberately uses the plain
 * per-field spec formulation (a serial bit reader, full integer-sequence
 * decode, formula unquantization, the spec's partition hash) so that it is
 * structurally independent of the table-driven product decoder.
 *
 * Output contract (pinned by the reference's archived fixtures, see tests):
 * each texel channel is a UNORM16 value C = (e0*(64-w) + e1*w + 32) >> 6 on
 * 16-bit endpoints e = e8*257, returned to the caller as an FP16 bit pattern:
 * C == 0xFFFF -> 1.0, otherwise C/65536 truncated toward zero to FP16.
 *
 * Scope: 2D LDR blocks. HDR endpoint modes and HDR void-extent blocks decode
 * to the LDR error colour (magenta); so do reserved/invalid encodings.
 *
 * Pinned against astcenc's archived outputs (the reference's fixtures): 6x6
 * blocks with endpoint modes 0/1, 1-4 partitions, reduced weight grids,
 * trit/quint weights, colour ranges of 10 to 256 levels (all but 16), and the
 * UNORM16 -> FP16 rule. Pinned by reduction to those blocks (tests/test_oracle_reductions.py,
 * with a specification-written block writer that is itself checked against
 * every archived block): endpoint modes 1 and 4-13 (direct, swapped with blue
 * contraction, bit transfer, base+scale, alpha pairs, partitions mixing
 * endpoint classes), dual-plane blocks, identity weight grids and reduced
 * grids of every footprint up to 64 texels. Pinned by closed forms: trit/quint
 * block codes, integer-sequence bit counts, unquantisation levels, void
 * extent, small-block partition coordinates. Each of eleven planted mistakes
 * (missing blue contraction, 5-bit offsets, swapped planes, swapped alpha
 * pairs, ...) fails at least one of these tests.
 * PARITY UNPINNED (no astcenc vector, no reduction reaches them): HDR modes
 * (decode to the error colour); the partition hash at coordinates above 5
 * (footprints under 31 texels, such as 6x5, evaluate it at doubled
 * coordinates up to (10, 8); the same arithmetic as the pinned 0..5); which
 * colour channel each endpoint value feeds (the specification's table;
 * luminance data cannot tell channels apart); colour unquantisation of the
 * 6-, 8- and 16-level ranges and weight unquantisation of the 12-, 20-, 24-
 * and 32-level ranges, which astcenc never chose on the archived data (closed
 * forms only).
 */
#include <stdint.h>
#include <string.h>

#define ORACLE_KIND_NORMAL 0
#define ORACLE_KIND_VOID 1
#define ORACLE_KIND_ERROR 2

/* ---- bit reader: little-endian bit order within the 128-bit block ---- */
static unsigned rd(const uint8_t *blk, int pos, int count)
{
    unsigned v = 0;
    for (int i = 0; i < count; i++) {
        int p = pos + i;
        if (p >= 0 && p < 128)
            v |= (unsigned)((blk[p >> 3] >> (p & 7)) & 1) << i;
    }
    return v;
}

/* ---- integer sequence encoding: (bits, trits, quints) per range ---- */
static const int ISE_BITS[21] = {1, 0, 2, 0, 1, 3, 1, 2, 4, 2, 3, 5, 3, 4, 6, 4, 5, 7, 5, 6, 8};
static const int ISE_TRIT[21] = {0, 1, 0, 0, 1, 0, 0, 1, 0, 0, 1, 0, 0, 1, 0, 0, 1, 0, 0, 1, 0};
static const int ISE_QUINT[21] = {0, 0, 0, 1, 0, 0, 1, 0, 0, 1, 0, 0, 1, 0, 0, 1, 0, 0, 1, 0, 0};
/* number of levels of each range, for reference: 2 3 4 5 6 8 10 12 16 20 24 32
   40 48 64 80 96 128 160 192 256 */

int oracle_ise_bits(int count, int range)
{
    int n = ISE_BITS[range];
    if (ISE_TRIT[range])
        return count * n + (8 * count + 4) / 5;
    if (ISE_QUINT[range])
        return count * n + (7 * count + 2) / 3;
    return count * n;
}

/* Trit block decode, spec "Integer Sequence Encoding": 8 bits -> 5 trits. */
void oracle_decode_trits(unsigned T, int t[5])
{
    unsigned C;
    int t3, t4;
    if (((T >> 2) & 7) == 7) {
        C = (((T >> 5) & 7) << 2) | (T & 3);
        t4 = 2;
        t3 = 2;
    } else {
        C = T & 0x1F;
        if (((T >> 5) & 3) == 3) {
            t4 = 2;
            t3 = (T >> 7) & 1;
        } else {
            t4 = (T >> 7) & 1;
            t3 = (T >> 5) & 3;
        }
    }
    unsigned c0 = C & 1, c1 = (C >> 1) & 1, c2 = (C >> 2) & 1, c3 = (C >> 3) & 1, c4 = (C >> 4) & 1;
    if ((C & 3) == 3) {
        t[2] = 2;
        t[1] = c4;
        t[0] = (c3 << 1) | (c2 & (c3 ^ 1));
    } else if (((C >> 2) & 3) == 3) {
        t[2] = 2;
        t[1] = 2;
        t[0] = C & 3;
    } else {
        t[2] = c4;
        t[1] = (C >> 2) & 3;
        t[0] = (c1 << 1) | (c0 & (c1 ^ 1));
    }
    t[3] = t3;
    t[4] = t4;
}

/* Quint block decode: 7 bits -> 3 quints. */
void oracle_decode_quints(unsigned Q, int q[3])
{
    unsigned q0b = Q & 1, q3b = (Q >> 3) & 1, q4b = (Q >> 4) & 1;
    if (((Q >> 1) & 3) == 3 && ((Q >> 5) & 3) == 0) {
        q[2] = (int)((q0b << 2) | ((q4b & (q0b ^ 1)) << 1) | (q3b & (q0b ^ 1)));
        q[1] = 4;
        q[0] = 4;
        return;
    }
    unsigned C;
    if (((Q >> 1) & 3) == 3) {
        q[2] = 4;
        C = (((Q >> 3) & 3) << 3) | ((~(Q >> 5) & 3) << 1) | q0b;
    } else {
        q[2] = (Q >> 5) & 3;
        C = Q & 0x1F;
    }
    if ((C & 7) == 5) {
        q[1] = 4;
        q[0] = (C >> 3) & 3;
    } else {
        q[1] = (C >> 3) & 3;
        q[0] = C & 7;
    }
}

/* Decode `count` values of range `range` starting at bit `pos` of `blk`.
   Only the chunks belonging to values that are present are read, so the
   trailing, absent part of a partial trit/quint block reads as zero. */
static void ise_decode(const uint8_t *blk, int pos, int count, int range, int *out)
{
    int n = ISE_BITS[range];
    if (ISE_TRIT[range]) {
        static const int tbits[5] = {2, 2, 1, 2, 1};
        static const int tshift[5] = {0, 2, 4, 5, 7};
        for (int g = 0; g < count; g += 5) {
            int m[5] = {0, 0, 0, 0, 0}, t[5];
            unsigned T = 0;
            for (int j = 0; j < 5 && g + j < count; j++) {
                m[j] = (int)rd(blk, pos, n);
                pos += n;
                T |= rd(blk, pos, tbits[j]) << tshift[j];
                pos += tbits[j];
            }
            oracle_decode_trits(T, t);
            for (int j = 0; j < 5 && g + j < count; j++)
                out[g + j] = (t[j] << n) | m[j];
        }
    } else if (ISE_QUINT[range]) {
        static const int qbits[3] = {3, 2, 2};
        static const int qshift[3] = {0, 3, 5};
        for (int g = 0; g < count; g += 3) {
            int m[3] = {0, 0, 0}, q[3];
            unsigned Q = 0;
            for (int j = 0; j < 3 && g + j < count; j++) {
                m[j] = (int)rd(blk, pos, n);
                pos += n;
                Q |= rd(blk, pos, qbits[j]) << qshift[j];
                pos += qbits[j];
            }
            oracle_decode_quints(Q, q);
            for (int j = 0; j < 3 && g + j < count; j++)
                out[g + j] = (q[j] << n) | m[j];
        }
    } else {
        for (int i = 0; i < count; i++) {
            out[i] = (int)rd(blk, pos, n);
            pos += n;
        }
    }
}

/* ---- unquantization (spec "Color Endpoint Unquantization" / "Weight
   Unquantization"): A/B/C/D bit-pattern formulation ---- */
static int replicate(int v, int n, int to)
{
    int r = 0, have = 0;
    while (have < to) {
        int take = n < to - have ? n : to - have;
        r = (r << take) | (v >> (n - take));
        have += take;
    }
    return r;
}

int oracle_unquant_color(int range, int v)
{
    int n = ISE_BITS[range];
    if (!ISE_TRIT[range] && !ISE_QUINT[range])
        return replicate(v, n, 8);
    int a = v & 1, b = (v >> 1) & 1, c = (v >> 2) & 1, d = (v >> 3) & 1, e = (v >> 4) & 1, f = (v >> 5) & 1;
    int A = a ? 0x1FF : 0, B = 0, C = 0, D = v >> n;
    if (ISE_TRIT[range]) {
        switch (n) {
        case 1: B = 0; C = 204; break;                                                    /* 000000000 */
        case 2: B = (b << 8) | (b << 4) | (b << 2) | (b << 1); C = 93; break;              /* b000b0bb0 */
        case 3: B = (c << 8) | (b << 7) | (c << 3) | (b << 2) | (c << 1) | b; C = 44; break; /* cb000cbcb */
        case 4: B = (d << 8) | (c << 7) | (b << 6) | (d << 2) | (c << 1) | b; C = 22; break; /* dcb000dcb */
        case 5: B = (e << 8) | (d << 7) | (c << 6) | (b << 5) | (e << 1) | d; C = 11; break; /* edcb000ed */
        case 6: B = (f << 8) | (e << 7) | (d << 6) | (c << 5) | (b << 4) | f; C = 5; break;  /* fedcb000f */
        default: return -1;
        }
    } else {
        switch (n) {
        case 1: B = 0; C = 113; break;                                                    /* 000000000 */
        case 2: B = (b << 8) | (b << 3) | (b << 2); C = 54; break;                         /* b0000bb00 */
        case 3: B = (c << 8) | (b << 7) | (c << 2) | (b << 1) | c; C = 26; break;          /* cb0000cbc */
        case 4: B = (d << 8) | (c << 7) | (b << 6) | (d << 1) | c; C = 13; break;          /* dcb0000dc */
        case 5: B = (e << 8) | (d << 7) | (c << 6) | (b << 5) | e; C = 6; break;           /* edcb0000e */
        default: return -1;
        }
    }
    int T = D * C + B;
    T ^= A;
    return (A & 0x80) | (T >> 2);
}

int oracle_unquant_weight(int range, int v)
{
    int n = ISE_BITS[range], r;
    if (!ISE_TRIT[range] && !ISE_QUINT[range]) {
        r = replicate(v, n, 6);
    } else if (n == 0) {
        static const int t0[3] = {0, 32, 63}, q0[5] = {0, 16, 32, 47, 63};
        r = ISE_TRIT[range] ? t0[v] : q0[v];
    } else {
        int a = v & 1, b = (v >> 1) & 1, c = (v >> 2) & 1;
        int A = a ? 0x7F : 0, B = 0, C = 0, D = v >> n;
        if (ISE_TRIT[range]) {
            if (n == 1) { B = 0; C = 50; }                                       /* 0000000 */
            else if (n == 2) { B = (b << 6) | (b << 2) | b; C = 23; }            /* b000b0b */
            else { B = (c << 6) | (b << 5) | (c << 1) | b; C = 11; }             /* cb000cb */
        } else {
            if (n == 1) { B = 0; C = 28; }                                       /* 0000000 */
            else { B = (b << 6) | (b << 1); C = 13; }                            /* b0000b0 */
        }
        r = (D * C + B) ^ A;
        r = (A & 0x20) | (r >> 2);
    }
    if (r > 32)
        r++;
    return r;
}

/* ---- block mode (spec "Block Mode" table, 2D) ---- */
typedef struct {
    int gw, gh, dual, range, bits;
} mode_t_;

static int decode_mode(unsigned m, mode_t_ *o)
{
    int R = (m >> 4) & 1, H = (m >> 9) & 1, D = (m >> 10) & 1;
    int A = (m >> 5) & 3, B;
    int W, Hh;
    if (m & 3) {
        R |= (int)(m & 3) << 1;
        B = (m >> 7) & 3;
        switch ((m >> 2) & 3) {
        case 0: W = B + 4; Hh = A + 2; break;
        case 1: W = B + 8; Hh = A + 2; break;
        case 2: W = A + 2; Hh = B + 8; break;
        default:
            B &= 1;
            if (m & 0x100) { W = B + 2; Hh = A + 2; }
            else { W = A + 2; Hh = B + 6; }
            break;
        }
    } else {
        R |= (int)((m >> 2) & 3) << 1;
        if (((m >> 2) & 3) == 0)
            return 0;
        B = (m >> 9) & 3;
        switch ((m >> 7) & 3) {
        case 0: W = 12; Hh = A + 2; break;
        case 1: W = A + 2; Hh = 12; break;
        case 2: W = A + 6; Hh = B + 6; D = 0; H = 0; break;
        default:
            if (A == 0) { W = 6; Hh = 10; }
            else if (A == 1) { W = 10; Hh = 6; }
            else return 0;
            break;
        }
    }
    int count = W * Hh * (D + 1);
    o->gw = W;
    o->gh = Hh;
    o->dual = D;
    o->range = (R - 2) + 6 * H;
    o->bits = oracle_ise_bits(count, o->range);
    return count <= 64 && o->bits >= 24 && o->bits <= 96;
}

/* ---- spec partition hash and selection function ---- */
static uint32_t hash52(uint32_t p)
{
    p ^= p >> 15;
    p -= p << 17;
    p += p << 7;
    p += p << 4;
    p ^= p >> 5;
    p += p << 16;
    p ^= p >> 7;
    p ^= p >> 3;
    p ^= p << 6;
    p ^= p >> 17;
    return p;
}

int oracle_select_partition(int seed, int x, int y, int z, int count, int small_block)
{
    if (small_block) {
        x <<= 1;
        y <<= 1;
        z <<= 1;
    }
    seed += (count - 1) * 1024;
    uint32_t r = hash52((uint32_t)seed);
    uint8_t s1 = r & 0xF, s2 = (r >> 4) & 0xF, s3 = (r >> 8) & 0xF, s4 = (r >> 12) & 0xF;
    uint8_t s5 = (r >> 16) & 0xF, s6 = (r >> 20) & 0xF, s7 = (r >> 24) & 0xF, s8 = (r >> 28) & 0xF;
    uint8_t s9 = (r >> 18) & 0xF, s10 = (r >> 22) & 0xF, s11 = (r >> 26) & 0xF;
    uint8_t s12 = ((r >> 30) | (r << 2)) & 0xF;
    s1 *= s1; s2 *= s2; s3 *= s3; s4 *= s4; s5 *= s5; s6 *= s6;
    s7 *= s7; s8 *= s8; s9 *= s9; s10 *= s10; s11 *= s11; s12 *= s12;
    int sh1, sh2, sh3;
    if (seed & 1) {
        sh1 = (seed & 2) ? 4 : 5;
        sh2 = (count == 3) ? 6 : 5;
    } else {
        sh1 = (count == 3) ? 6 : 5;
        sh2 = (seed & 2) ? 4 : 5;
    }
    sh3 = (seed & 0x10) ? sh1 : sh2;
    s1 >>= sh1; s2 >>= sh2; s3 >>= sh1; s4 >>= sh2;
    s5 >>= sh1; s6 >>= sh2; s7 >>= sh1; s8 >>= sh2;
    s9 >>= sh3; s10 >>= sh3; s11 >>= sh3; s12 >>= sh3;
    int a = s1 * x + s2 * y + s11 * z + (int)(r >> 14);
    int b = s3 * x + s4 * y + s12 * z + (int)(r >> 10);
    int c = s5 * x + s6 * y + s9 * z + (int)(r >> 6);
    int d = s7 * x + s8 * y + s10 * z + (int)(r >> 2);
    a &= 0x3F; b &= 0x3F; c &= 0x3F; d &= 0x3F;
    if (count <= 3) d = 0;
    if (count <= 2) c = 0;
    if (count <= 1) b = 0;
    if (a >= b && a >= c && a >= d) return 0;
    if (b >= c && b >= d) return 1;
    if (c >= d) return 2;
    return 3;
}

/* ---- colour endpoint modes (LDR) ---- */
static void bit_transfer_signed(int *a, int *b)
{
    *b = (*b >> 1) | (*a & 0x80);
    *a = (*a >> 1) & 0x3F;
    if (*a & 0x20)
        *a -= 0x40;
}

static int clamp8(int v) { return v < 0 ? 0 : (v > 255 ? 255 : v); }

static void blue_contract(int c[4])
{
    c[0] = (c[0] + c[2]) >> 1;
    c[1] = (c[1] + c[2]) >> 1;
}

/* Returns 0 for an LDR mode (endpoints written), 1 for an HDR mode. */
static int decode_endpoints(int cem, const int *v, int e0[4], int e1[4])
{
    switch (cem) {
    case 0:
        e0[0] = e0[1] = e0[2] = v[0]; e0[3] = 255;
        e1[0] = e1[1] = e1[2] = v[1]; e1[3] = 255;
        return 0;
    case 1: {
        int L0 = (v[0] >> 2) | (v[1] & 0xC0);
        int L1 = L0 + (v[1] & 0x3F);
        if (L1 > 255) L1 = 255;
        e0[0] = e0[1] = e0[2] = L0; e0[3] = 255;
        e1[0] = e1[1] = e1[2] = L1; e1[3] = 255;
        return 0;
    }
    case 4:
        e0[0] = e0[1] = e0[2] = v[0]; e0[3] = v[2];
        e1[0] = e1[1] = e1[2] = v[1]; e1[3] = v[3];
        return 0;
    case 5: {
        int v0 = v[0], v1 = v[1], v2 = v[2], v3 = v[3];
        bit_transfer_signed(&v1, &v0);
        bit_transfer_signed(&v3, &v2);
        e0[0] = e0[1] = e0[2] = v0; e0[3] = v2;
        e1[0] = e1[1] = e1[2] = clamp8(v0 + v1); e1[3] = clamp8(v2 + v3);
        return 0;
    }
    case 6:
        e0[0] = (v[0] * v[3]) >> 8; e0[1] = (v[1] * v[3]) >> 8; e0[2] = (v[2] * v[3]) >> 8; e0[3] = 255;
        e1[0] = v[0]; e1[1] = v[1]; e1[2] = v[2]; e1[3] = 255;
        return 0;
    case 8:
    case 12: {
        int alpha0 = cem == 12 ? v[6] : 255, alpha1 = cem == 12 ? v[7] : 255;
        int s0 = v[0] + v[2] + v[4], s1 = v[1] + v[3] + v[5];
        if (s1 >= s0) {
            e0[0] = v[0]; e0[1] = v[2]; e0[2] = v[4]; e0[3] = alpha0;
            e1[0] = v[1]; e1[1] = v[3]; e1[2] = v[5]; e1[3] = alpha1;
        } else {
            e0[0] = v[1]; e0[1] = v[3]; e0[2] = v[5]; e0[3] = alpha1;
            e1[0] = v[0]; e1[1] = v[2]; e1[2] = v[4]; e1[3] = alpha0;
            blue_contract(e0);
            blue_contract(e1);
        }
        return 0;
    }
    case 9:
    case 13: {
        int r0 = v[0], r1 = v[1], g0 = v[2], g1 = v[3], b0 = v[4], b1 = v[5];
        int a0 = cem == 13 ? v[6] : 255, a1 = cem == 13 ? v[7] : 0;
        bit_transfer_signed(&r1, &r0);
        bit_transfer_signed(&g1, &g0);
        bit_transfer_signed(&b1, &b0);
        if (cem == 13)
            bit_transfer_signed(&a1, &a0);
        if (r1 + g1 + b1 >= 0) {
            e0[0] = r0; e0[1] = g0; e0[2] = b0; e0[3] = a0;
            e1[0] = r0 + r1; e1[1] = g0 + g1; e1[2] = b0 + b1; e1[3] = a0 + a1;
        } else {
            e0[0] = r0 + r1; e0[1] = g0 + g1; e0[2] = b0 + b1; e0[3] = a0 + a1;
            e1[0] = r0; e1[1] = g0; e1[2] = b0; e1[3] = a0;
            blue_contract(e0);
            blue_contract(e1);
        }
        for (int i = 0; i < 4; i++) {
            e0[i] = clamp8(e0[i]);
            e1[i] = clamp8(e1[i]);
        }
        return 0;
    }
    case 10:
        e0[0] = (v[0] * v[3]) >> 8; e0[1] = (v[1] * v[3]) >> 8; e0[2] = (v[2] * v[3]) >> 8; e0[3] = v[4];
        e1[0] = v[0]; e1[1] = v[1]; e1[2] = v[2]; e1[3] = v[5];
        return 0;
    default:
        return 1; /* 2, 3, 7, 11, 14, 15: HDR */
    }
}

uint16_t oracle_unorm16_to_fp16(unsigned c)
{
    if (c == 0xFFFF)
        return 0x3C00;
    if (c < 4)
        return (uint16_t)(c << 8); /* FP16 subnormal c * 2^-16 */
    int msb = 15;
    while (!((c >> msb) & 1))
        msb--;
    /* c * 2^-16 lies in [2^(msb-16), 2^(msb-15)): biased exponent msb - 1;
       the ten bits below the leading one are kept, the rest truncated. */
    unsigned frac = msb >= 10 ? (c >> (msb - 10)) & 0x3FF : (c << (10 - msb)) & 0x3FF;
    return (uint16_t)(((unsigned)(msb - 1) << 10) | frac);
}

static void fill_error(int bx, int by, uint16_t *out)
{
    for (int i = 0; i < bx * by; i++) {
        out[4 * i + 0] = 0xFFFF;
        out[4 * i + 1] = 0;
        out[4 * i + 2] = 0xFFFF;
        out[4 * i + 3] = 0xFFFF;
    }
}

/* Decode one block to UNORM16 RGBA texels, row-major [by][bx][4].
   Returns the block kind. */
int oracle_decode_block_unorm16(const uint8_t *blk, int bx, int by, uint16_t *out)
{
    unsigned mode = rd(blk, 0, 11);
    int texels = bx * by;
    if ((mode & 0x1FF) == 0x1FC) {
        int hdr = rd(blk, 9, 1);
        unsigned s0 = rd(blk, 12, 13), s1 = rd(blk, 25, 13), t0 = rd(blk, 38, 13), t1 = rd(blk, 51, 13);
        int all_ones = s0 == 0x1FFF && s1 == 0x1FFF && t0 == 0x1FFF && t1 == 0x1FFF;
        if (hdr || (!all_ones && (s0 >= s1 || t0 >= t1))) {
            fill_error(bx, by, out);
            return ORACLE_KIND_ERROR;
        }
        for (int i = 0; i < texels; i++)
            for (int ch = 0; ch < 4; ch++)
                out[4 * i + ch] = (uint16_t)rd(blk, 64 + 16 * ch, 16);
        return ORACLE_KIND_VOID;
    }
    mode_t_ m;
    if (!decode_mode(mode, &m) || m.gw > bx || m.gh > by) {
        fill_error(bx, by, out);
        return ORACLE_KIND_ERROR;
    }
    int parts = (int)rd(blk, 11, 2) + 1;
    if (m.dual && parts == 4) {
        fill_error(bx, by, out);
        return ORACLE_KIND_ERROR;
    }
    int cem[4] = {0, 0, 0, 0};
    int seed = 0, config_start, below = 128 - m.bits;
    if (parts == 1) {
        cem[0] = (int)rd(blk, 13, 4);
        config_start = 17;
    } else {
        seed = (int)rd(blk, 13, 10);
        unsigned field = rd(blk, 23, 6);
        config_start = 29;
        if ((field & 3) == 0) {
            for (int p = 0; p < parts; p++)
                cem[p] = (int)(field >> 2);
        } else {
            int extra = 3 * parts - 4;
            below -= extra;
            unsigned enc = field | (rd(blk, below, extra) << 6);
            int base = (int)(enc & 3) - 1;
            for (int p = 0; p < parts; p++) {
                int cls = (int)((enc >> (2 + p)) & 1);
                int mm = (int)((enc >> (2 + parts + 2 * p)) & 3);
                cem[p] = ((base + cls) << 2) | mm;
            }
        }
    }
    int ccs = 0;
    if (m.dual) {
        below -= 2;
        ccs = (int)rd(blk, below, 2);
    }
    int nvals = 0;
    for (int p = 0; p < parts; p++)
        nvals += 2 * ((cem[p] >> 2) + 1);
    int avail = below - config_start;
    int crange = -1;
    if (nvals <= 18 && avail > 0)
        for (int r = 20; r >= 0; r--)
            if (oracle_ise_bits(nvals, r) <= avail) {
                crange = r;
                break;
            }
    if (nvals > 18 || crange < 4) { /* range index 4 = 6 levels */
        fill_error(bx, by, out);
        return ORACLE_KIND_ERROR;
    }
    int cv[18];
    ise_decode(blk, config_start, nvals, crange, cv);
    for (int i = 0; i < nvals; i++)
        cv[i] = oracle_unquant_color(crange, cv[i]);
    int ep0[4][4], ep1[4][4], ep_hdr[4];
    for (int p = 0, k = 0; p < parts; p++) {
        ep_hdr[p] = decode_endpoints(cem[p], cv + k, ep0[p], ep1[p]);
        k += 2 * ((cem[p] >> 2) + 1);
    }
    /* weights: integer sequence read from the bit-reversed block */
    uint8_t rev[16];
    for (int i = 0; i < 16; i++) {
        uint8_t b = blk[15 - i], r = 0;
        for (int k = 0; k < 8; k++)
            r |= (uint8_t)(((b >> k) & 1) << (7 - k));
        rev[i] = r;
    }
    int nw = m.gw * m.gh * (m.dual + 1);
    int wq[160], wu[160]; /* zero padding: infill taps with a zero factor may index past the grid */
    memset(wq, 0, sizeof(wq));
    memset(wu, 0, sizeof(wu));
    ise_decode(rev, 0, nw, m.range, wq);
    for (int i = 0; i < nw; i++)
        wu[i] = oracle_unquant_weight(m.range, wq[i]);
    /* weight infill: grid -> texels (spec "Weight Infill") */
    int Ds = (1024 + bx / 2) / (bx - 1), Dt = (1024 + by / 2) / (by - 1);
    int planes = m.dual + 1;
    int small = texels < 31;
    for (int t = 0; t < by; t++) {
        for (int s = 0; s < bx; s++) {
            int w[2] = {0, 0};
            for (int pl = 0; pl < planes; pl++) {
                int cs = Ds * s, ct = Dt * t;
                int gs = (cs * (m.gw - 1) + 32) >> 6, gt = (ct * (m.gh - 1) + 32) >> 6;
                int js = gs >> 4, fs = gs & 15, jt = gt >> 4, ft = gt & 15;
                int v0 = js + jt * m.gw;
                int w11 = (fs * ft + 8) >> 4, w10 = ft - w11, w01 = fs - w11, w00 = 16 - fs - ft + w11;
                int i00 = v0, i01 = v0 + 1, i10 = v0 + m.gw, i11 = v0 + m.gw + 1;
                int p00 = wu[i00 * planes + pl], p01 = wu[i01 * planes + pl];
                int p10 = wu[i10 * planes + pl], p11 = wu[i11 * planes + pl];
                w[pl] = (p00 * w00 + p01 * w01 + p10 * w10 + p11 * w11 + 8) >> 4;
            }
            int part = parts > 1 ? oracle_select_partition(seed, s, t, 0, parts, small) : 0;
            int i = t * bx + s;
            for (int ch = 0; ch < 4; ch++) {
                if (ep_hdr[part]) {
                    out[4 * i + ch] = (ch == 1) ? 0 : 0xFFFF;
                    continue;
                }
                int e0 = ep0[part][ch] * 257, e1 = ep1[part][ch] * 257;
                int ww = (m.dual && ch == ccs) ? w[1] : w[0];
                out[4 * i + ch] = (uint16_t)((e0 * (64 - ww) + e1 * ww + 32) >> 6);
            }
        }
    }
    return ORACLE_KIND_NORMAL;
}

int oracle_decode_block_fp16(const uint8_t *blk, int bx, int by, uint16_t *out)
{
    int kind = oracle_decode_block_unorm16(blk, bx, by, out);
    for (int i = 0; i < bx * by * 4; i++)
        out[i] = oracle_unorm16_to_fp16(out[i]);
    return kind;
}

/* Decode many independent blocks: out is [n][by][bx][4] FP16 bits. */
void oracle_decode_blocks_fp16(const uint8_t *blocks, long n, int bx, int by, uint16_t *out, int *kinds)
{
    for (long b = 0; b < n; b++) {
        int k = oracle_decode_block_fp16(blocks + 16 * b, bx, by, out + (long)b * bx * by * 4);
        if (kinds)
            kinds[b] = k;
    }
}

/* Decode a row-major block payload into an RGBA float image [h][w][4]
   (astcenc_decompress_image semantics with an F32 image and identity
   swizzle; reference call site astc_kv/bridge.cpp:27-35). */
int oracle_decode_image(const uint8_t *data, long bytes, int bx, int by, int w, int h, float *img)
{
    int cols = (w + bx - 1) / bx, rows = (h + by - 1) / by;
    if (bytes < (long)cols * rows * 16)
        return 1;
    uint16_t tex[12 * 12 * 4];
    for (int r = 0; r < rows; r++)
        for (int c = 0; c < cols; c++) {
            oracle_decode_block_fp16(data + 16L * (r * cols + c), bx, by, tex);
            for (int t = 0; t < by; t++)
                for (int s = 0; s < bx; s++) {
                    int y = r * by + t, x = c * bx + s;
                    if (y >= h || x >= w)
                        continue;
                    for (int ch = 0; ch < 4; ch++) {
                        uint16_t hbits = tex[4 * (t * bx + s) + ch];
                        /* FP16 -> FP32 (exact) */
                        unsigned sign = (hbits >> 15) & 1, ex = (hbits >> 10) & 31, fr = hbits & 0x3FF;
                        float f;
                        if (ex == 0)
                            f = (float)fr * (1.0f / 16777216.0f);
                        else if (ex == 31)
                            f = fr ? 0.0f / 0.0f : 1.0f / 0.0f;
                        else {
                            uint32_t u = ((ex - 15 + 127) << 23) | (fr << 13);
                            memcpy(&f, &u, 4);
                        }
                        img[((long)y * w + x) * 4 + ch] = sign ? -f : f;
                    }
                }
        }
    return 0;
}
