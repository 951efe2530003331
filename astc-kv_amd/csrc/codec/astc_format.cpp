// Table construction for the ASTC LDR decode (see astc_format.h).
#include "astc_format.h"

#include <array>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>

namespace akv {

namespace {

// Bit-pattern strings of the unquantisation "B" term, most significant bit
// first; '0' is a zero bit and 'b'..'f' copy bit 1..5 of the ISE value's plain
// part. Indexed by plain bit count (1..6 for colours, 1..3 for weights) with
// the multiplier C of the trit/quint digit.
struct Pattern {
    const char* bits;
    int c;
};
constexpr Pattern kColorTrit[7] = {{"", 0},           {"000000000", 204}, {"b000b0bb0", 93},
                                   {"cb000cbcb", 44}, {"dcb000dcb", 22},  {"edcb000ed", 11},
                                   {"fedcb000f", 5}};
constexpr Pattern kColorQuint[6] = {{"", 0},           {"000000000", 113}, {"b0000bb00", 54},
                                    {"cb0000cbc", 26}, {"dcb0000dc", 13},  {"edcb0000e", 6}};
constexpr Pattern kWeightTrit[4] = {{"", 0}, {"0000000", 50}, {"b000b0b", 23}, {"cb000cb", 11}};
constexpr Pattern kWeightQuint[3] = {{"", 0}, {"0000000", 28}, {"b0000b0", 13}};

int expand_pattern(const char* p, int value) {
    int r = 0;
    for (const char* s = p; *s; ++s) {
        int bit = *s == '0' ? 0 : (value >> (*s - 'a')) & 1;
        r = (r << 1) | bit;
    }
    return r;
}

// Replicate the n-bit value v into `width` bits (MSB-aligned repetition).
int replicate_bits(int v, int n, int width) {
    int r = 0;
    for (int filled = 0; filled < width; filled += n) {
        int shift = width - filled - n;
        r |= shift >= 0 ? v << shift : v >> -shift;
    }
    return r;
}

int unquant_digit(const Pattern& pat, int bits, int value, int width) {
    int digit = value >> bits;             // the trit or quint
    int mirror = (value & 1) ? (1 << width) - 1 : 0;
    int t = (digit * pat.c + expand_pattern(pat.bits, value)) ^ mirror;
    int top = 1 << (width - 2);            // 0x80 for colours, 0x20 for weights
    return (mirror & top) | (t >> 2);
}

}  // namespace

int ise_bits(int r) { return kIse[r].bits; }
bool ise_trit(int r) { return kIse[r].trit; }
bool ise_quint(int r) { return kIse[r].quint; }
int ise_levels(int r) { return (1 + 2 * kIse[r].trit + 4 * kIse[r].quint) << kIse[r].bits; }

int ise_sequence_bits(int count, int r) {
    int total = count * kIse[r].bits;
    if (kIse[r].trit) total += (count * 8 + 4) / 5;
    if (kIse[r].quint) total += (count * 7 + 2) / 3;
    return total;
}

int unquant_color(int r, int v) {
    const IseRange& e = kIse[r];
    if (!e.trit && !e.quint) return replicate_bits(v, e.bits, 8);
    const Pattern& p = e.trit ? kColorTrit[e.bits] : kColorQuint[e.bits];
    return unquant_digit(p, e.bits, v, 9);
}

int unquant_weight(int r, int v) {
    const IseRange& e = kIse[r];
    int w;
    if (!e.trit && !e.quint) {
        w = replicate_bits(v, e.bits, 6);
    } else if (e.bits == 0) {
        // A lone trit/quint spreads evenly over 0..63.
        w = e.trit ? (v * 63 + 1) / 2 : (v * 63 + 2) / 4;
    } else {
        const Pattern& p = e.trit ? kWeightTrit[e.bits] : kWeightQuint[e.bits];
        w = unquant_digit(p, e.bits, v, 7);
    }
    return w > 32 ? w + 1 : w;
}

void trits_from_block(unsigned T, int t[5]) {
    auto bit = [&](int i) { return int((T >> i) & 1); };
    unsigned c;
    if ((T & 0x1C) == 0x1C) {          // T[4:2] == 111
        c = ((T >> 3) & 0x1C) | (T & 3);
        t[4] = 2;
        t[3] = 2;
    } else {
        c = T & 0x1F;
        if ((T & 0x60) == 0x60) {
            t[4] = 2;
            t[3] = bit(7);
        } else {
            t[4] = bit(7);
            t[3] = (T >> 5) & 3;
        }
    }
    int c4 = (c >> 4) & 1, c3 = (c >> 3) & 1, c2 = (c >> 2) & 1, c1 = (c >> 1) & 1, c0 = c & 1;
    if ((c & 3) == 3) {
        t[2] = 2;
        t[1] = c4;
        t[0] = 2 * c3 + (c2 & ~c3 & 1);
    } else if ((c & 0xC) == 0xC) {
        t[2] = 2;
        t[1] = 2;
        t[0] = c & 3;
    } else {
        t[2] = c4;
        t[1] = (c >> 2) & 3;
        t[0] = 2 * c1 + (c0 & ~c1 & 1);
    }
}

void quints_from_block(unsigned Q, int q[3]) {
    int q0 = Q & 1, q3 = (Q >> 3) & 1, q4 = (Q >> 4) & 1;
    if ((Q & 6) == 6 && (Q & 0x60) == 0) {
        q[0] = 4;
        q[1] = 4;
        q[2] = 4 * q0 + 2 * (q4 & ~q0 & 1) + (q3 & ~q0 & 1);
        return;
    }
    unsigned c;
    if ((Q & 6) == 6) {
        q[2] = 4;
        c = (Q & 0x18) | ((~Q >> 4) & 6) | q0;
    } else {
        q[2] = (Q >> 5) & 3;
        c = Q & 0x1F;
    }
    if ((c & 7) == 5) {
        q[1] = 4;
        q[0] = (c >> 3) & 3;
    } else {
        q[1] = (c >> 3) & 3;
        q[0] = c & 7;
    }
}

uint32_t decode_block_mode(uint32_t m, int bx, int by) {
    if ((m & 0x1FF) == 0x1FC) return 0;  // void extent
    int r = (m >> 4) & 1, h = (m >> 9) & 1, d = (m >> 10) & 1;
    int a = (m >> 5) & 3;
    int gw, gh;
    if (m & 3) {
        r |= (m & 3) << 1;
        int b = (m >> 7) & 3;
        switch ((m >> 2) & 3) {
            case 0: gw = b + 4; gh = a + 2; break;
            case 1: gw = b + 8; gh = a + 2; break;
            case 2: gw = a + 2; gh = b + 8; break;
            default:
                if (m & 0x100) { gw = (b & 1) + 2; gh = a + 2; }
                else { gw = a + 2; gh = (b & 1) + 6; }
        }
    } else {
        if ((m & 0xC) == 0) return 0;    // reserved
        r |= ((m >> 2) & 3) << 1;
        int b = (m >> 9) & 3;
        switch ((m >> 7) & 3) {
            case 0: gw = 12; gh = a + 2; break;
            case 1: gw = a + 2; gh = 12; break;
            case 2: gw = a + 6; gh = b + 6; d = 0; h = 0; break;
            default:
                if (a > 1) return 0;
                gw = a ? 10 : 6;
                gh = a ? 6 : 10;
        }
    }
    int range = r - 2 + 6 * h;
    int count = gw * gh * (d + 1);
    int wbits = ise_sequence_bits(count, range);
    if (count > 64 || wbits < 24 || wbits > 96 || gw > bx || gh > by) return 0;
    uint32_t ident = (gw == bx && gh == by) ? 1u : 0u;
    return kModeValid | uint32_t(gw) | uint32_t(gh) << 4 | uint32_t(d) << 8 | uint32_t(range) << 9 |
           uint32_t(wbits) << 13 | ident << 20;
}

int partition_of(int seed, int x, int y, int count, bool small_block) {
    if (count <= 1) return 0;
    if (small_block) {
        x *= 2;
        y *= 2;
    }
    seed += (count - 1) * 1024;
    uint32_t h = uint32_t(seed);
    h ^= h >> 15;
    h *= 0xEEDE0891u;   // == (1 - 2^17)(1 + 2^7)(1 + 2^4) mod 2^32
    h ^= h >> 5;
    h += h << 16;
    h ^= h >> 7;
    h ^= h >> 3;
    h ^= h << 6;
    h ^= h >> 17;
    // Eight 4-bit seeds (the z-coordinate seeds are irrelevant in 2D), squared.
    int s[8];
    for (int i = 0; i < 8; ++i) {
        int v = (h >> (4 * i)) & 0xF;
        s[i] = v * v;
    }
    int sh_odd = (seed & 2) ? 4 : 5, sh_three = (count == 3) ? 6 : 5;
    int sh_x = (seed & 1) ? sh_odd : sh_three;   // applies to seeds 0,2,4,6
    int sh_y = (seed & 1) ? sh_three : sh_odd;   // applies to seeds 1,3,5,7
    int line[4];
    const int bias[4] = {int(h >> 14), int(h >> 10), int(h >> 6), int(h >> 2)};
    for (int k = 0; k < 4; ++k)
        line[k] = ((s[2 * k] >> sh_x) * x + (s[2 * k + 1] >> sh_y) * y + bias[k]) & 0x3F;
    for (int k = count; k < 4; ++k) line[k] = 0;
    int best = 0;
    for (int k = 1; k < 4; ++k)
        if (line[k] > line[best]) best = k;
    return best;
}

uint16_t unorm16_to_fp16_bits(uint32_t c) {
    if (c >= 0xFFFF) return 0x3C00;
    if (c < 4) return uint16_t(c << 8);
    int lead = 31 - __builtin_clz(c);   // 2..15
    uint32_t frac = lead >= 10 ? (c >> (lead - 10)) : (c << (10 - lead));
    return uint16_t(((lead - 1) << 10) | (frac & 0x3FF));
}

bool build_tables(int bx, int by, AkvTables* t) {
    if (bx < 4 || by < 4 || bx > 12 || by > 12 || bx * by > kMaxTexels) return false;
    std::memset(t, 0, sizeof(*t));
    t->block_x = uint32_t(bx);
    t->block_y = uint32_t(by);
    for (uint32_t m = 0; m < 2048; ++m) t->block_mode[m] = decode_block_mode(m, bx, by);
    const bool small = bx * by < 31;
    for (int pc = 2; pc <= 4; ++pc)
        for (int seed = 0; seed < 1024; ++seed)
            for (int y = 0; y < by; ++y)
                for (int x = 0; x < bx; ++x) {
                    int i = y * bx + x;
                    uint32_t p = uint32_t(partition_of(seed, x, y, pc, small));
                    t->partition[pc - 2][seed][i >> 4] |= p << (2 * (i & 15));
                }
    for (unsigned T = 0; T < 256; ++T) {
        int d[5];
        trits_from_block(T, d);
        uint16_t packed = 0;
        for (int j = 0; j < 5; ++j) packed |= uint16_t(d[j] << (2 * j));
        t->trit[T] = packed;
    }
    for (unsigned Q = 0; Q < 128; ++Q) {
        int d[3];
        quints_from_block(Q, d);
        t->quint[Q] = uint16_t(d[0] | d[1] << 3 | d[2] << 6);
    }
    for (int r = 0; r < kNumRanges; ++r)
        t->ise[r] = uint16_t(kIse[r].bits | kIse[r].trit << 8 | kIse[r].quint << 9);
    for (int r = 0; r < 12; ++r)
        for (int v = 0; v < ise_levels(r); ++v) t->weight_unq[r][v] = uint8_t(unquant_weight(r, v));
    for (int r = 0; r < 12; ++r) t->weight_levels[r] = uint8_t(ise_levels(r));
    for (int r = 0; r < kNumRanges; ++r)
        for (int v = 0; v < ise_levels(r); ++v) t->color_unq[r][v] = uint8_t(unquant_color(r, v));
    for (int pairs = 0; pairs < 10; ++pairs)
        for (int bits = 0; bits < 128; ++bits) {
            int best = -1;
            if (pairs > 0)
                for (int r = kNumRanges - 1; r >= 0 && best < 0; --r)
                    if (ise_sequence_bits(2 * pairs, r) <= bits) best = r;
            t->color_range[pairs][bits] = int8_t(best);
        }
    return true;
}

const AkvTables* tables_for(int bx, int by) {
    static std::mutex mu;
    static std::map<int, std::unique_ptr<AkvTables>> cache;
    std::lock_guard<std::mutex> lock(mu);
    int key = bx * 16 + by;
    auto it = cache.find(key);
    if (it != cache.end()) return it->second.get();
    auto t = std::make_unique<AkvTables>();
    if (!build_tables(bx, by, t.get())) return nullptr;
    const AkvTables* raw = t.get();
    cache.emplace(key, std::move(t));
    return raw;
}

}  // namespace akv
