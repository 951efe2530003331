// Table-driven CPU decode of ASTC LDR blocks (the akv_decode half of the
// bridge; reference binding astc_kv/bridge.cpp:27-35). The gfx950 kernels run
// the same steps per wavefront; both are checked against the oracle.
#include <algorithm>

#include "astc_bits.h"
#include "astc_codec.h"

namespace akv {

namespace {

// Unpack `count` integer-sequence values of `range` starting at bit `start`.
// A trit group is m0 T01 m1 T23 m2 T4 m3 T56 m4 T7 (5n+8 bits), a quint group
// m0 Q012 m1 Q34 m2 Q56 (3n+7 bits). Bits past the end of the sequence are
// treated as zero, which is how a truncated last group is defined.
void ise_unpack(const AkvTables& t, const Bits128& src, int start, int count, int range, int* out) {
    const int n = t.ise[range] & 0xFF;
    const bool trit = (t.ise[range] >> 8) & 1, quint = (t.ise[range] >> 9) & 1;
    const int end = start + ise_sequence_bits(count, range);
    const uint64_t mask = (uint64_t(1) << n) - 1;
    if (trit) {
        const int gbits = 5 * n + 8;
        const int moff[5] = {0, n + 2, 2 * n + 4, 3 * n + 5, 4 * n + 7};
        for (int i = 0, pos = start; i < count; i += 5, pos += gbits) {
            uint64_t g = src.get(pos, std::min(gbits, end - pos));
            unsigned T = unsigned((g >> n) & 3) | unsigned((g >> (2 * n + 2)) & 3) << 2 |
                         unsigned((g >> (3 * n + 4)) & 1) << 4 | unsigned((g >> (4 * n + 5)) & 3) << 5 |
                         unsigned((g >> (5 * n + 7)) & 1) << 7;
            unsigned digits = t.trit[T];
            for (int j = 0; j < 5 && i + j < count; ++j)
                out[i + j] = int(((digits >> (2 * j)) & 3) << n | ((g >> moff[j]) & mask));
        }
    } else if (quint) {
        const int gbits = 3 * n + 7;
        const int moff[3] = {0, n + 3, 2 * n + 5};
        for (int i = 0, pos = start; i < count; i += 3, pos += gbits) {
            uint64_t g = src.get(pos, std::min(gbits, end - pos));
            unsigned Q = unsigned((g >> n) & 7) | unsigned((g >> (2 * n + 3)) & 3) << 3 |
                         unsigned((g >> (3 * n + 5)) & 3) << 5;
            unsigned digits = t.quint[Q];
            for (int j = 0; j < 3 && i + j < count; ++j)
                out[i + j] = int(((digits >> (3 * j)) & 7) << n | ((g >> moff[j]) & mask));
        }
    } else {
        for (int i = 0; i < count; ++i) out[i] = int(src.get(start + i * n, n));
    }
}

inline int clamp255(int v) { return v < 0 ? 0 : (v > 255 ? 255 : v); }

// Signed base+offset transfer: the offset keeps a 6-bit two's complement
// value, its top bit moves into the base.
inline void transfer(int& offset, int& base) {
    base = (base >> 1) | (offset & 0x80);
    offset = (offset >> 1) & 0x3F;
    if (offset & 0x20) offset -= 0x40;
}

inline void blue_contract(int* e) {
    e[0] = (e[0] + e[2]) >> 1;
    e[1] = (e[1] + e[2]) >> 1;
}

// Eight-bit RGBA endpoints of one partition. False for HDR endpoint modes.
bool ldr_endpoints(int cem, const int* v, int* e0, int* e1) {
    auto rgba = [](int* e, int r, int g, int b, int a) {
        e[0] = r;
        e[1] = g;
        e[2] = b;
        e[3] = a;
    };
    switch (cem) {
        case 0:
            rgba(e0, v[0], v[0], v[0], 255);
            rgba(e1, v[1], v[1], v[1], 255);
            return true;
        case 1: {
            int l0 = (v[0] >> 2) | (v[1] & 0xC0);
            int l1 = std::min(l0 + (v[1] & 0x3F), 255);
            rgba(e0, l0, l0, l0, 255);
            rgba(e1, l1, l1, l1, 255);
            return true;
        }
        case 4:
            rgba(e0, v[0], v[0], v[0], v[2]);
            rgba(e1, v[1], v[1], v[1], v[3]);
            return true;
        case 5: {
            int l0 = v[0], dl = v[1], a0 = v[2], da = v[3];
            transfer(dl, l0);
            transfer(da, a0);
            int l1 = clamp255(l0 + dl);
            rgba(e0, l0, l0, l0, a0);
            rgba(e1, l1, l1, l1, clamp255(a0 + da));
            return true;
        }
        case 6:
        case 10: {
            int s = v[3];
            int a0 = cem == 10 ? v[4] : 255, a1 = cem == 10 ? v[5] : 255;
            rgba(e0, (v[0] * s) >> 8, (v[1] * s) >> 8, (v[2] * s) >> 8, a0);
            rgba(e1, v[0], v[1], v[2], a1);
            return true;
        }
        case 8:
        case 12: {
            int a0 = cem == 12 ? v[6] : 255, a1 = cem == 12 ? v[7] : 255;
            if (v[1] + v[3] + v[5] >= v[0] + v[2] + v[4]) {
                rgba(e0, v[0], v[2], v[4], a0);
                rgba(e1, v[1], v[3], v[5], a1);
            } else {
                rgba(e0, v[1], v[3], v[5], a1);
                rgba(e1, v[0], v[2], v[4], a0);
                blue_contract(e0);
                blue_contract(e1);
            }
            return true;
        }
        case 9:
        case 13: {
            int base[4] = {v[0], v[2], v[4], cem == 13 ? v[6] : 255};
            int off[4] = {v[1], v[3], v[5], cem == 13 ? v[7] : 0};
            for (int c = 0; c < (cem == 13 ? 4 : 3); ++c) transfer(off[c], base[c]);
            int sum[4];
            for (int c = 0; c < 4; ++c) sum[c] = base[c] + off[c];
            if (off[0] + off[1] + off[2] >= 0) {
                std::copy(base, base + 4, e0);
                std::copy(sum, sum + 4, e1);
            } else {
                std::copy(sum, sum + 4, e0);
                std::copy(base, base + 4, e1);
                blue_contract(e0);
                blue_contract(e1);
            }
            for (int c = 0; c < 4; ++c) {
                e0[c] = clamp255(e0[c]);
                e1[c] = clamp255(e1[c]);
            }
            return true;
        }
        default:
            return false;
    }
}

void error_block(const AkvTables& t, uint16_t* texels) {
    int n = int(t.block_x * t.block_y);
    for (int i = 0; i < n; ++i) {
        texels[4 * i + 0] = 0xFFFF;
        texels[4 * i + 1] = 0;
        texels[4 * i + 2] = 0xFFFF;
        texels[4 * i + 3] = 0xFFFF;
    }
}

}  // namespace

int decode_block_unorm16(const AkvTables& t, const uint8_t* block, uint16_t* texels) {
    const int bx = int(t.block_x), by = int(t.block_y), ntex = bx * by;
    const Bits128 b = Bits128::load(block);
    const uint32_t mode_bits = uint32_t(b.get(0, 11));
    if ((mode_bits & 0x1FF) == 0x1FC) {
        // Void extent: constant colour, UNORM16 RGBA in bits 64..127.
        bool hdr = b.get(9, 1);
        uint32_t s0 = uint32_t(b.get(12, 13)), s1 = uint32_t(b.get(25, 13));
        uint32_t t0 = uint32_t(b.get(38, 13)), t1 = uint32_t(b.get(51, 13));
        bool unbounded = (s0 & s1 & t0 & t1) == 0x1FFF;
        if (hdr || (!unbounded && (s0 >= s1 || t0 >= t1))) {
            error_block(t, texels);
            return kBlockError;
        }
        for (int i = 0; i < ntex; ++i)
            for (int c = 0; c < 4; ++c) texels[4 * i + c] = uint16_t(b.get(64 + 16 * c, 16));
        return kBlockVoid;
    }
    const uint32_t md = t.block_mode[mode_bits];
    const int parts = int(b.get(11, 2)) + 1;
    if (!md || (mode_dual(md) && parts == 4)) {
        error_block(t, texels);
        return kBlockError;
    }
    int cem[4] = {0, 0, 0, 0};
    int seed = 0, color_start = 17;
    int below = 128 - int(mode_wbits(md));
    if (parts == 1) {
        cem[0] = int(b.get(13, 4));
    } else {
        seed = int(b.get(13, 10));
        color_start = 29;
        uint32_t sel = uint32_t(b.get(23, 6));
        if ((sel & 3) == 0) {
            std::fill(cem, cem + parts, int(sel >> 2));
        } else {
            int extra = 3 * parts - 4;
            below -= extra;
            sel |= uint32_t(b.get(below, extra)) << 6;
            int base_class = int(sel & 3) - 1;
            for (int p = 0; p < parts; ++p) {
                int up = (sel >> (2 + p)) & 1;
                int low = (sel >> (2 + parts + 2 * p)) & 3;
                cem[p] = (base_class + up) * 4 + low;
            }
        }
    }
    int plane2_channel = -1;
    if (mode_dual(md)) {
        below -= 2;
        plane2_channel = int(b.get(below, 2));
    }
    int pairs = 0;
    for (int p = 0; p < parts; ++p) pairs += (cem[p] >> 2) + 1;
    const int avail = below - color_start;
    const int crange = (pairs <= 9 && avail > 0) ? t.color_range[pairs][std::min(avail, 127)] : -1;
    if (crange < kRange6) {
        error_block(t, texels);
        return kBlockError;
    }
    int vals[18];
    ise_unpack(t, b, color_start, 2 * pairs, crange, vals);
    for (int i = 0; i < 2 * pairs; ++i) vals[i] = t.color_unq[crange][vals[i]];
    // 16-bit endpoints (e8 * 257) and LDR flags per partition.
    // (HDR endpoint modes leave their endpoints unset: error texels.)
    int e0[4][4] = {}, e1[4][4] = {};
    bool ldr[4];
    for (int p = 0, k = 0; p < parts; ++p) {
        ldr[p] = ldr_endpoints(cem[p], vals + k, e0[p], e1[p]);
        k += 2 * ((cem[p] >> 2) + 1);
        for (int c = 0; c < 4 && ldr[p]; ++c) {
            e0[p][c] *= 257;
            e1[p][c] *= 257;
        }
    }
    // Grid weights, read from the bit-reversed block, then unquantised.
    const int gw = int(mode_gw(md)), gh = int(mode_gh(md)), planes = int(mode_dual(md)) + 1;
    const int wrange = int(mode_range(md));
    int grid[160] = {0};
    ise_unpack(t, b.reversed(), 0, gw * gh * planes, wrange, grid);
    for (int i = 0; i < gw * gh * planes; ++i) grid[i] = t.weight_unq[wrange][grid[i]];
    const int ds = (1024 + bx / 2) / (bx - 1), dt = (1024 + by / 2) / (by - 1);
    for (int y = 0; y < by; ++y) {
        for (int x = 0; x < bx; ++x) {
            const int i = y * bx + x;
            int w[2];
            if (mode_identity(md)) {
                for (int pl = 0; pl < planes; ++pl) w[pl] = grid[i * planes + pl];
            } else {
                int gs = (ds * x * (gw - 1) + 32) >> 6, gt = (dt * y * (gh - 1) + 32) >> 6;
                int fs = gs & 15, ft = gt & 15, base = (gs >> 4) + (gt >> 4) * gw;
                int f11 = (fs * ft + 8) >> 4;
                int f = 16 - fs - ft + f11, f01 = fs - f11, f10 = ft - f11;
                for (int pl = 0; pl < planes; ++pl) {
                    const int* g = grid + pl;
                    w[pl] = (g[base * planes] * f + g[(base + 1) * planes] * f01 +
                             g[(base + gw) * planes] * f10 + g[(base + gw + 1) * planes] * f11 + 8) >> 4;
                }
            }
            const int p = parts > 1 ? int((t.partition[parts - 2][seed][i >> 4] >> (2 * (i & 15))) & 3) : 0;
            for (int c = 0; c < 4; ++c) {
                if (!ldr[p]) {
                    texels[4 * i + c] = c == 1 ? 0 : 0xFFFF;
                    continue;
                }
                int ww = c == plane2_channel ? w[1] : w[0];
                texels[4 * i + c] = uint16_t((e0[p][c] * 64 + 32 + (e1[p][c] - e0[p][c]) * ww) >> 6);
            }
        }
    }
    return kBlockNormal;
}

int decode_block_fp16(const AkvTables& t, const uint8_t* block, uint16_t* texels) {
    int kind = decode_block_unorm16(t, block, texels);
    for (uint32_t i = 0; i < 4 * t.block_x * t.block_y; ++i) texels[i] = unorm16_to_fp16_bits(texels[i]);
    return kind;
}

namespace {
float half_bits_to_float(uint16_t h) {
    uint32_t sign = uint32_t(h >> 15) << 31, e = (h >> 10) & 31, m = h & 0x3FF, bits;
    if (e == 0) {
        float f = float(m) * (1.0f / 16777216.0f);
        return sign ? -f : f;
    }
    if (e == 31) bits = sign | 0x7F800000u | (m << 13);
    else bits = sign | ((e + 112) << 23) | (m << 13);
    float f;
    std::memcpy(&f, &bits, 4);
    return f;
}
}  // namespace

int decode_image(const AkvTables& t, const uint8_t* data, size_t bytes, float* rgba, unsigned w, unsigned h) {
    const unsigned bx = t.block_x, by = t.block_y;
    const unsigned cols = (w + bx - 1) / bx, rows = (h + by - 1) / by;
    if (bytes < size_t(cols) * rows * 16) return 1;
    uint16_t tex[kMaxTexels * 4];
    for (unsigned r = 0; r < rows; ++r)
        for (unsigned c = 0; c < cols; ++c) {
            decode_block_fp16(t, data + 16 * (size_t(r) * cols + c), tex);
            for (unsigned y = 0; y < by && r * by + y < h; ++y)
                for (unsigned x = 0; x < bx && c * bx + x < w; ++x)
                    for (int ch = 0; ch < 4; ++ch)
                        rgba[(size_t(r * by + y) * w + c * bx + x) * 4 + ch] =
                            half_bits_to_float(tex[4 * (y * bx + x) + ch]);
        }
    return 0;
}

}  // namespace akv
