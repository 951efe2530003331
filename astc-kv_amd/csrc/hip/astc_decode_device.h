// gfx950 software ASTC LDR decode in two stages that each keep a whole
// workgroup busy.
//
//  1. decode_header: one lane per 16-byte block. Block mode, partitioning,
//     colour endpoint modes, colour integer-sequence (BISE) unpack, endpoint
//     unquantisation and decode, and the weight BISE unpacked into plain
//     nb-bit fields (grid order). The result is a 104-byte BlockDesc in LDS.
//     When the block has an identity weight grid, one plane, and few enough
//     partitions x weight levels, the header also evaluates every possible
//     texel value, (partition, weight level) -> FP16 per channel, so that the
//     texel stage is a table lookup ("table path"). Constant blocks (void
//     extent, error colour) are one-entry tables.
//  2. texel_fp16: one lane per texel. Table path: weight field + partition
//     index -> table entry. Otherwise ("compute path"): weight unquantisation,
//     bilinear infill for reduced grids, dual-plane selection, and the
//     interpolation C = (e0*(64-w) + e1*w + 32) >> 6 as one packed-u16 dot
//     product per channel.
// Values are astcenc's: UNORM16 C, output FP16 = 1.0 if C == 0xFFFF, else
// C / 65536 rounded toward zero.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

#include "astc_format.h"

namespace akv_hip {

using akv::AkvTables;

// Per-workgroup lookup tables in LDS.
struct SmallLuts {
    uint16_t trit[256];
    uint16_t quint[128];
    uint16_t ise[akv::kNumRanges];
    uint8_t levels[12];
    uint8_t pad[6];
    uint8_t wunq[12][32];
};

// BlockDesc.info fields (bits 0-3 grid width, 4-7 grid height).
constexpr uint32_t kInfoDual = 1u << 8;         // bits 9-10: colour component of plane 1
constexpr int kInfoNbShift = 11;                // bits 11-13: weight field width
constexpr int kInfoRangeShift = 14;             // bits 14-17: weight range
constexpr int kInfoLevelsShift = 18;            // bits 18-23: table row length (weight levels)
constexpr uint32_t kInfoIdentity = 1u << 24;
constexpr uint32_t kInfoTable = 1u << 25;

template <int NCH>
struct alignas(8) BlockDesc {
    static constexpr int kTabEntries = 32 / NCH;   // 64 bytes of FP16 texel values
    union {
        uint32_t ep[4][NCH];   // compute path: e0 | e1 << 16 (UNORM16) per partition and channel
        uint32_t tab[16];      // table path: entry p * levels + weight field -> NCH fp16
    };
    uint32_t qw[5];            // weight fields, nb bits each, grid order (planes interleaved); qw[4] = 0
    uint32_t part[4];          // 2-bit partition index per texel (texel i: word i / 16, bits 2 * (i % 16))
    uint32_t info;
};
static_assert(sizeof(BlockDesc<4>) == 104 && sizeof(BlockDesc<1>) == 104, "BlockDesc layout");

struct Footprint {
    int bx, by, ntex, ds, dt;   // ds, dt: weight infill steps (1024 + b/2) / (b - 1)
};

__device__ inline void stage_luts(const AkvTables* __restrict__ tab, SmallLuts& L, int tid, int nthreads) {
    constexpr uint8_t kLevels[12] = {2, 3, 4, 5, 6, 8, 10, 12, 16, 20, 24, 32};
    for (int i = tid; i < 256; i += nthreads) L.trit[i] = tab->trit[i];
    for (int i = tid; i < 128; i += nthreads) L.quint[i] = tab->quint[i];
    for (int i = tid; i < akv::kNumRanges; i += nthreads) L.ise[i] = tab->ise[i];
    for (int i = tid; i < 12; i += nthreads) L.levels[i] = kLevels[i];
    for (int i = tid; i < 12 * 32; i += nthreads) (&L.wunq[0][0])[i] = (&tab->weight_unq[0][0])[i];
}

// Bits [pos, pos+n) of a 128-bit value, 0 < n <= 40; bits past 127 read zero.
struct Bits128 {
    uint64_t lo, hi;
    __device__ inline uint64_t get(int pos, int n) const {
        uint64_t v;
        if (pos >= 64) v = hi >> (pos - 64);
        else if (pos == 0) v = lo;
        else v = (lo >> pos) | (hi << (64 - pos));
        return v & ((uint64_t(1) << n) - 1);
    }
};

__device__ inline int ise_sequence_bits(int count, int n, bool trit, bool quint) {
    int b = count * n;
    if (trit) b += (count * 8 + 4) / 5;
    if (quint) b += (count * 7 + 2) / 3;
    return b;
}

// Colour value j of this lane's unpacked colour integers (bytes in LDS,
// column-major [5][stride] dwords).
__device__ inline int cval(const uint32_t* cv, int stride, int j) {
    return int((cv[(j >> 2) * stride] >> (8 * (j & 3))) & 0xFF);
}

__device__ inline int clamp255(int v) { return v < 0 ? 0 : (v > 255 ? 255 : v); }

__device__ inline void bit_transfer(int& offset, int& base) {
    base = (base >> 1) | (offset & 0x80);
    offset = (offset >> 1) & 0x3F;
    if (offset & 0x20) offset -= 0x40;
}

// Endpoint decode of one partition: 8-bit RGBA pairs. False for HDR modes.
__device__ inline bool cem_endpoints(int cem, const uint32_t* cv, int stride, int k, int* e0, int* e1) {
    int v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = (j < 2 * ((cem >> 2) + 1)) ? cval(cv, stride, k + j) : 0;
    switch (cem) {
        case 0:
            e0[0] = e0[1] = e0[2] = v[0]; e0[3] = 255;
            e1[0] = e1[1] = e1[2] = v[1]; e1[3] = 255;
            return true;
        case 1: {
            int l0 = (v[0] >> 2) | (v[1] & 0xC0);
            int l1 = min(l0 + (v[1] & 0x3F), 255);
            e0[0] = e0[1] = e0[2] = l0; e0[3] = 255;
            e1[0] = e1[1] = e1[2] = l1; e1[3] = 255;
            return true;
        }
        case 4:
            e0[0] = e0[1] = e0[2] = v[0]; e0[3] = v[2];
            e1[0] = e1[1] = e1[2] = v[1]; e1[3] = v[3];
            return true;
        case 5: {
            int l0 = v[0], dl = v[1], a0 = v[2], da = v[3];
            bit_transfer(dl, l0);
            bit_transfer(da, a0);
            int l1 = clamp255(l0 + dl);
            e0[0] = e0[1] = e0[2] = l0; e0[3] = a0;
            e1[0] = e1[1] = e1[2] = l1; e1[3] = clamp255(a0 + da);
            return true;
        }
        case 6:
        case 10: {
            int s = v[3];
            e0[0] = (v[0] * s) >> 8; e0[1] = (v[1] * s) >> 8; e0[2] = (v[2] * s) >> 8;
            e0[3] = cem == 10 ? v[4] : 255;
            e1[0] = v[0]; e1[1] = v[1]; e1[2] = v[2];
            e1[3] = cem == 10 ? v[5] : 255;
            return true;
        }
        case 8:
        case 12: {
            int a0 = cem == 12 ? v[6] : 255, a1 = cem == 12 ? v[7] : 255;
            if (v[1] + v[3] + v[5] >= v[0] + v[2] + v[4]) {
                e0[0] = v[0]; e0[1] = v[2]; e0[2] = v[4]; e0[3] = a0;
                e1[0] = v[1]; e1[1] = v[3]; e1[2] = v[5]; e1[3] = a1;
            } else {
                // Swapped endpoints with blue contraction.
                e0[0] = (v[1] + v[5]) >> 1; e0[1] = (v[3] + v[5]) >> 1; e0[2] = v[5]; e0[3] = a1;
                e1[0] = (v[0] + v[4]) >> 1; e1[1] = (v[2] + v[4]) >> 1; e1[2] = v[4]; e1[3] = a0;
            }
            return true;
        }
        case 9:
        case 13: {
            int b0 = v[0], o0 = v[1], b1 = v[2], o1 = v[3], b2 = v[4], o2 = v[5];
            int b3 = cem == 13 ? v[6] : 255, o3 = cem == 13 ? v[7] : 0;
            bit_transfer(o0, b0);
            bit_transfer(o1, b1);
            bit_transfer(o2, b2);
            if (cem == 13) bit_transfer(o3, b3);
            int s0 = b0 + o0, s1 = b1 + o1, s2 = b2 + o2, s3 = b3 + o3;
            if (o0 + o1 + o2 >= 0) {
                e0[0] = b0; e0[1] = b1; e0[2] = b2; e0[3] = b3;
                e1[0] = s0; e1[1] = s1; e1[2] = s2; e1[3] = s3;
            } else {
                e0[0] = (s0 + s2) >> 1; e0[1] = (s1 + s2) >> 1; e0[2] = s2; e0[3] = s3;
                e1[0] = (b0 + b2) >> 1; e1[1] = (b1 + b2) >> 1; e1[2] = b2; e1[3] = b3;
            }
#pragma unroll
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

// C' for one channel: astcenc's UNORM16 value, except that 0xFFFF becomes
// 0x10000, so that C' / 65536 rounded toward zero is the FP16 value astcenc
// returns. With y = dot + 96 = (C + 1) * 64 + r (0 <= r < 64),
// C' = (y >> 6) + (y >> 22) - 1.
__device__ inline uint32_t interp_c(uint32_t ep, uint32_t wp) {
    typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
    const uint32_t y =
        __builtin_amdgcn_udot2(__builtin_bit_cast(u16x2, ep), __builtin_bit_cast(u16x2, wp), 96u, false);
    return (y >> 6) + (y >> 22) - 1u;
}

// Two C' values -> their FP16 values (round toward zero), packed.
__device__ inline uint32_t pack_fp16_rtz(uint32_t c0, uint32_t c1) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(float(c0) * (1.0f / 65536.0f),
                                                                   float(c1) * (1.0f / 65536.0f)));
}

__device__ inline uint32_t weight_pair(int w) { return uint32_t(64 - w) | (uint32_t(w) << 16); }

// The NCH fp16 values of one (partition, weight) as table entry `entry`;
// entries are 2 * NCH bytes (NCH == 1: two entries share a dword).
template <int NCH>
__device__ inline void put_entry(uint32_t* tab, int entry, const uint32_t* ep, uint32_t wp) {
    if constexpr (NCH == 4) {
        tab[2 * entry] = pack_fp16_rtz(interp_c(ep[0], wp), interp_c(ep[1], wp));
        tab[2 * entry + 1] = pack_fp16_rtz(interp_c(ep[2], wp), interp_c(ep[3], wp));
    } else {
        reinterpret_cast<uint16_t*>(tab)[entry] = uint16_t(pack_fp16_rtz(interp_c(ep[0], wp), 0));
    }
}

// A constant block (void extent or error colour): one table entry.
template <int NCH>
__device__ inline void set_constant(BlockDesc<NCH>& d, uint32_t r, uint32_t g, uint32_t b, uint32_t a) {
    const uint32_t c[4] = {r, g, b, a};
    uint32_t ep[NCH];
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch) ep[ch] = c[ch] | (c[ch] << 16);
    put_entry<NCH>(d.tab, 0, ep, weight_pair(0));
#pragma unroll
    for (int i = 0; i < 5; ++i) d.qw[i] = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) d.part[i] = 0;
    d.info = kInfoTable | kInfoIdentity | (1u << kInfoLevelsShift);
}

// Appends nb-bit fields to the five-word weight stream of a BlockDesc.
struct FieldWriter {
    uint32_t* out;
    uint64_t acc;
    int bits, words;
    __device__ inline void put(uint32_t v, int nb) {
        acc |= uint64_t(v) << bits;
        bits += nb;
        if (bits >= 32) {
            out[words++] = uint32_t(acc);
            acc >>= 32;
            bits -= 32;
        }
    }
    __device__ inline void finish() {
        if (bits > 0) out[words++] = uint32_t(acc);
        for (; words < 5; ++words) out[words] = 0;
    }
};

// Stage 1: one lane decodes one block into `d`. `cv` is this lane's column of
// a [5][stride] dword scratch array for the unpacked colour values.
template <int NCH>
__device__ void decode_header(uint4 raw, const AkvTables* __restrict__ tab, const SmallLuts& L, BlockDesc<NCH>& d,
                              uint32_t* cv, int stride) {
    const Bits128 b{uint64_t(raw.x) | (uint64_t(raw.y) << 32), uint64_t(raw.z) | (uint64_t(raw.w) << 32)};
    const uint32_t mode = raw.x & 0x7FF;
    if ((mode & 0x1FF) == 0x1FC) {
        // Void extent: LDR constant colour (UNORM16 RGBA in bits 64..127).
        uint32_t s0 = uint32_t(b.get(12, 13)), s1 = uint32_t(b.get(25, 13));
        uint32_t t0 = uint32_t(b.get(38, 13)), t1 = uint32_t(b.get(51, 13));
        bool unbounded = (s0 & s1 & t0 & t1) == 0x1FFF;
        bool hdr = (raw.x >> 9) & 1;
        if (hdr || (!unbounded && (s0 >= s1 || t0 >= t1))) set_constant(d, 0xFFFF, 0, 0xFFFF, 0xFFFF);
        else set_constant(d, raw.z & 0xFFFF, raw.z >> 16, raw.w & 0xFFFF, raw.w >> 16);
        return;
    }
    const uint32_t md = tab->block_mode[mode];
    const int parts = int((raw.x >> 11) & 3) + 1;
    if (!md || (akv::mode_dual(md) && parts == 4)) {
        set_constant(d, 0xFFFF, 0, 0xFFFF, 0xFFFF);
        return;
    }
    const int wbits = int(akv::mode_wbits(md));
    int below = 128 - wbits;
    int color_start = 17, seed = 0;
    uint32_t cems;  // 4 bits per partition
    if (parts == 1) {
        cems = (raw.x >> 13) & 15;
    } else {
        seed = int((raw.x >> 13) & 0x3FF);
        color_start = 29;
        uint32_t sel = (raw.x >> 23) & 0x3F;
        if ((sel & 3) == 0) {
            cems = (sel >> 2) * 0x1111u;
        } else {
            int extra = 3 * parts - 4;
            below -= extra;
            sel |= uint32_t(b.get(below, extra)) << 6;
            int base_class = int(sel & 3) - 1;
            cems = 0;
            for (int p = 0; p < parts; ++p) {
                int up = (sel >> (2 + p)) & 1;
                int low = (sel >> (2 + parts + 2 * p)) & 3;
                cems |= uint32_t(((base_class + up) << 2) | low) << (4 * p);
            }
        }
    }
    const bool dual = akv::mode_dual(md);
    uint32_t ccs = 0;
    if (dual) {
        below -= 2;
        ccs = uint32_t(b.get(below, 2));
    }
    int pairs = 0;
    for (int p = 0; p < parts; ++p) pairs += int((cems >> (4 * p)) & 15) / 4 + 1;
    const int avail = below - color_start;
    const int crange = (pairs <= 9 && avail > 0) ? int(tab->color_range[pairs][min(avail, 127)]) : -1;
    if (crange < akv::kRange6) {
        set_constant(d, 0xFFFF, 0, 0xFFFF, 0xFFFF);
        return;
    }
    // Partition pattern, issued before the colour unpack needs its own loads.
    uint4 pw = uint4{0, 0, 0, 0};
    if (parts > 1) pw = *reinterpret_cast<const uint4*>(tab->partition[parts - 2][seed]);

    // Colour integer sequence -> unquantised bytes, four per scratch dword.
    {
        const int nv = 2 * pairs;
        const uint32_t ise = L.ise[crange];
        const int n = int(ise & 0xFF);
        const bool trit = (ise >> 8) & 1, quint = (ise >> 9) & 1;
        const int end = color_start + ise_sequence_bits(nv, n, trit, quint);
        const uint64_t mask = (uint64_t(1) << n) - 1;
        const uint8_t* unq = tab->color_unq[crange];
        uint32_t packed[5] = {0, 0, 0, 0, 0};
        if (trit) {
            const int gb = 5 * n + 8;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                if (5 * g < nv) {
                    int pos = color_start + g * gb;
                    uint64_t G = b.get(pos, min(gb, end - pos));
                    uint32_t T = uint32_t((G >> n) & 3) | uint32_t((G >> (2 * n + 2)) & 3) << 2 |
                                 uint32_t((G >> (3 * n + 4)) & 1) << 4 | uint32_t((G >> (4 * n + 5)) & 3) << 5 |
                                 uint32_t((G >> (5 * n + 7)) & 1) << 7;
                    uint32_t dig = L.trit[T];
                    const int moff[5] = {0, n + 2, 2 * n + 4, 3 * n + 5, 4 * n + 7};
#pragma unroll
                    for (int j = 0; j < 5; ++j) {
                        const int idx = 5 * g + j;
                        if (idx < 20 && idx < nv) {
                            uint32_t v = (((dig >> (2 * j)) & 3) << n) | uint32_t((G >> moff[j]) & mask);
                            packed[idx >> 2] |= uint32_t(unq[v]) << (8 * (idx & 3));
                        }
                    }
                }
            }
        } else if (quint) {
            const int gb = 3 * n + 7;
#pragma unroll
            for (int g = 0; g < 6; ++g) {
                if (3 * g < nv) {
                    int pos = color_start + g * gb;
                    uint64_t G = b.get(pos, min(gb, end - pos));
                    uint32_t Q = uint32_t((G >> n) & 7) | uint32_t((G >> (2 * n + 3)) & 3) << 3 |
                                 uint32_t((G >> (3 * n + 5)) & 3) << 5;
                    uint32_t dig = L.quint[Q];
                    const int moff[3] = {0, n + 3, 2 * n + 5};
#pragma unroll
                    for (int j = 0; j < 3; ++j) {
                        const int idx = 3 * g + j;
                        if (idx < nv) {
                            uint32_t v = (((dig >> (3 * j)) & 7) << n) | uint32_t((G >> moff[j]) & mask);
                            packed[idx >> 2] |= uint32_t(unq[v]) << (8 * (idx & 3));
                        }
                    }
                }
            }
        } else {
#pragma unroll
            for (int idx = 0; idx < 18; ++idx)
                if (idx < nv) packed[idx >> 2] |= uint32_t(unq[b.get(color_start + idx * n, n)]) << (8 * (idx & 3));
        }
#pragma unroll
        for (int i = 0; i < 5; ++i) cv[i * stride] = packed[i];
    }

    // Weights: the BISE stream runs from bit 127 downwards, so in the
    // bit-reversed block it starts at bit 0. Unpack it to nb-bit fields.
    const int wrange = int(akv::mode_range(md));
    const uint32_t wise = L.ise[wrange];
    const int n = int(wise & 0xFF);
    const bool wtrit = (wise >> 8) & 1, wquint = (wise >> 9) & 1;
    const int nw = int(akv::mode_gw(md) * akv::mode_gh(md)) << (dual ? 1 : 0);
    const uint32_t rev[5] = {__builtin_bitreverse32(raw.w), __builtin_bitreverse32(raw.z),
                             __builtin_bitreverse32(raw.y), __builtin_bitreverse32(raw.x), 0u};
    int nb = n;
    if (!wtrit && !wquint) {
        // Plain binary fields are nb-bit fields of the reversed stream already;
        // fields past the weight count are never read.
#pragma unroll
        for (int i = 0; i < 5; ++i) d.qw[i] = rev[i];
    } else {
        FieldWriter fw{d.qw, 0, 0, 0};
        if (wtrit) {
            nb = n + 2;
            const int gb = 5 * n + 8;
            for (int g = 0, pos = 0; 5 * g < nw; ++g, pos += gb) {
                const int w = pos >> 5;
                uint32_t G = __builtin_amdgcn_alignbit(rev[w + 1], rev[w], uint32_t(pos & 31));
                const int len = min(gb, wbits - pos);
                if (len < 32) G &= (1u << len) - 1;
                const uint32_t T = __builtin_amdgcn_ubfe(G, n, 2) | __builtin_amdgcn_ubfe(G, 2 * n + 2, 2) << 2 |
                                   __builtin_amdgcn_ubfe(G, 3 * n + 4, 1) << 4 |
                                   __builtin_amdgcn_ubfe(G, 4 * n + 5, 2) << 5 |
                                   __builtin_amdgcn_ubfe(G, 5 * n + 7, 1) << 7;
                const uint32_t dig = L.trit[T];
                const int cnt = min(5, nw - 5 * g);
                for (int j = 0; j < cnt; ++j) {
                    const int moff = j * n + int((0x75420u >> (4 * j)) & 15);
                    fw.put((((dig >> (2 * j)) & 3) << n) | __builtin_amdgcn_ubfe(G, moff, n), nb);
                }
            }
        } else {
            nb = n + 3;
            const int gb = 3 * n + 7;
            for (int g = 0, pos = 0; 3 * g < nw; ++g, pos += gb) {
                const int w = pos >> 5;
                uint32_t G = __builtin_amdgcn_alignbit(rev[w + 1], rev[w], uint32_t(pos & 31));
                const int len = min(gb, wbits - pos);
                if (len < 32) G &= (1u << len) - 1;
                const uint32_t Q = __builtin_amdgcn_ubfe(G, n, 3) | __builtin_amdgcn_ubfe(G, 2 * n + 3, 2) << 3 |
                                   __builtin_amdgcn_ubfe(G, 3 * n + 5, 2) << 5;
                const uint32_t dig = L.quint[Q];
                const int cnt = min(3, nw - 3 * g);
                for (int j = 0; j < cnt; ++j) {
                    const int moff = j * n + int((0x530u >> (4 * j)) & 15);
                    fw.put((((dig >> (3 * j)) & 7) << n) | __builtin_amdgcn_ubfe(G, moff, n), nb);
                }
            }
        }
        fw.finish();
    }

    // Endpoints per partition -> endpoint pairs, or the texel table.
    const int levels = L.levels[wrange];
    const bool identity = akv::mode_identity(md);
    const bool table = identity && !dual && parts * levels <= BlockDesc<NCH>::kTabEntries;
    for (int p = 0, k = 0; p < parts; ++p) {
        const int cem = int((cems >> (4 * p)) & 15);
        int e0[4], e1[4];
        uint32_t ep[NCH];
        if (cem_endpoints(cem, cv, stride, k, e0, e1)) {
#pragma unroll
            for (int ch = 0; ch < NCH; ++ch) ep[ch] = uint32_t(e0[ch] * 257) | (uint32_t(e1[ch] * 257) << 16);
        } else {
            const uint32_t err[4] = {0xFFFFFFFFu, 0u, 0xFFFFFFFFu, 0xFFFFFFFFu};
#pragma unroll
            for (int ch = 0; ch < NCH; ++ch) ep[ch] = err[ch];
        }
        k += 2 * ((cem >> 2) + 1);
        if (table) {
            for (int q = 0; q < levels; ++q)
                put_entry<NCH>(d.tab, p * levels + q, ep, weight_pair(L.wunq[wrange][q]));
        } else {
#pragma unroll
            for (int ch = 0; ch < NCH; ++ch) d.ep[p][ch] = ep[ch];
        }
    }
    d.part[0] = pw.x;
    d.part[1] = pw.y;
    d.part[2] = pw.z;
    d.part[3] = pw.w;
    d.info = (md & 0xFFu) | (dual ? kInfoDual : 0u) | (ccs << 9) | (uint32_t(nb) << kInfoNbShift) |
             (uint32_t(wrange) << kInfoRangeShift) | (uint32_t(levels) << kInfoLevelsShift) |
             (identity ? kInfoIdentity : 0u) | (table ? kInfoTable : 0u);
}

// Weight field `idx` (grid order, planes interleaved) of a block.
template <int NCH>
__device__ inline uint32_t field_at(const BlockDesc<NCH>& d, uint32_t nb, int idx) {
    const uint32_t pos = uint32_t(idx) * nb, w = pos >> 5;
    return __builtin_amdgcn_ubfe(__builtin_amdgcn_alignbit(d.qw[w + 1], d.qw[w], pos & 31), 0, nb);
}

// Unquantised, infilled weight of texel (x, y) on plane `plane` (compute path).
template <int NCH>
__device__ inline int texel_weight(const BlockDesc<NCH>& d, const SmallLuts& L, const Footprint& f, uint32_t info,
                                   int x, int y, int plane) {
    const uint32_t nb = (info >> kInfoNbShift) & 7;
    const uint8_t* unq = L.wunq[(info >> kInfoRangeShift) & 15];
    const int sh = (info & kInfoDual) ? 1 : 0;
    if (info & kInfoIdentity) return unq[field_at(d, nb, ((y * f.bx + x) << sh) + plane)];
    const int gw = int(info & 15), gh = int((info >> 4) & 15);
    const int gs = (f.ds * x * (gw - 1) + 32) >> 6, gt = (f.dt * y * (gh - 1) + 32) >> 6;
    const int fs = gs & 15, ft = gt & 15, base = (gs >> 4) + (gt >> 4) * gw;
    const int f11 = (fs * ft + 8) >> 4, f01 = fs - f11, f10 = ft - f11, f00 = 16 - fs - ft + f11;
    // Taps with a zero factor may lie outside the grid: read the base tap instead.
    const int i01 = f01 ? base + 1 : base, i10 = f10 ? base + gw : base, i11 = f11 ? base + gw + 1 : base;
    return (unq[field_at(d, nb, (base << sh) + plane)] * f00 + unq[field_at(d, nb, (i01 << sh) + plane)] * f01 +
            unq[field_at(d, nb, (i10 << sh) + plane)] * f10 + unq[field_at(d, nb, (i11 << sh) + plane)] * f11 + 8) >>
           4;
}

// Stage 2: the FP16 values of texel (x, y) of a block (NCH == 4:
// {R | G << 16, B | A << 16}; NCH == 1: R in the low half of .x).
template <int NCH>
__device__ inline uint2 texel_fp16(const BlockDesc<NCH>& d, const SmallLuts& L, const Footprint& f, int x, int y) {
    const uint32_t info = d.info;
    const int i = y * f.bx + x;
    const int p = int(__builtin_amdgcn_ubfe(d.part[i >> 4], 2 * (i & 15), 2));
    if (info & kInfoTable) {
        const uint32_t nb = (info >> kInfoNbShift) & 7;
        const int entry = p * int((info >> kInfoLevelsShift) & 63) + int(field_at(d, nb, i));
        if constexpr (NCH == 4) return *reinterpret_cast<const uint2*>(&d.tab[2 * entry]);
        else return uint2{reinterpret_cast<const uint16_t*>(d.tab)[entry], 0u};
    }
    const uint32_t wp0 = weight_pair(texel_weight(d, L, f, info, x, y, 0));
    const uint32_t wp1 = (info & kInfoDual) ? weight_pair(texel_weight(d, L, f, info, x, y, 1)) : wp0;
    const int ccs = (info & kInfoDual) ? int((info >> 9) & 3) : 4;
    uint32_t C[NCH];
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch) C[ch] = interp_c(d.ep[p][ch], ch == ccs ? wp1 : wp0);
    if constexpr (NCH == 4) return uint2{pack_fp16_rtz(C[0], C[1]), pack_fp16_rtz(C[2], C[3])};
    else return uint2{pack_fp16_rtz(C[0], 0) & 0xFFFFu, 0u};
}

}  // namespace akv_hip
