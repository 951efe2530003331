// gfx950 software ASTC LDR decode, split in two stages so that a workgroup
// can decode many blocks in parallel:
//   1. decode_header: one lane per 16-byte block. Block mode, partitioning,
//      colour endpoint modes, colour integer-sequence unpack, endpoint
//      unquantisation and decode -> a BlockDesc in LDS (UNORM16 endpoint pairs
//      per partition and channel, the bit-reversed weight stream, the
//      partition pattern, the weight-grid descriptor).
//   2. decode_texel: one lane per texel. Random-access weight unpack from the
//      reversed stream (trit/quint block LUTs in LDS), weight infill for
//      reduced grids, partition lookup, then per channel
//      C = (e0*(64-w) + e1*w + 32) >> 6 as a single packed-u16 dot product.
// The result is astcenc's UNORM16 value; unorm16_scaled() maps it to the FP16
// value astcenc returns (0xFFFF -> 1.0, else c/65536 truncated), which a
// round-toward-zero FP16 pack (v_cvt_pkrtz_f16_f32) produces exactly.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

#include "astc_format.h"

namespace akv_hip {

using akv::AkvTables;

// Per-texel lookup tables staged in LDS by every workgroup.
struct SmallLuts {
    uint16_t trit[256];
    uint16_t quint[128];
    uint16_t ise[akv::kNumRanges];
    uint16_t pad[3];
    uint8_t wunq[12][32];
};

// BlockDesc.info bits.
constexpr uint32_t kInfoDual = 1u << 8;
constexpr uint32_t kInfoIdentity = 1u << 22;
constexpr uint32_t kInfoConst = 1u << 23;

template <int NCH>
struct BlockDesc {
    uint32_t ep[4][NCH];   // e0 | e1 << 16, UNORM16, per partition and channel
    uint32_t rev[5];       // block bits reversed (weight stream at bit 0), rev[4] = 0
    uint32_t part[4];      // 2-bit partition index per texel
    uint32_t info;         // gw | gh<<4 | dual<<8 | ccs<<9 | wrange<<11 | seqbits<<15 | flags
    uint32_t pad[2];
};
static_assert(sizeof(BlockDesc<4>) % 16 == 0, "desc alignment");
static_assert(sizeof(BlockDesc<1>) % 16 == 0, "desc alignment");

__device__ inline void stage_luts(const AkvTables* __restrict__ tab, SmallLuts& L, int tid, int nthreads) {
    for (int i = tid; i < 256; i += nthreads) L.trit[i] = tab->trit[i];
    for (int i = tid; i < 128; i += nthreads) L.quint[i] = tab->quint[i];
    for (int i = tid; i < akv::kNumRanges; i += nthreads) L.ise[i] = tab->ise[i];
    for (int i = tid; i < 12 * 32; i += nthreads) (&L.wunq[0][0])[i] = (&tab->weight_unq[0][0])[i];
}

// Bits [pos, pos+n) of a 128-bit value, n <= 40; bits past 127 read zero.
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
// column-major [5][nthreads] dwords).
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

template <int NCH>
__device__ inline void set_constant(BlockDesc<NCH>& d, uint32_t r, uint32_t g, uint32_t b, uint32_t a) {
    const uint32_t c[4] = {r, g, b, a};
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch) d.ep[0][ch] = c[ch] | (c[ch] << 16);
#pragma unroll
    for (int i = 0; i < 4; ++i) d.part[i] = 0;
    d.info = kInfoConst;
}

// Stage 1: one lane decodes one block into `d`. `cv` is this lane's column of
// a [5][stride] dword scratch array used to hold the unpacked colour values.
template <int NCH>
__device__ void decode_header(uint4 raw, const AkvTables* __restrict__ tab, const SmallLuts& L, BlockDesc<NCH>& d,
                              uint32_t* cv, int stride) {
    const Bits128 b{uint64_t(raw.x) | (uint64_t(raw.y) << 32), uint64_t(raw.z) | (uint64_t(raw.w) << 32)};
    d.rev[0] = __builtin_bitreverse32(raw.w);
    d.rev[1] = __builtin_bitreverse32(raw.z);
    d.rev[2] = __builtin_bitreverse32(raw.y);
    d.rev[3] = __builtin_bitreverse32(raw.x);
    d.rev[4] = 0;
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
    int below = 128 - int(akv::mode_wbits(md));
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
    uint32_t ccs = 0;
    if (akv::mode_dual(md)) {
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
    // Endpoints per partition.
    for (int p = 0, k = 0; p < 4; ++p) {
        if (p >= parts) break;
        const int cem = int((cems >> (4 * p)) & 15);
        int e0[4], e1[4];
        if (cem_endpoints(cem, cv, stride, k, e0, e1)) {
#pragma unroll
            for (int ch = 0; ch < NCH; ++ch) d.ep[p][ch] = uint32_t(e0[ch] * 257) | (uint32_t(e1[ch] * 257) << 16);
        } else {
            const uint32_t err[4] = {0xFFFFFFFFu, 0u, 0xFFFFFFFFu, 0xFFFFFFFFu};
#pragma unroll
            for (int ch = 0; ch < NCH; ++ch) d.ep[p][ch] = err[ch];
        }
        k += 2 * ((cem >> 2) + 1);
    }
    if (parts > 1) {
        const uint32_t* pw = tab->partition[parts - 2][seed];
#pragma unroll
        for (int i = 0; i < 4; ++i) d.part[i] = pw[i];
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) d.part[i] = 0;
    }
    d.info = (md & 0x1FFu) | (ccs << 9) | (akv::mode_range(md) << 11) | (akv::mode_wbits(md) << 15) |
             (akv::mode_identity(md) ? kInfoIdentity : 0u);
}

// Unquantised grid weight `idx` (plane-interleaved index) of a block.
template <int NCH>
__device__ inline int weight_at(const BlockDesc<NCH>& d, const SmallLuts& L, uint32_t info, int idx) {
    const int range = int((info >> 11) & 15);
    const int seq = int((info >> 15) & 127);
    const uint32_t ise = L.ise[range];
    const int n = int(ise & 0xFF);
    int v;
    if (ise & 0x100) {
        const int g = idx / 5, j = idx - 5 * g, gb = 5 * n + 8, pos = g * gb;
        const int w = pos >> 5, sh = pos & 31;
        uint32_t G = __builtin_amdgcn_alignbit(d.rev[w + 1], d.rev[w], sh);
        const int len = min(gb, seq - pos);
        G &= len >= 32 ? 0xFFFFFFFFu : ((1u << len) - 1);
        uint32_t T = __builtin_amdgcn_ubfe(G, n, 2) | __builtin_amdgcn_ubfe(G, 2 * n + 2, 2) << 2 |
                     __builtin_amdgcn_ubfe(G, 3 * n + 4, 1) << 4 | __builtin_amdgcn_ubfe(G, 4 * n + 5, 2) << 5 |
                     __builtin_amdgcn_ubfe(G, 5 * n + 7, 1) << 7;
        const int moff = j * n + int((0x75420u >> (4 * j)) & 15);
        v = int(((uint32_t(L.trit[T]) >> (2 * j)) & 3) << n | __builtin_amdgcn_ubfe(G, moff, n));
    } else if (ise & 0x200) {
        const int g = idx / 3, j = idx - 3 * g, gb = 3 * n + 7, pos = g * gb;
        const int w = pos >> 5, sh = pos & 31;
        uint32_t G = __builtin_amdgcn_alignbit(d.rev[w + 1], d.rev[w], sh);
        const int len = min(gb, seq - pos);
        G &= len >= 32 ? 0xFFFFFFFFu : ((1u << len) - 1);
        uint32_t Q = __builtin_amdgcn_ubfe(G, n, 3) | __builtin_amdgcn_ubfe(G, 2 * n + 3, 2) << 3 |
                     __builtin_amdgcn_ubfe(G, 3 * n + 5, 2) << 5;
        const int moff = j * n + int((0x530u >> (4 * j)) & 15);
        v = int(((uint32_t(L.quint[Q]) >> (3 * j)) & 7) << n | __builtin_amdgcn_ubfe(G, moff, n));
    } else {
        const int pos = idx * n, w = pos >> 5, sh = pos & 31;
        v = int(__builtin_amdgcn_ubfe(__builtin_amdgcn_alignbit(d.rev[w + 1], d.rev[w], sh), 0, n));
    }
    return L.wunq[range][v];
}

// Stage 2: UNORM16 value of channels 0..NCH-1 of texel (x, y). `ds`/`dt` are
// the infill steps (1024 + b/2) / (b - 1) of the footprint.
template <int NCH>
__device__ inline void decode_texel(const BlockDesc<NCH>& d, const SmallLuts& L, int x, int y, int bx, int ds,
                                    int dt, uint32_t* C) {
    const uint32_t info = d.info;
    const int i = y * bx + x;
    uint32_t wp0 = 64, wp1 = 64;  // packed (64 - w) | w << 16 for planes 0 and 1
    const bool dual = info & kInfoDual;
    if (!(info & kInfoConst)) {
        int w0, w1 = 0;
        if (info & kInfoIdentity) {
            w0 = weight_at(d, L, info, dual ? 2 * i : i);
            if (dual) w1 = weight_at(d, L, info, 2 * i + 1);
        } else {
            const int gw = int(info & 15), gh = int((info >> 4) & 15);
            const int gs = (ds * x * (gw - 1) + 32) >> 6, gt = (dt * y * (gh - 1) + 32) >> 6;
            const int fs = gs & 15, ft = gt & 15, base = (gs >> 4) + (gt >> 4) * gw;
            const int f11 = (fs * ft + 8) >> 4, f01 = fs - f11, f10 = ft - f11, f00 = 16 - fs - ft + f11;
            const int i01 = f01 ? base + 1 : base, i10 = f10 ? base + gw : base, i11 = f11 ? base + gw + 1 : base;
            const int planes = dual ? 2 : 1;
            w0 = (weight_at(d, L, info, base * planes) * f00 + weight_at(d, L, info, i01 * planes) * f01 +
                  weight_at(d, L, info, i10 * planes) * f10 + weight_at(d, L, info, i11 * planes) * f11 + 8) >> 4;
            if (dual)
                w1 = (weight_at(d, L, info, base * 2 + 1) * f00 + weight_at(d, L, info, i01 * 2 + 1) * f01 +
                      weight_at(d, L, info, i10 * 2 + 1) * f10 + weight_at(d, L, info, i11 * 2 + 1) * f11 + 8) >> 4;
        }
        wp0 = uint32_t(64 - w0) | (uint32_t(w0) << 16);
        wp1 = uint32_t(64 - w1) | (uint32_t(w1) << 16);
    }
    const int p = int((d.part[i >> 4] >> (2 * (i & 15))) & 3);
    const int ccs = dual ? int((info >> 9) & 3) : -1;
    typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch) {
        const uint32_t wp = ch == ccs ? wp1 : wp0;
        C[ch] = __builtin_amdgcn_udot2(__builtin_bit_cast(u16x2, d.ep[p][ch]), __builtin_bit_cast(u16x2, wp), 32u,
                                       false) >> 6;
    }
}

// UNORM16 -> the FP16 value astcenc outputs, as an exactly representable
// float: 0xFFFF maps to 1.0, anything else to c/65536 (truncated by the RTZ pack).
__device__ inline float unorm16_scaled(uint32_t c) {
    c += (c + 1) >> 16;
    return float(c) * (1.0f / 65536.0f);
}

__device__ inline uint32_t pack_fp16_rtz(uint32_t c0, uint32_t c1) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(unorm16_scaled(c0), unorm16_scaled(c1)));
}

}  // namespace akv_hip
