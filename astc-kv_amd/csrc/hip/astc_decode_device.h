// gfx950 software ASTC LDR decode in two stages that each keep a whole
// workgroup busy.
//
//  1. decode_header: one lane per 16-byte block, every lookup table in LDS
//     except the partition patterns. Block mode, partitioning,
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
#include <type_traits>

#include "astc_format.h"

namespace akv_hip {

using akv::AkvTables;

// The per-block decode tables, copied into LDS by every workgroup: the
// leading akv::kLdsTableBytes bytes of AkvTables, field for field.
struct alignas(16) LdsTables {
    uint32_t block_mode[2048];
    uint8_t color_unq[akv::kNumRanges][256];
    int8_t color_range[10][128];
    uint16_t trit[256];
    uint16_t quint[128];
    uint16_t ise[akv::kNumRanges];
    uint16_t pad0;
    uint8_t weight_unq[12][32];
    uint8_t weight_levels[12];
    uint8_t pad1[8];
};
static_assert(sizeof(LdsTables) == akv::kLdsTableBytes, "LdsTables mirrors the head of AkvTables");
static_assert(offsetof(LdsTables, color_unq) == offsetof(AkvTables, color_unq) &&
                  offsetof(LdsTables, color_range) == offsetof(AkvTables, color_range) &&
                  offsetof(LdsTables, trit) == offsetof(AkvTables, trit) &&
                  offsetof(LdsTables, quint) == offsetof(AkvTables, quint) &&
                  offsetof(LdsTables, ise) == offsetof(AkvTables, ise) &&
                  offsetof(LdsTables, weight_unq) == offsetof(AkvTables, weight_unq) &&
                  offsetof(LdsTables, weight_levels) == offsetof(AkvTables, weight_levels),
              "LdsTables field offsets");
static_assert(offsetof(LdsTables, weight_unq) % 4 == 0, "weight rows are read a dword at a time");

// BlockDesc.info fields (bits 0-3 grid width, 4-7 grid height).
constexpr uint32_t kInfoDual = 1u << 8;         // bits 9-10: colour component of plane 1
constexpr int kInfoNbShift = 11;                // bits 11-13: weight field width
constexpr int kInfoRangeShift = 14;             // bits 14-17: weight range
constexpr int kInfoLevelsShift = 18;            // bits 18-23: table row length (weight levels)
constexpr uint32_t kInfoIdentity = 1u << 24;
constexpr uint32_t kInfoTable = 1u << 25;
// A reduced weight grid with one plane whose texels a fill stage
// (fill_values) computes once per chunk: texel i is entry slot * ntex + i of
// the chunk's fill area (FillArea), slot in bits 27-31.
constexpr uint32_t kInfoFilled = 1u << 26;
constexpr int kInfoFillShift = 27;
constexpr int kFillSlots = 32;

// Texel values of the chunk's filled blocks: 1024 RGBA texels (8 bytes
// each, 8 KB: 32 blocks of 6x5) or 2048 scalar texels (2 bytes, 4 KB).
template <int NCH>
struct FillArea {
    static constexpr int kTexels = NCH == 4 ? 1024 : 2048;
    uint16_t v[kTexels * NCH];
};

template <int NCH>
struct BlockDesc {
    static constexpr int kTabEntries = 32 / NCH;   // 64 bytes of FP16 texel values
    union {
        uint32_t ep[4][NCH];   // compute path: e0 | e1 << 16 (UNORM16) per partition and channel
        uint32_t tab[16];      // table path: entry p * levels + weight field -> NCH fp16
    };
    uint32_t qw[5];            // weight fields, nb bits each, grid order (planes interleaved); qw[4] = 0
    uint32_t part[4];          // 2-bit partition index per texel (texel i: word i / 16, bits 2 * (i % 16))
    uint32_t info;
    uint32_t pad;              // 27 dwords: consecutive records start in different LDS banks
};
static_assert(sizeof(BlockDesc<4>) == 108 && sizeof(BlockDesc<1>) == 108, "BlockDesc layout");

struct Footprint {
    int bx, by, ntex, ds, dt;   // ds, dt: weight infill steps (1024 + b/2) / (b - 1)
};

// Copy the decode tables into LDS (16-byte copies; `tab` is 256-byte aligned).
// The copy in two halves, so that a kernel can issue the loads early and
// store them after other work: every load is issued before the first store
// (one memory latency, not one per pass), and the stores are unconditional
// (lanes past the end rewrite the last entry with its own value; a guarded
// store would let the compiler sink its load into the guard).
template <int NT>
struct TableStage {
    static constexpr int kN = int(sizeof(LdsTables) / 16), kIter = (kN + NT - 1) / NT;
    uint4 v[kIter];
    __device__ void load(const AkvTables* __restrict__ tab, int tid) {
        const uint4* src = reinterpret_cast<const uint4*>(tab);
#pragma unroll
        for (int j = 0; j < kIter; ++j) v[j] = src[min(tid + j * NT, kN - 1)];
    }
    __device__ void store(LdsTables& L, int tid) const {
        uint4* dst = reinterpret_cast<uint4*>(&L);
#pragma unroll
        for (int j = 0; j < kIter; ++j) dst[min(tid + j * NT, kN - 1)] = v[j];
    }
};

template <int NT>
__device__ inline void stage_tables(const AkvTables* __restrict__ tab, LdsTables& L, int tid) {
    TableStage<NT> t;
    t.load(tab, tid);
    t.store(L, tid);
}

// Bits [pos, pos + len) of a little-endian bit stream held in LDS dwords
// (0 <= len < 32; the dword after the one holding bit pos must be readable).
__device__ inline uint32_t stream_bits(const uint32_t* s, int pos, int len) {
    const int w = pos >> 5;
    return __builtin_amdgcn_ubfe(__builtin_amdgcn_alignbit(s[w + 1], s[w], uint32_t(pos & 31)), 0, uint32_t(len));
}

// As stream_bits, with the bits at or past `end` read as zero (the last group
// of an integer sequence may be cut short). Branch-free.
__device__ inline uint32_t stream_bits_until(const uint32_t* s, int pos, int len, int end) {
    return stream_bits(s, pos, min(max(end - pos, 0), len));
}

// Up to 40 bits [pos, pos + len) of an LDS bit stream as a 64-bit value,
// bits at or past `end` zero (reads three dwords).
__device__ inline uint64_t stream_bits64_until(const uint32_t* s, int pos, int len, int end) {
    const int w = pos >> 5, sh = pos & 31;
    const uint32_t lo = __builtin_amdgcn_alignbit(s[w + 1], s[w], uint32_t(sh));
    const uint32_t hi = __builtin_amdgcn_alignbit(s[w + 2], s[w + 1], uint32_t(sh));
    const int n = min(max(end - pos, 0), len);
    const uint64_t v = uint64_t(lo) | (uint64_t(hi) << 32);
    return n >= 64 ? v : v & ((uint64_t(1) << n) - 1);
}

__device__ inline uint32_t field64(uint64_t g, int pos, int len) {
    return uint32_t(g >> pos) & ((1u << len) - 1);
}

// --- Integer-sequence (BISE) unpacking specialised per range -----------------
// The header stage dispatches each integer sequence on its range: the lanes of
// a wave are walked in groups of equal range (readfirstlane loop), so inside a
// group the range is a wave-uniform constant and every bit position below is a
// compile-time constant of a 128-bit stream held in four registers.

template <int I>
using Idx = std::integral_constant<int, I>;

template <int B, int E, typename F>
__device__ __attribute__((always_inline)) inline void static_for(F&& f) {
    if constexpr (B < E) {
        f(Idx<B>{});
        static_for<B + 1, E>(f);
    }
}

// Bits [P, P + N) of a 128-bit little-endian value (N <= 32); bits past the
// 128 read as zero.
template <int P, int N>
__device__ inline uint32_t bits_at(const uint32_t (&s)[4]) {
    static_assert(N >= 0 && N <= 32 && P >= 0, "field");
    constexpr int w = P >> 5, o = P & 31;
    if constexpr (N == 0 || P >= 128) {
        return 0u;
    } else if constexpr (P + N > 128) {
        return bits_at<P, 128 - P>(s);
    } else if constexpr (o + N <= 32) {
        return N == 32 ? s[w] : __builtin_amdgcn_ubfe(s[w], uint32_t(o), uint32_t(N));
    } else {
        return __builtin_amdgcn_ubfe(__builtin_amdgcn_alignbit(s[w + 1], s[w], uint32_t(o)), 0u, uint32_t(N));
    }
}

// s >>= k (0 <= k < 32) and zero every bit at or past `end` (0 <= end).
__device__ inline void shift_and_cut(uint32_t (&s)[4], uint32_t k, int end) {
    s[0] = __builtin_amdgcn_alignbit(s[1], s[0], k);
    s[1] = __builtin_amdgcn_alignbit(s[2], s[1], k);
    s[2] = __builtin_amdgcn_alignbit(s[3], s[2], k);
    s[3] = s[3] >> k;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int keep = end - 32 * i;
        s[i] &= keep >= 32 ? ~0u : (keep <= 0 ? 0u : (1u << keep) - 1u);
    }
}

// Sequence bits of `count` values of range R.
template <int R>
__device__ inline int ise_seq_bits(int count) {
    constexpr akv::IseRange e = akv::kIse[R];
    return count * e.bits + (e.trit ? (count * 8 + 4) / 5 : 0) + (e.quint ? (count * 7 + 2) / 3 : 0);
}

constexpr int ise_seq_bits_c(int count, int r) {
    return count * akv::kIse[r].bits + (akv::kIse[r].trit ? (count * 8 + 4) / 5 : 0) +
           (akv::kIse[r].quint ? (count * 7 + 2) / 3 : 0);
}

// Largest value count (<= cap) of range r whose sequence fits in `budget` bits.
constexpr int ise_max_values(int r, int cap, int budget) {
    int v = cap;
    while (v > 0 && ise_seq_bits_c(v, r) > budget) --v;
    return v;
}

// Values 0 .. V-1 of an integer sequence of range R starting at bit 0 of s:
// emit(Idx<j>, value) with value = digit << bits | plain bits. Values past the
// real sequence are garbage (bits past its end must already be zero, since a
// truncated trit/quint group decodes with its missing bits as zero).
// vlim (wave-uniform): the trit/quint groups that hold only values vlim and
// up are skipped, at two branch points (past 16 and past 36 values), so that
// the groups below stay straight-line code. A vlim the compiler knows to be
// >= the value count removes the branches.
// B1, B2: the two branch points (value counts), 16 and 36 for weight
// sequences, 4 and 8 for colour sequences.
template <int GS, int NG, int B1 = 16, int B2 = 36, typename Group>
__device__ __attribute__((always_inline)) inline void ise_groups(int vlim, Group&& group) {
    constexpr int G1 = NG < (B1 + GS - 1) / GS ? NG : (B1 + GS - 1) / GS;
    constexpr int G2 = NG < (B2 + GS - 1) / GS ? NG : (B2 + GS - 1) / GS;
    static_for<0, G1>(group);
    if (vlim > B1) {
        static_for<G1, G2>(group);
        if (vlim > B2) static_for<G2, NG>(group);
    }
}

template <int R, int V, int B1 = 16, int B2 = 36, typename Emit>
__device__ __attribute__((always_inline)) inline void ise_unpack(const uint32_t (&s)[4], const LdsTables& L, int vlim,
                                                                 Emit&& emit) {
    constexpr akv::IseRange e = akv::kIse[R];
    constexpr int n = e.bits;
    if constexpr (e.trit) {
        constexpr int gb = 5 * n + 8;
        ise_groups<5, (V + 4) / 5, B1, B2>(vlim, [&](auto gi) {
            constexpr int p = decltype(gi)::value * gb;
            uint32_t T;
            if constexpr (n == 0) {
                T = bits_at<p, 8>(s);
            } else {
                T = bits_at<p + n, 2>(s) | bits_at<p + 2 * n + 2, 2>(s) << 2 | bits_at<p + 3 * n + 4, 1>(s) << 4 |
                    bits_at<p + 4 * n + 5, 2>(s) << 5 | bits_at<p + 5 * n + 7, 1>(s) << 7;
            }
            const uint32_t dig = L.trit[T];
            constexpr int moff[5] = {0, n + 2, 2 * n + 4, 3 * n + 5, 4 * n + 7};
            static_for<0, 5>([&](auto ji) {
                constexpr int j = decltype(ji)::value, v = 5 * decltype(gi)::value + j;
                if constexpr (v < V)
                    emit(Idx<v>{}, (((dig >> (2 * j)) & 3u) << n) | bits_at<p + moff[j], n>(s));
            });
        });
    } else if constexpr (e.quint) {
        constexpr int gb = 3 * n + 7;
        ise_groups<3, (V + 2) / 3, B1, B2>(vlim, [&](auto gi) {
            constexpr int p = decltype(gi)::value * gb;
            uint32_t Q;
            if constexpr (n == 0) {
                Q = bits_at<p, 7>(s);
            } else {
                Q = bits_at<p + n, 3>(s) | bits_at<p + 2 * n + 3, 2>(s) << 3 | bits_at<p + 3 * n + 5, 2>(s) << 5;
            }
            const uint32_t dig = L.quint[Q];
            constexpr int moff[3] = {0, n + 3, 2 * n + 5};
            static_for<0, 3>([&](auto ji) {
                constexpr int j = decltype(ji)::value, v = 3 * decltype(gi)::value + j;
                if constexpr (v < V)
                    emit(Idx<v>{}, (((dig >> (3 * j)) & 7u) << n) | bits_at<p + moff[j], n>(s));
            });
        });
    } else {
        ise_groups<1, V, B1, B2>(vlim, [&](auto ji) { emit(ji, bits_at<decltype(ji)::value * n, n>(s)); });
    }
}

// Colour values of range R (4..20): at most 18, and never more than fit in the
// 111 bits after the 17-bit header.
// The values are packed four to a dword (value j in byte j % 4 of dword
// j / 4) and stored as dwords: ColourScratch.
// vlim (wave-uniform): with CAP, the values from vlim on (past 4 or 8) are
// not decoded (their bytes of cv stay zero; the block does not read them).
template <int R, bool CAP = false>
__device__ __attribute__((always_inline)) inline void colour_values(const uint32_t (&s)[4], const LdsTables& L,
                                                                    uint32_t* cv, int vlim = 64) {
    constexpr int V = ise_max_values(R, 18, 111);
    uint32_t w[(V + 3) / 4] = {};
    ise_unpack<R, V, 4, 8>(s, L, CAP ? vlim : 64, [&](auto ji, uint32_t v) {
        constexpr int j = decltype(ji)::value;
        w[j / 4] |= uint32_t(L.color_unq[R][v]) << (8 * (j % 4));
    });
#pragma unroll
    for (int i = 0; i < (V + 3) / 4; ++i) cv[i] = w[i];
}

// Weight fields of trit/quint range R as plain nb-bit fields (nb = bits + 2
// for trits, bits + 3 for quints), field j at bit j * nb of q (five words).
// At most 64 weights, never more than fit in 96 bits.
// vlim: as ise_unpack's (at least the block's weight count).
template <int R>
__device__ __attribute__((always_inline)) inline void weight_fields(const uint32_t (&s)[4], const LdsTables& L,
                                                                    uint32_t (&q)[5], int vlim) {
    constexpr akv::IseRange e = akv::kIse[R];
    constexpr int nb = e.bits + (e.trit ? 2 : 3);
    constexpr int V = ise_max_values(R, 64, 96);
    static_assert(V * nb <= 160, "weight fields fit five words");
#pragma unroll
    for (int i = 0; i < 5; ++i) q[i] = 0;
    if constexpr ((e.trit || e.quint) && e.bits == 0) {
        // No plain bits: a group's table entry (digit j at bit nb * j) is
        // already its fields, so each group is one lookup and one insert.
        constexpr int gs = e.trit ? 5 : 3, gb = e.trit ? 8 : 7;
        static_assert(((V + gs - 1) / gs) * gs * nb <= 160, "whole groups fit five words");
        ise_groups<gs, (V + gs - 1) / gs>(vlim, [&](auto gi) {
            constexpr int g = decltype(gi)::value, P = g * gs * nb, w = P >> 5, o = P & 31;
            const uint32_t dig = e.trit ? L.trit[bits_at<g * gb, gb>(s)] : L.quint[bits_at<g * gb, gb>(s)];
            q[w] |= dig << o;
            if constexpr (o + gs * nb > 32) q[w + 1] |= dig >> (32 - o);
        });
    } else {
        ise_unpack<R, V>(s, L, vlim, [&](auto ji, uint32_t v) {
            constexpr int P = decltype(ji)::value * nb, w = P >> 5, o = P & 31;
            q[w] |= v << o;
            if constexpr (o + nb > 32) q[w + 1] |= v >> (32 - o);
        });
    }
}

// Colour integer sequence of this lane's block: range `crange`, `nv` values
// from bit `start` of the block `blk` (four words in LDS) -> cv (packed bytes).
// With CAP, each pass decodes only up to the largest value count among its
// lanes (4, 8 or all): one luminance partition needs 2 values where a high
// range fits 13.
template <bool CAP = false>
__device__ __attribute__((always_inline)) inline void decode_colour_values(const uint32_t* blk, int start, int crange, int nv, const LdsTables& L,
                                            uint32_t* cv) {
    const uint4 b4 = uint4{blk[0], blk[1], blk[2], blk[3]};   // records are 4-byte aligned
    while (true) {
        const int r = __builtin_amdgcn_readfirstlane(crange);
        if (crange == r) {
            uint32_t s[4] = {b4.x, b4.y, b4.z, b4.w};
            int vlim = 64;
            if constexpr (CAP)   // the lanes of this pass are the active ones
                vlim = __builtin_amdgcn_ballot_w64(nv > 8) ? 64 : __builtin_amdgcn_ballot_w64(nv > 4) ? 8 : 4;
            auto run = [&](auto ri) {
                constexpr int R = decltype(ri)::value;
                shift_and_cut(s, uint32_t(start), ise_seq_bits<R>(nv));
                colour_values<R, CAP>(s, L, cv, vlim);
            };
            switch (r) {
                case 4: run(Idx<4>{}); break;
                case 5: run(Idx<5>{}); break;
                case 6: run(Idx<6>{}); break;
                case 7: run(Idx<7>{}); break;
                case 8: run(Idx<8>{}); break;
                case 9: run(Idx<9>{}); break;
                case 10: run(Idx<10>{}); break;
                case 11: run(Idx<11>{}); break;
                case 12: run(Idx<12>{}); break;
                case 13: run(Idx<13>{}); break;
                case 14: run(Idx<14>{}); break;
                case 15: run(Idx<15>{}); break;
                case 16: run(Idx<16>{}); break;
                case 17: run(Idx<17>{}); break;
                case 18: run(Idx<18>{}); break;
                case 19: run(Idx<19>{}); break;
                default: run(Idx<20>{}); break;
            }
            break;
        }
    }
}

// Weight integer sequence of this lane's block (range `wrange`, `wbits` bits
// of the bit-reversed block `rev`, `count` weights) -> nb-bit fields in q.
// Plain ranges are already nb-bit fields. With CAP, a wave takes one pass
// per distinct (range, cap of the weight count: 16, 36 or 64), the blocks of
// one class sharing both, and decodes only the trit/quint groups below the
// cap (4x4 grids: 16 values rather than up to 41). The uniform branches cost
// about 13 registers: the D=64 kernels (which would spill) and the paged
// kernel (measured slower) decode every value that fits.
template <bool CAP>
__device__ __attribute__((always_inline)) inline void decode_weight_fields(const uint32_t* rev, int wrange, int wbits,
                                                                           int count, const LdsTables& L,
                                                                           uint32_t (&q)[5]) {
    const uint4 r4 = uint4{rev[0], rev[1], rev[2], rev[3]};
    const int key = CAP ? (wrange | ((count <= 16 ? 0 : count <= 36 ? 1 : 2) << 4)) : wrange;
    while (true) {
        const int rk = __builtin_amdgcn_readfirstlane(key);
        if (key == rk) {
            uint32_t s[4] = {r4.x, r4.y, r4.z, r4.w};
            const int r = CAP ? (rk & 15) : rk;
            const int vlim = CAP ? ((rk >> 4) == 0 ? 16 : ((rk >> 4) == 1 ? 36 : 64)) : 64;
            auto run = [&](auto ri) {
                constexpr int R = decltype(ri)::value;
                shift_and_cut(s, 0u, wbits);
                weight_fields<R>(s, L, q, vlim);
            };
            switch (r) {
                case 1: run(Idx<1>{}); break;
                case 3: run(Idx<3>{}); break;
                case 4: run(Idx<4>{}); break;
                case 6: run(Idx<6>{}); break;
                case 7: run(Idx<7>{}); break;
                case 9: run(Idx<9>{}); break;
                case 10: run(Idx<10>{}); break;
                default:   // plain binary: the fields are the reversed stream itself
                    q[0] = r4.x;
                    q[1] = r4.y;
                    q[2] = r4.z;
                    q[3] = r4.w;
                    q[4] = 0;
                    break;
            }
            break;
        }
    }
}

__device__ inline int clamp255(int v) { return v < 0 ? 0 : (v > 255 ? 255 : v); }

__device__ inline void bit_transfer(int& offset, int& base) {
    base = (base >> 1) | (offset & 0x80);
    offset = (offset >> 1) & 0x3F;
    if (offset & 0x20) offset -= 0x40;
}

// Endpoint decode of one partition from its unquantised colour values, bytes
// k .. k + 7 of the packed scratch (k even, at most 16: three dword reads and
// two byte alignments; the dword past a window that starts on a dword
// boundary is not needed, so the read index is clamped to the scratch).
// 8-bit RGBA pairs. False for HDR modes.
constexpr int kColourScratchWords = 6;   // 18 values, and the window's third dword
__device__ inline bool cem_endpoints(int cem, const uint32_t* cv, int k, int* e0, int* e1) {
    const int k4 = k >> 2;
    const uint32_t a = cv[k4], b = cv[k4 + 1], c = cv[min(k4 + 2, kColourScratchWords - 1)];
    const uint32_t lo = __builtin_amdgcn_alignbyte(b, a, uint32_t(k & 3));
    const uint32_t hi = __builtin_amdgcn_alignbyte(c, b, uint32_t(k & 3));
    int v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
        v[j] = (j < 2 * ((cem >> 2) + 1)) ? int(((j < 4 ? lo : hi) >> (8 * (j % 4))) & 0xFFu) : 0;
    // The common modes first (RGB(A) direct, luminance direct): in a wave
    // whose lanes all take them, the rest is one skipped branch rather than a
    // compare per case.
    if (cem == 8 || cem == 12) {
        const int a0 = cem == 12 ? v[6] : 255, a1 = cem == 12 ? v[7] : 255;
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
    if (cem == 0) {
        e0[0] = e0[1] = e0[2] = v[0]; e0[3] = 255;
        e1[0] = e1[1] = e1[2] = v[1]; e1[3] = 255;
        return true;
    }
    switch (cem) {
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
//
// C' is carried biased, as the bits of the float 128 + C' / 65536 (C' in the
// mantissa of 2^7, whose ulp is 2^-16; C' <= 0x10000 < 2^23): the bias folds
// into the add, and one exact subtraction of 128 (Sterbenz) replaces an
// integer-to-float conversion and a scale.
constexpr uint32_t kCBias = 0x43000000u;   // bits of 128.0f

__device__ inline uint32_t interp_c(uint32_t ep, uint32_t wp) {
    typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
    const uint32_t y =
        __builtin_amdgcn_udot2(__builtin_bit_cast(u16x2, ep), __builtin_bit_cast(u16x2, wp), 96u, false);
    return (y >> 6) + (y >> 22) + (kCBias - 1u);
}

// Two biased C' values -> their FP16 values (round toward zero), packed.
__device__ inline uint32_t pack_fp16_rtz(uint32_t c0, uint32_t c1) {
    return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(__builtin_bit_cast(float, c0) - 128.0f,
                                                                   __builtin_bit_cast(float, c1) - 128.0f));
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
        reinterpret_cast<uint16_t*>(tab)[entry] = uint16_t(pack_fp16_rtz(interp_c(ep[0], wp), kCBias));
    }
}

// Table entry of weight 0 (sh = 0, endpoint e0) or 64 (sh = 16, e1): interp_c
// of such a weight is the endpoint e itself, except 0xFFFF -> 0x10000 (FP16
// 1.0).
template <int NCH>
__device__ inline void put_end_entry(uint32_t* tab, int entry, const uint32_t* ep, int sh) {
    uint32_t C[NCH];
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch) {
        const uint32_t e = (ep[ch] >> sh) & 0xFFFFu;
        C[ch] = e + ((e + 1) >> 16) + kCBias;
    }
    if constexpr (NCH == 4) {
        tab[2 * entry] = pack_fp16_rtz(C[0], C[1]);
        tab[2 * entry + 1] = pack_fp16_rtz(C[2], C[3]);
    } else {
        reinterpret_cast<uint16_t*>(tab)[entry] = uint16_t(pack_fp16_rtz(C[0], kCBias));
    }
}

// A constant block (void extent or error colour): one table entry.
template <int NCH>
__device__ inline void set_constant(BlockDesc<NCH>& d, uint32_t r, uint32_t g, uint32_t b, uint32_t a) {
    const uint32_t c[4] = {r, g, b, a};
    uint32_t ep[NCH];
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch) ep[ch] = c[ch] | (c[ch] << 16);
    // Entries 0..3 all hold the colour: a texel reads entry p (one level,
    // weight field 0), whatever partition index p the block's bits select.
#pragma unroll
    for (int e = 0; e < 4; ++e) put_entry<NCH>(d.tab, e, ep, weight_pair(0));
#pragma unroll
    for (int i = 0; i < 5; ++i) d.qw[i] = 0;
    d.info = kInfoTable | kInfoIdentity | (1u << kInfoLevelsShift);
}

// Appends fields (at most 25 bits at a time) to the five-word weight stream
// of a BlockDesc, low bits first. Branch-free: the current partial word is
// stored on every put and overwritten once it fills.
struct FieldWriter {
    uint32_t* out;
    uint32_t cur;
    int bits, words;
    __device__ inline void put(uint32_t v, int len) {   // v < 2^len, 0 <= len <= 25
        const uint64_t a = uint64_t(cur) | (uint64_t(v) << bits);
        const bool full = bits + len >= 32;
        out[words] = uint32_t(a);
        cur = full ? uint32_t(a >> 32) : uint32_t(a);
        bits += len - (full ? 32 : 0);
        words += full ? 1 : 0;
    }
    __device__ inline void finish() {
        out[words] = cur;
        for (int w = words + 1; w < 5; ++w) out[w] = 0;
    }
};

// Before decode_header runs, a block waits in its own BlockDesc::tab:
//   tab[0..3]   the 128-bit block, little endian;
//   tab[8..11]  the block bit-reversed (the weight stream from bit 0), tab[12] = 0.
// BlockDesc::part is not the header stage's: the lane that loaded the block
// writes it (block_part_words) any time before the texel stage.
template <int NCH>
__device__ inline void stash_block(BlockDesc<NCH>& d, uint4 raw) {
    d.tab[0] = raw.x;
    d.tab[1] = raw.y;
    d.tab[2] = raw.z;
    d.tab[3] = raw.w;
    d.tab[8] = __builtin_bitreverse32(raw.w);
    d.tab[9] = __builtin_bitreverse32(raw.z);
    d.tab[10] = __builtin_bitreverse32(raw.y);
    d.tab[11] = __builtin_bitreverse32(raw.x);
    d.tab[12] = 0;
}

// Decode-path class of a block, 0..kPathKeys-1, only a sort key: a hash of
// the bits that fix the block's path through decode_header (block mode,
// partition count, colour endpoint mode or selector; blocks that agree on
// them share weight grid and range, colour range and branches), so sorting a
// chunk's blocks by class keeps the lanes of a wave on one path. Void-extent
// blocks are class kPathKeys - 1. No table lookups.
constexpr int kPathKeys = 64;

__device__ inline int block_path_key(uint4 raw) {
    const uint32_t mode = raw.x & 0x7FF;
    if ((mode & 0x1FF) == 0x1FC) return kPathKeys - 1;
    const uint32_t parts = (raw.x >> 11) & 3;   // partitions - 1
    const uint32_t sel = parts == 0 ? (raw.x >> 13) & 15 : (raw.x >> 23) & 0x3F;
    const uint32_t h = (mode | (parts << 11) | (sel << 13)) * 0x9E3779B1u;
    return int(__umulhi(h, uint32_t(kPathKeys - 1)));   // 0 .. kPathKeys - 2
}

// The partition-pattern table entry a block's bits select (any 128-bit value
// selects an in-range entry; block_part_words zeroes it for one partition).
// A plain load, so that callers can issue it early and use it late.
__device__ inline uint4 partition_words(uint4 raw, const AkvTables* __restrict__ tab) {
    const int parts = int((raw.x >> 11) & 3) + 1;
    return *reinterpret_cast<const uint4*>(tab->partition[max(parts - 2, 0)][(raw.x >> 13) & 0x3FF]);
}

// BlockDesc::part of a block: its pattern words, or zero for one partition.
// (Blocks that decode_header turns into a constant colour may keep any
// pattern: their table repeats the colour in every entry a partition index
// can select.)
__device__ inline uint4 block_part_words(uint4 raw, uint4 words) {
    const bool zero = ((raw.x >> 11) & 3) == 0;
    const uint32_t m = zero ? 0u : ~0u;
    return uint4{words.x & m, words.y & m, words.z & m, words.w & m};
}

// Stage 1: one lane decodes the block stashed in `d` (stash_block) into `d`.
// `cv` is this lane's scratch for the unquantised colour values
// (kColourScratchWords dwords, four values per dword).
// Every table read is from LDS.
// With FILL, a reduced single-plane grid of a footprint of at most 64
// texels is marked kInfoFilled: the caller gives it a slot of its fill area
// (or clears the mark) and runs fill_values before the texel stage.
// CCAP: decode_colour_values<true> (colour values up to the pass's largest count).
// Bits of a weight field as the header stores it (a value of weight range
// r: its plain bits, plus 2 for a trit, 3 for a quint), four bits per range:
// decode_header's NBC variant uses it instead of the table read, whose value
// the register-tight paged kernel spilled across the colour decode.
constexpr uint64_t weight_field_bits() {
    uint64_t t = 0;
    for (int r = 0; r < 12; ++r)
        t |= uint64_t(akv::kIse[r].bits + (akv::kIse[r].trit ? 2 : akv::kIse[r].quint ? 3 : 0)) << (4 * r);
    return t;
}
inline constexpr uint64_t kWeightFieldBits = weight_field_bits();
static_assert(kWeightFieldBits == 0x555444333221ull, "field bits of weight ranges 0-11");

template <int NCH, bool CAP = false, bool FILL = false, bool CCAP = false, bool NBC = false>
__device__ __attribute__((always_inline)) inline void decode_header(const LdsTables& L, BlockDesc<NCH>& d,
                                                                   uint32_t* cv, int ntex = 0) {
    const uint32_t* blk = d.tab;        // block bits
    const uint32_t* rev = d.tab + 8;    // weight stream
    const uint32_t w0 = blk[0];
    const uint32_t mode = w0 & 0x7FF;
    if ((mode & 0x1FF) == 0x1FC) {
        // Void extent: LDR constant colour (UNORM16 RGBA in bits 64..127).
        const uint32_t s0 = stream_bits(blk, 12, 13), s1 = stream_bits(blk, 25, 13);
        const uint32_t t0 = stream_bits(blk, 38, 13), t1 = stream_bits(blk, 51, 13);
        const uint32_t c01 = blk[2], c23 = blk[3];
        const bool unbounded = (s0 & s1 & t0 & t1) == 0x1FFF;
        const bool hdr = (w0 >> 9) & 1;
        if (hdr || (!unbounded && (s0 >= s1 || t0 >= t1))) set_constant(d, 0xFFFF, 0, 0xFFFF, 0xFFFF);
        else set_constant(d, c01 & 0xFFFF, c01 >> 16, c23 & 0xFFFF, c23 >> 16);
        return;
    }
    const uint32_t md = L.block_mode[mode];
    const int parts = int((w0 >> 11) & 3) + 1;
    if (!md || (akv::mode_dual(md) && parts == 4)) {
        set_constant(d, 0xFFFF, 0, 0xFFFF, 0xFFFF);
        return;
    }
    const int wbits = int(akv::mode_wbits(md));
    int below = 128 - wbits;
    int color_start = 17;
    uint32_t cems;  // 4 bits per partition
    if (parts == 1) {
        cems = (w0 >> 13) & 15;
    } else {
        color_start = 29;
        uint32_t sel = (w0 >> 23) & 0x3F;
        if ((sel & 3) == 0) {
            cems = (sel >> 2) * 0x1111u;
        } else {
            const int extra = 3 * parts - 4;
            below -= extra;
            sel |= stream_bits(blk, below, extra) << 6;
            const int base_class = int(sel & 3) - 1;
            cems = 0;
            for (int p = 0; p < parts; ++p) {
                const int up = (sel >> (2 + p)) & 1;
                const int low = (sel >> (2 + parts + 2 * p)) & 3;
                cems |= uint32_t(((base_class + up) << 2) | low) << (4 * p);
            }
        }
    }
    const bool dual = akv::mode_dual(md);
    uint32_t ccs = 0;
    if (dual) {
        below -= 2;
        ccs = stream_bits(blk, below, 2);
    }
    int pairs = 0;
    for (int p = 0; p < parts; ++p) pairs += int((cems >> (4 * p)) & 15) / 4 + 1;
    const int avail = below - color_start;
    const int crange = (pairs <= 9 && avail > 0) ? int(L.color_range[pairs][min(avail, 127)]) : -1;
    if (crange < akv::kRange6) {
        set_constant(d, 0xFFFF, 0, 0xFFFF, 0xFFFF);
        return;
    }
    // Colour integer sequence -> unquantised colour bytes.
    decode_colour_values<CCAP>(blk, color_start, crange, 2 * pairs, L, cv);

    // Weights: the integer sequence runs from bit 127 downwards, so in the
    // bit-reversed block it starts at bit 0; unpacked to nb-bit fields.
    const int wrange = int(akv::mode_range(md));
    int nb;
    if constexpr (NBC) {
        nb = int((kWeightFieldBits >> (4 * wrange)) & 15u);
    } else {
        const uint32_t wi = L.ise[wrange];
        nb = int(wi & 0xFF) + ((wi & 0x100) ? 2 : (wi & 0x200) ? 3 : 0);
    }
    {
        uint32_t q[5];
        const int count = int(akv::mode_gw(md) * akv::mode_gh(md)) << (dual ? 1 : 0);
        decode_weight_fields<CAP>(rev, wrange, wbits, count, L, q);
#pragma unroll
        for (int i = 0; i < 5; ++i) d.qw[i] = q[i];
    }

    // Endpoints per partition -> endpoint pairs, or the texel table. (The
    // table and endpoint pairs overwrite the stash, which is no longer read.)
    const int levels = L.weight_levels[wrange];
    const bool identity = akv::mode_identity(md);
    const bool table = identity && !dual && parts * levels <= BlockDesc<NCH>::kTabEntries;
    // Unquantised weights of the first 8 fields (all an RGBA table row can
    // hold), one LDS read rather than one per entry.
    const uint32_t* wrow_words = reinterpret_cast<const uint32_t*>(&L.weight_unq[wrange][0]);
    const uint2 wrow = {wrow_words[0], wrow_words[1]};
    for (int p = 0, k = 0; p < parts; ++p) {
        const int cem = int((cems >> (4 * p)) & 15);
        int e0[4], e1[4];
        uint32_t ep[NCH];
        if (cem_endpoints(cem, cv, k, e0, e1)) {
#pragma unroll
            for (int ch = 0; ch < NCH; ++ch)   // e * 257 = the byte twice (endpoints are 0..255)
                ep[ch] = __builtin_amdgcn_perm(uint32_t(e1[ch]), uint32_t(e0[ch]), 0x04040000u);
        } else {
            const uint32_t err[4] = {0xFFFFFFFFu, 0u, 0xFFFFFFFFu, 0xFFFFFFFFu};
#pragma unroll
            for (int ch = 0; ch < NCH; ++ch) ep[ch] = err[ch];
        }
        k += 2 * ((cem >> 2) + 1);
        if (table) {
            // One row of `levels` entries per partition (parts * levels fits).
            // Entries are indexed by the raw weight field, whose order is not
            // the weights' order for trit and quint ranges with extra bits;
            // field 0 always unquantises to weight 0, i.e. endpoint e0.
            put_end_entry<NCH>(d.tab, p * levels, ep, 0);
#pragma unroll
            for (int q = 1; q < BlockDesc<NCH>::kTabEntries; ++q) {
                if (q >= levels) break;
                const int w = q < 8 ? int(((q < 4 ? wrow.x : wrow.y) >> (8 * (q & 3))) & 0xFFu)
                                    : int(L.weight_unq[wrange][q]);
                put_entry<NCH>(d.tab, p * levels + q, ep, weight_pair(w));
            }
        } else {
#pragma unroll
            for (int ch = 0; ch < NCH; ++ch) d.ep[p][ch] = ep[ch];
        }
    }
    const bool fill = FILL && !identity && !dual && ntex <= 64;
    d.info = (md & 0xFFu) | (dual ? kInfoDual : 0u) | (ccs << 9) | (uint32_t(nb) << kInfoNbShift) |
             (uint32_t(wrange) << kInfoRangeShift) | (uint32_t(levels) << kInfoLevelsShift) |
             (identity ? kInfoIdentity : 0u) | (table ? kInfoTable : 0u) |
             (fill ? kInfoFilled : 0u);
}

// Weight field `idx` (grid order, planes interleaved) of a block.
template <int NCH>
__device__ inline uint32_t field_at(const BlockDesc<NCH>& d, uint32_t nb, int idx) {
    const uint32_t pos = __umul24(uint32_t(idx), nb), w = pos >> 5;
    return __builtin_amdgcn_ubfe(__builtin_amdgcn_alignbit(d.qw[w + 1], d.qw[w], pos & 31), 0, nb);
}

// Unquantised, infilled weight of texel (x, y) on plane `plane` (compute path).
// bx: footprint width; ds, dt: the footprint's infill steps.
template <int NCH>
__device__ inline int texel_weight(const BlockDesc<NCH>& d, const LdsTables& L, int bx, int ds, int dt, uint32_t info,
                                   int x, int y, int plane) {
    const uint32_t nb = (info >> kInfoNbShift) & 7;
    const uint8_t* unq = L.weight_unq[(info >> kInfoRangeShift) & 15];
    const int sh = (info & kInfoDual) ? 1 : 0;
    if (info & kInfoIdentity) return unq[field_at(d, nb, ((y * bx + x) << sh) + plane)];
    const int gw = int(info & 15), gh = int((info >> 4) & 15);
    const int gs = (ds * x * (gw - 1) + 32) >> 6, gt = (dt * y * (gh - 1) + 32) >> 6;
    const int fs = gs & 15, ft = gt & 15, base = (gs >> 4) + (gt >> 4) * gw;
    const int f11 = (fs * ft + 8) >> 4, f01 = fs - f11, f10 = ft - f11, f00 = 16 - fs - ft + f11;
    // Taps with a zero factor may lie outside the grid: read the base tap instead.
    const int i01 = f01 ? base + 1 : base, i10 = f10 ? base + gw : base, i11 = f11 ? base + gw + 1 : base;
    return (unq[field_at(d, nb, (base << sh) + plane)] * f00 + unq[field_at(d, nb, (i01 << sh) + plane)] * f01 +
            unq[field_at(d, nb, (i10 << sh) + plane)] * f10 + unq[field_at(d, nb, (i11 << sh) + plane)] * f11 + 8) >>
           4;
}

// Stage 2, compute path (blocks that are not a table): kept out of line, so
// the table path that nearly every block takes stays small where it is
// inlined. `p` is the texel's partition; scalars are passed by value so that
// nothing of the caller's has to live in memory for the call.
template <int NCH>
__device__ __attribute__((noinline)) uint2 texel_compute(const BlockDesc<NCH>& d, const LdsTables& L, int bx, int ds,
                                                         int dt, int x, int y, int p) {
    const uint32_t info = d.info;
    const uint32_t wp0 = weight_pair(texel_weight(d, L, bx, ds, dt, info, x, y, 0));
    const uint32_t wp1 =
        (info & kInfoDual) ? weight_pair(texel_weight(d, L, bx, ds, dt, info, x, y, 1)) : wp0;
    const int ccs = (info & kInfoDual) ? int((info >> 9) & 3) : 4;
    uint32_t C[NCH];
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch) C[ch] = interp_c(d.ep[p][ch], ch == ccs ? wp1 : wp0);
    if constexpr (NCH == 4) return uint2{pack_fp16_rtz(C[0], C[1]), pack_fp16_rtz(C[2], C[3])};
    else return uint2{pack_fp16_rtz(C[0], kCBias) & 0xFFFFu, 0u};
}

// Stage 2, compute path of a block with one weight plane and a weight grid
// the size of the block (texel i reads weight field i): inlined for RGBA,
// since at RGBA 4x4 most blocks (two partitions, 5-10 weight levels) have
// more entries than a table holds and take this path. (A scalar table holds
// 32 entries, so scalar blocks rarely miss it.)
template <int NCH>
__device__ inline uint2 texel_identity(const BlockDesc<NCH>& d, const LdsTables& L, uint32_t info, int i, int p) {
    const uint32_t nb = (info >> kInfoNbShift) & 7;
    const uint32_t wp = weight_pair(L.weight_unq[(info >> kInfoRangeShift) & 15][field_at(d, nb, i)]);
    uint32_t C[NCH];
#pragma unroll
    for (int ch = 0; ch < NCH; ++ch) C[ch] = interp_c(d.ep[p][ch], wp);
    if constexpr (NCH == 4) return uint2{pack_fp16_rtz(C[0], C[1]), pack_fp16_rtz(C[2], C[3])};
    else return uint2{pack_fp16_rtz(C[0], kCBias) & 0xFFFFu, 0u};
}

// Stage 1b: the texels of the kInfoFilled blocks `list[0..n)` (block
// list[e] has slot e), by whole waves, one lane per texel: a wave takes
// 64 / span blocks per pass (span: the texel count rounded up to 16, 32 or
// 64, so ntex <= 64). Each lane infills its texel's weight, finds its
// partition and interpolates the endpoints, into `fa`. A workgroup barrier
// must follow before the texel stage.
template <int NCH, int NT>
__device__ inline void fill_values(const BlockDesc<NCH>* desc, const LdsTables& L, Footprint f, const uint8_t* list,
                                   int n, FillArea<NCH>& fa, int tid) {
    const int span = f.ntex <= 16 ? 16 : f.ntex <= 32 ? 32 : 64;
    const int per = 64 / span;
    const int lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int sub = lane / span, t = lane & (span - 1);
    const int y = int((float(t) + 0.5f) * (1.0f / float(f.bx)));   // t < 64, bx <= 12: exact
    const int x = t - y * f.bx;
    for (int base = wave * per; base < n; base += (NT / 64) * per) {
        const int e = base + sub;
        if (e < n && t < f.ntex) {
            const BlockDesc<NCH>& d = desc[list[e]];
            const uint32_t info = d.info;
            const uint32_t wp = weight_pair(texel_weight(d, L, f.bx, f.ds, f.dt, info, x, y, 0));
            const int p = int(__builtin_amdgcn_ubfe(d.part[t >> 4], uint32_t(2 * t), 2));
            uint32_t C[NCH];
#pragma unroll
            for (int ch = 0; ch < NCH; ++ch) C[ch] = interp_c(d.ep[p][ch], wp);
            const int slot = e * f.ntex + t;
            if constexpr (NCH == 4)
                *reinterpret_cast<uint2*>(&fa.v[4 * slot]) = uint2{pack_fp16_rtz(C[0], C[1]), pack_fp16_rtz(C[2], C[3])};
            else
                fa.v[slot] = uint16_t(pack_fp16_rtz(C[0], kCBias));
        }
    }
}

// Stage 2 of a kInfoFilled block: its texel from the fill area.
template <int NCH>
__device__ inline uint2 texel_filled(const FillArea<NCH>& fa, uint32_t info, int i, int ntex) {
    const int slot = int(info >> kInfoFillShift) * ntex + i;
    if constexpr (NCH == 4) return *reinterpret_cast<const uint2*>(&fa.v[4 * slot]);
    else return uint2{uint32_t(fa.v[slot]), 0u};
}

// Stage 2: the FP16 values of texel (x, y) of a block (NCH == 4:
// {R | G << 16, B | A << 16}; NCH == 1: R in the low half of .x).
template <int NCH>
__device__ inline uint2 texel_fp16(const BlockDesc<NCH>& d, const LdsTables& L, Footprint f, int x, int y) {
    const uint32_t info = d.info;
    const int i = y * f.bx + x;
    const int p = int(__builtin_amdgcn_ubfe(d.part[i >> 4], 2 * (i & 15), 2));
    if (info & kInfoTable) {
        const uint32_t nb = (info >> kInfoNbShift) & 7;
        const int entry = p * int((info >> kInfoLevelsShift) & 63) + int(field_at(d, nb, i));
        if constexpr (NCH == 4) return uint2{d.tab[2 * entry], d.tab[2 * entry + 1]};
        else return uint2{reinterpret_cast<const uint16_t*>(d.tab)[entry], 0u};
    }
    return texel_compute<NCH>(d, L, f.bx, f.ds, f.dt, x, y, p);
}

// Stage 2 for K texels at once, the way the attention loop needs them: the
// table lookups of all K are straight-line code (their LDS reads issue
// together), and the compute path runs only where a block needs it. The
// table read of a block that is not a table may land anywhere in the first
// kilobyte past its record (entry < 128); its value is replaced.
// FILL: the kernel runs the fill stage (kInfoFilled blocks are in `fa`).
template <int NCH, int K, bool FILL>
__device__ inline void texels_fp16(const BlockDesc<NCH>* desc, const int (&blk)[K], const int (&i)[K],
                                   const int (&x)[K], const int (&y)[K], const LdsTables& L, Footprint f,
                                   const FillArea<NCH>* fa, uint2 (&out)[K]) {
    uint32_t info[K];
    int p[K];
    bool all_table = true;
#pragma unroll
    for (int k = 0; k < K; ++k) {
        info[k] = desc[blk[k]].info;
        // v_bfe_u32 reads its offset mod 32: 2 * i selects bits 2 * (i % 16).
        p[k] = int(__builtin_amdgcn_ubfe(desc[blk[k]].part[i[k] >> 4], uint32_t(2 * i[k]), 2));
    }
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const BlockDesc<NCH>& d = desc[blk[k]];
        const uint32_t nb = (info[k] >> kInfoNbShift) & 7;
        const int entry = int(__umul24(uint32_t(p[k]), (info[k] >> kInfoLevelsShift) & 63)) + int(field_at(d, nb, i[k]));
        if constexpr (NCH == 4) out[k] = uint2{d.tab[2 * entry], d.tab[2 * entry + 1]};
        else out[k] = uint2{reinterpret_cast<const uint16_t*>(d.tab)[entry], 0u};
        all_table = all_table && (info[k] & kInfoTable);
    }
    if (!all_table) {
#pragma unroll
        for (int k = 0; k < K; ++k)
            if (!(info[k] & kInfoTable)) {
                if (FILL && (info[k] & kInfoFilled))
                    out[k] = texel_filled<NCH>(*fa, info[k], i[k], f.ntex);
                else if (NCH == 4 && (info[k] & (kInfoIdentity | kInfoDual)) == kInfoIdentity)
                    out[k] = texel_identity<NCH>(desc[blk[k]], L, info[k], i[k], p[k]);
                else
                    out[k] = texel_compute<NCH>(desc[blk[k]], L, f.bx, f.ds, f.dt, x[k], y[k], p[k]);
            }
    }
}

}  // namespace akv_hip
