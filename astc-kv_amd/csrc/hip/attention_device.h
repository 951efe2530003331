// Device code shared by the split kernels (contiguous and paged atlases):
// workgroup shape, the grouped MFMA attention of one tile group, the wave and
// split-state combine, the in-kernel merge, and the texel-column operand
// builders over the header stage's block descriptors.
//
// Reference semantics: metal/attention_gqa_v10.metal:168-225 (online softmax,
// factored token affine acc = sum p*s*u + sum p*o) and :229-253 (exact merge
// of split states).
#pragma once
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>

#include "astc_decode_device.h"
#include "astc_format.h"
#include "astc_kv_hip.h"

namespace akv_hip {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr uint64_t kCUs = 256;   // compute units of an MI355X (gfx950)
constexpr int kMaxG = 8;   // query heads per kv head
#ifndef AKV_ASTC_WAVES
#define AKV_ASTC_WAVES 3   // waves per SIMD the split kernel is register-limited to
#endif

typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

// WIDE: the launch has at most one workgroup per CU (small batches, few
// splits), so LDS has room for a full 256-block chunk at head dim 64 too:
// fewer chunks, hence a shorter critical path, per split.
// MAXB: blocks per chunk when not 0 (a kernel that needs less LDS).
template <int D, int NCH, bool WIDE = false, int MAXB = 0>
struct Cfg {
    // Blocks per chunk (header stage, one per lane): at head dim 128 the
    // kernel runs two workgroups per CU, which leaves room for a full 256.
    static constexpr int kMaxBlocks = MAXB ? MAXB : (D == 64 && !WIDE) ? 160 : 256;
    static constexpr int kMaxTok = D == 64 ? 320 : 128;          // tokens per chunk
    static constexpr int kMaxTiles = kMaxTok / 16;
    static constexpr int kWaveTiles = kMaxTiles / kWaves;        // tiles per wave per chunk
    static constexpr int kRowLoads = D / 32;                     // K: 16-byte loads per lane per tile
    static constexpr int kKSteps = D / 16;
    static constexpr int kMBlocks = D / 16;
    static constexpr int kColGroups = NCH == 4 ? D / 64 : D / 16; // texel columns per lane
    static constexpr int kRowBlocksPerGroup = NCH == 4 ? 4 : 1;    // P.V row blocks fed by one column
};

struct KernelArgs {
    AkvAttnParams p;
    Footprint fp;
    uint32_t chunk_tokens;   // tokens per full chunk
    uint32_t mag_by, mag_bx; // ceil(2^24 / divisor)
    float qscale;            // log2(e) / sqrt(dim)
    uint32_t wide;           // the split kernel's Cfg<..., WIDE = true> variant
};

// a / d with magic = ceil(2^24 / d): exact when a * d < 2^24 (the error term
// a * (magic * d - 2^24) stays below 2^24), which holds for every use below;
// a and magic fit 24 bits and a * magic fits 32, so one 24-bit multiply.
__device__ inline uint32_t fdiv(uint32_t a, uint32_t magic) { return __umul24(a, magic) >> 24; }
__device__ inline float half_to_float(uint16_t h) { return float(__builtin_bit_cast(_Float16, h)); }

// Channel held by row `row` of MFMA row block `mb` of P.V. RGBA texels (and the
// FP16 control) feed row blocks 4k + j with channel j of texel column
// 16k + row; scalar texels feed row block k with texel column 16k + row.
template <int NCH>
__device__ inline int pv_channel(int mb, int row) {
    if constexpr (NCH == 4) return 64 * (mb >> 2) + 4 * row + (mb & 3);
    else return 16 * mb + row;
}

// Grouped attention. One 16x16x16 MFMA output holds TPG 16-token tiles x Gs
// head slots: rows r = t * Gs + h (tile t of the group, query head h), so that
// for G <= 4 the softmax runs on 4 head slots instead of the 16 columns of one
// tile. Q is block-diagonal (row r sees only the K rows of tile t), P likewise
// for P.V; the MFMA count is the same as one tile at a time.
template <int G, int D>
struct Grp {
    // Head slots per tile: 4 when G <= 4, except at head dim 128, where the K
    // rows of four tiles (64 registers) do not fit beside the rest.
    static constexpr int Gs = (G <= 4 && D <= 64) ? 4 : 8;
    static constexpr int TPG = 16 / Gs;          // tiles per group
};

// Q as the B operand of the block-diagonal S^T = K.Q^T, split into fp16 high
// and low parts, kept in LDS (the same for every wave): qs[2 * ks + part][lane]
// for lane (column r, g) holds head r % Gs, dims 32*(ks/2) + 8*g + 4*(ks%2) + j
// (j = 0..3), matching the K row loads. Loaded and stored by the first wave,
// in two halves so that a kernel can issue the loads early: `qrow` is 16-byte
// aligned, every load is unconditional (slots h >= G read head G - 1 and are
// zeroed).
template <int D, int G>
struct QStage {
    float4 x[D / 16];
    __device__ void load(const float* __restrict__ qrow) {
        const int lane = threadIdx.x & 63, h = (lane & 15) % Grp<G, D>::Gs, g = lane >> 4;
        const float* src = qrow + size_t(min(h, G - 1)) * D + 8 * g;
#pragma unroll
        for (int ks = 0; ks < D / 16; ++ks)
            x[ks] = *reinterpret_cast<const float4*>(src + 32 * (ks / 2) + 4 * (ks % 2));
    }
    __device__ void store(float qscale, uint2* qs) const {
        const int lane = threadIdx.x & 63, h = (lane & 15) % Grp<G, D>::Gs;
#pragma unroll
        for (int ks = 0; ks < D / 16; ++ks) {
            const float e[4] = {x[ks].x, x[ks].y, x[ks].z, x[ks].w};
            half4 hi, lo;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float v = h < G ? e[j] * qscale : 0.0f;
                hi[j] = _Float16(v);
                lo[j] = _Float16(v - float(hi[j]));
            }
            qs[(2 * ks) * 64 + lane] = __builtin_bit_cast(uint2, hi);
            qs[(2 * ks + 1) * 64 + lane] = __builtin_bit_cast(uint2, lo);
        }
    }
};

template <int D, int G>
__device__ inline void store_q(const float* __restrict__ qrow, float qscale, uint2* qs) {
    QStage<D, G> st;
    st.load(qrow);
    st.store(qscale, qs);
}

__device__ inline half4 masked(uint2 v, uint32_t m) { return __builtin_bit_cast(half4, uint2{v.x & m, v.y & m}); }

// Cross-lane all-reductions over the lanes whose index agrees with this
// lane's in the bits below `from` (a power of two, 4 .. 32): DPP row rotations
// inside each 16-lane row, then the gfx950 row-swap moves across rows (with
// both operands the same register, the two results of a swap hold the two
// halves being combined, so op(first, second) is already the all-reduce).
// Vector elements are copied to scalars before __builtin_bit_cast: applied to
// an element of an ext_vector_type value directly it reads element 0.
template <typename Op>
__device__ inline float lane_allreduce(float v, int from, Op op) {
    auto f32 = [](uint32_t u) { return __builtin_bit_cast(float, u); };
    auto u32 = [](float f) { return __builtin_bit_cast(uint32_t, f); };
    if (from <= 4) v = op(v, f32(__builtin_amdgcn_mov_dpp(int(u32(v)), 0x124, 0xF, 0xF, false)));
    if (from <= 8) v = op(v, f32(__builtin_amdgcn_mov_dpp(int(u32(v)), 0x128, 0xF, 0xF, false)));
    if (from <= 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(u32(v), u32(v), false, false);
        const uint32_t a = r[0], b = r[1];
        v = op(f32(a), f32(b));
    }
    const auto r = __builtin_amdgcn_permlane32_swap(u32(v), u32(v), false, false);
    const uint32_t a = r[0], b = r[1];
    return op(f32(a), f32(b));
}
struct MaxOp { __device__ float operator()(float a, float b) const { return fmaxf(a, b); } };
struct AddOp { __device__ float operator()(float a, float b) const { return a + b; } };

// A lane mask the optimizer cannot see through (keeps selects on it as plain
// bit operations instead of dynamic vector indexing).
__device__ inline uint32_t opaque_mask(bool c) {
    uint32_t m = c ? ~0u : 0u;
    asm volatile("" : "+v"(m));
    return m;
}

// Inclusive prefix sum over the 64 lanes of a wave, without LDS: DPP row
// shifts (1, 2, 4, 8; lanes shifted in from outside the 16-lane row read 0)
// scan each row, then each row adds the totals of the rows before it (read
// with readlane).
__device__ inline uint32_t wave_inclusive_scan(uint32_t v) {
    v += uint32_t(__builtin_amdgcn_update_dpp(0, int(v), 0x111, 0xF, 0xF, false));   // row_shr:1
    v += uint32_t(__builtin_amdgcn_update_dpp(0, int(v), 0x112, 0xF, 0xF, false));   // row_shr:2
    v += uint32_t(__builtin_amdgcn_update_dpp(0, int(v), 0x114, 0xF, 0xF, false));   // row_shr:4
    v += uint32_t(__builtin_amdgcn_update_dpp(0, int(v), 0x118, 0xF, 0xF, false));   // row_shr:8
    const uint32_t r0 = uint32_t(__builtin_amdgcn_readlane(int(v), 15));
    const uint32_t r1 = uint32_t(__builtin_amdgcn_readlane(int(v), 31));
    const uint32_t r2 = uint32_t(__builtin_amdgcn_readlane(int(v), 47));
    const int row = int(threadIdx.x & 63) >> 4;
    return v + (row >= 1 ? r0 : 0u) + (row >= 2 ? r1 : 0u) + (row >= 3 ? r2 : 0u);
}

// Second half of the counting sort of a chunk's blocks by decode-path class
// (after the class counts are complete): every wave scans the 64 counts
// itself and writes the sorted positions of its own blocks; the base of a
// lane's class comes from the scanning lane of that class.
__device__ inline void place_by_class(const uint32_t* key_count, uint8_t* order, int key, int rank, bool mine,
                                      int tid) {
    const uint32_t c = key_count[tid & 63];
    const uint32_t excl = wave_inclusive_scan(c) - c;
    const uint32_t base = uint32_t(__shfl(int(excl), key, 64));
    if (mine) order[base + uint32_t(rank)] = uint8_t(tid);
}

// Buffer resource over `bytes` bytes from `base` (raw, stride 0): loads past
// the end return zero without touching memory.
__device__ inline __amdgpu_buffer_rsrc_t seq_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, int(bytes), 0x00020000);
}

// K rows of one 16-token tile as the A operand (lane (token, g) holds dims
// 32 * L + 8 * g .. + 7 in kreg[L]); rs covers the tokens that exist, so rows
// past them read as zero.
template <int D>
__device__ inline void load_k_tile(uint4* r, __amdgpu_buffer_rsrc_t rs, int t0, int lane) {
    const uint32_t tok = uint32_t(t0 + (lane & 15)), g = uint32_t(lane >> 4);
#pragma unroll
    for (int L = 0; L < D / 32; ++L) {
        const auto v = __builtin_amdgcn_raw_buffer_load_b128(rs, 2 * (tok * D + 32 * L + 8 * g), 0, 0);
        r[L] = uint4{v[0], v[1], v[2], v[3]};
    }
}

// Softmax state of one wave. In the row layout (lane (r, g): tile r / Gs,
// head r % Gs) m is the head's running maximum (log2 units) and l, off are
// this lane's partial sums; o[mb] are the P.V accumulators in the MFMA output
// layout (lane (channel, g): rows 4g .. 4g+3).
template <int D>
struct AttnState {
    float m, l, off;
    floatx4 o[D / 16];
};

// One group of up to TPG tiles (ng of them exist) starting at chunk token tb0:
// kop supplies tile t's K operands (above); vtile(t, kc, va) produces tile t's
// V operands for row blocks MPB*kc .. MPB*kc + MPB-1 (lane (row, g): tokens
// 4g..4g+3 of the tile), called with kc = 0, 1, ... in order for each tile.
// so: per-token scale | offset << 16 for the chunk (AFFINE).
// K operands of the S stage. kop(t, ks, qh, ql, acc) adds tile t's k-step ks
// (dims 32*(ks/2) + 8g + 4*(ks%2) + 0..3 of the lane's token row) times the Q
// operand halves to acc.
//
// FP16 K rows: kreg[t * D/32 + L] holds dims 32L + 8g .. + 7 of the lane's row.
template <int D>
struct Fp16KOperands {
    const uint4* kreg;
    __device__ inline floatx4 operator()(int t, int ks, half4 qh, half4 ql, floatx4 acc) const {
        const uint4 kk = kreg[t * (D / 32) + ks / 2];
        const half4 ka = __builtin_bit_cast(half4, (ks & 1) ? uint2{kk.z, kk.w} : uint2{kk.x, kk.y});
        acc = __builtin_amdgcn_mfma_f32_16x16x16f16(ka, qh, acc, 0, 0, 0);
        return __builtin_amdgcn_mfma_f32_16x16x16f16(ka, ql, acc, 0, 0, 0);
    }
};

// 4-bit K in groups of 32 channels (codec.py:218-250 with axis="token",
// group=32): kq[t * 2*(D/32) + L] holds the 8 codes of dims 32L + 8g .. + 7
// (low nibble = even dim), kq[t * 2*(D/32) + D/32 + L] group L's (offset,
// scale) fp16 pair. k = code * scale + offset in fp32 (the product is exact,
// so this is the reference's float32 dequantisation), split into fp16 high
// and low parts: three MFMAs (k_hi q_hi + k_hi q_lo + k_lo q_hi).
template <int D>
struct U4KOperands {
    const uint32_t* kq;
    __device__ inline floatx4 operator()(int t, int ks, half4 qh, half4 ql, floatx4 acc) const {
        const uint32_t codes = kq[t * (D / 16) + ks / 2] >> (16 * (ks & 1));
        const uint32_t os = kq[t * (D / 16) + D / 32 + ks / 2];
        const float o = float(__builtin_bit_cast(_Float16, uint16_t(os)));
        const float sc = float(__builtin_bit_cast(_Float16, uint16_t(os >> 16)));
        float kv[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) kv[j] = fmaf(float(__builtin_amdgcn_ubfe(codes, 4 * j, 4)), sc, o);
        const uint32_t h01 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(kv[0], kv[1]));
        const uint32_t h23 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(kv[2], kv[3]));
        auto lo16 = [](uint32_t w) { return float(__builtin_bit_cast(_Float16, uint16_t(w))); };
        auto hi16 = [](uint32_t w) { return float(__builtin_bit_cast(_Float16, uint16_t(w >> 16))); };
        const uint32_t l01 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(kv[0] - lo16(h01), kv[1] - hi16(h01)));
        const uint32_t l23 = __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_pkrtz(kv[2] - lo16(h23), kv[3] - hi16(h23)));
        const half4 khi = __builtin_bit_cast(half4, uint2{h01, h23});
        const half4 klo = __builtin_bit_cast(half4, uint2{l01, l23});
        acc = __builtin_amdgcn_mfma_f32_16x16x16f16(khi, qh, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x16f16(khi, ql, acc, 0, 0, 0);
        return __builtin_amdgcn_mfma_f32_16x16x16f16(klo, qh, acc, 0, 0, 0);
    }
};

template <int D, int G, bool AFFINE, int MPB, int TPGMAX = Grp<G, D>::TPG, typename KOp, typename VTile>
__device__ __attribute__((always_inline)) inline void attend_group(const KOp& kop, const uint2* qs, int ng, int tb0,
                                                                   int ntok, const uint32_t* so, int so_cap,
                                                                   AttnState<D>& st, VTile&& vtile) {
    constexpr int Gs = Grp<G, D>::Gs, TPG = TPGMAX;   // TPGMAX <= Grp's TPG: fewer tiles per group
    static_assert(TPGMAX >= 1 && TPGMAX <= Grp<G, D>::TPG, "tiles per group");
    const int lane = threadIdx.x & 63, n16 = lane & 15, g = lane >> 4;
    const int rt = n16 / Gs, h = n16 % Gs;   // this lane's row of S and P: tile, head
    // S^T = K . Q^T per tile, K rows as the A operand and Q as the B operand:
    // output lane (column r, g) of tile t holds head r % Gs's scores for tokens
    // 4g .. 4g+3 of tile t, the layout P needs as an A operand. Lane (r, g)
    // keeps tile r / Gs. The Q operands are read from LDS here rather than
    // kept in registers (the asm statement keeps the compiler from hoisting
    // them out of the loop).
    asm volatile("" ::: "memory");
    floatx4 sacc[TPG];
#pragma unroll
    for (int t = 0; t < TPG; ++t) sacc[t] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
        const half4 qh = __builtin_bit_cast(half4, qs[(2 * ks) * 64 + lane]);
        const half4 ql = __builtin_bit_cast(half4, qs[(2 * ks + 1) * 64 + lane]);
#pragma unroll
        for (int t = 0; t < TPG; ++t) {
            if (t >= ng) break;
            sacc[t] = kop(t, ks, qh, ql, sacc[t]);
        }
    }
    uint32_t tmask[TPG];   // lane keeps tile t
#pragma unroll
    for (int t = 0; t < TPG; ++t) tmask[t] = opaque_mask(rt == t);
    float x[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint32_t xb = 0;
#pragma unroll
        for (int t = 0; t < TPG; ++t) {
            const float e = sacc[t][i];
            xb |= __builtin_bit_cast(uint32_t, e) & tmask[t];
        }
        x[i] = __builtin_bit_cast(float, xb);
    }
    const int tb = tb0 + 16 * rt + 4 * g;   // chunk token of x[0]
    float mt = -INFINITY;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        if (h < G && rt < ng && tb + i < ntok) mt = fmaxf(mt, x[i]);
    mt = lane_allreduce(mt, Gs, MaxOp{});
    const float m_new = fmaxf(st.m, mt);
    const float mref = m_new == -INFINITY ? 0.0f : m_new;   // rows with no token yet
    // v_exp_f32 directly: ~1 ulp for normal results; results below 2^-126 of
    // the running maximum flush to zero.
    const float alpha = __builtin_amdgcn_exp2f(st.m - mref);
    st.m = m_new;
    uint4 so4 = uint4{0x3C00u, 0x3C00u, 0x3C00u, 0x3C00u};   // scale 1, offset 0
    if constexpr (AFFINE) so4 = *reinterpret_cast<const uint4*>(&so[min(tb, so_cap - 4)]);
    const uint32_t sov[4] = {so4.x, so4.y, so4.z, so4.w};
    float psum = 0.0f, poff = 0.0f;
    half4 phi, plo;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const bool ok = h < G && rt < ng && tb + i < ntok;
        const float pr = ok ? __builtin_amdgcn_exp2f(x[i] - mref) : 0.0f;
        psum += pr;
        float pv = pr;
        if constexpr (AFFINE) {   // rows or tokens that do not exist: scale = offset = 0
            const uint32_t sv = ok ? sov[i] : 0u;
            pv = pr * half_to_float(uint16_t(sv));
            poff = fmaf(pr, half_to_float(uint16_t(sv >> 16)), poff);
        }
        const _Float16 hh = _Float16(pv);
        phi[i] = hh;
        plo[i] = _Float16(pv - float(hh));
    }
    st.l = fmaf(st.l, alpha, psum);
    st.off = fmaf(st.off, alpha, poff);
    // Rescale the accumulators by their row's alpha when any maximum moved:
    // output row 4g + i has head (4g + i) % Gs, whose alpha lane h = row holds.
    if (__builtin_amdgcn_ballot_w64(alpha != 1.0f)) {
        float ar[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if constexpr (Gs == 4) {
                ar[i] = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, alpha), i));
            } else {
                const float a0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, alpha), i));
                const float a1 =
                    __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, alpha), 4 + i));
                ar[i] = (g & 1) ? a1 : a0;
            }
        }
#pragma unroll
        for (int mb = 0; mb < D / 16; ++mb)
#pragma unroll
            for (int i = 0; i < 4; ++i) st.o[mb][i] *= ar[i];
    }
    const uint2 phib = __builtin_bit_cast(uint2, phi), plob = __builtin_bit_cast(uint2, plo);
    // O += Pbd . V per tile, one column group of V operands at a time (MPB
    // row blocks each), so that only one group's operands are live.
#pragma unroll
    for (int t = 0; t < TPG; ++t) {
        if (t >= ng) break;
        const half4 ah = masked(phib, tmask[t]), al = masked(plob, tmask[t]);
#pragma unroll
        for (int kc = 0; kc < D / 16 / MPB; ++kc) {
            half4 va[MPB];
            vtile(t, kc, va);
#pragma unroll
            for (int j = 0; j < MPB; ++j) {
                const int mb = kc * MPB + j;
                st.o[mb] = __builtin_amdgcn_mfma_f32_16x16x16f16(ah, va[j], st.o[mb], 0, 0, 0);
                st.o[mb] = __builtin_amdgcn_mfma_f32_16x16x16f16(al, va[j], st.o[mb], 0, 0, 0);
            }
        }
    }
}

struct WaveStats {
    float wm[kWaves][kMaxG], wl[kWaves][kMaxG], wo[kWaves][kMaxG];
    int last;   // this workgroup is the last split of its (sequence, kv head) to finish
};

// Merge done by the split kernel itself: after writing its split state, a
// workgroup counts itself in `arrival` (one counter per (sequence, kv head));
// the last of the S workgroups merges the G query heads' S states into `out`
// exactly as merge_kernel does, and leaves the counter at zero for the next
// launch. No workgroup waits for another.
// Ordering is the memory model's release/acquire pair, not a hardware
// argument: every wave's state stores happen before the workgroup barrier;
// the first lane then issues an agent-scope release fence and the counter
// increment, and the workgroup whose increment completes the count issues an
// agent-scope acquire fence before its barrier, so the states of all S
// workgroups (on any XCD) happen before its loads. The states themselves are
// written and read with agent-scope atomic accesses.
// S: splits of this (sequence, kv head); SS: the split stride of partial and
// stats (S for a uniform batch).
template <int D, int G>
__device__ inline void merge_if_last(uint32_t* arrival, const float* partial, const float2* stats,
                                     float* __restrict__ out, size_t qh0, int S, int SS, WaveStats& ws, float* lds,
                                     int lds_floats) {
    // Each wave's state stores complete before the barrier (the workgroup
    // barrier alone does not wait for global stores to be acknowledged).
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        const bool last =
            __hip_atomic_fetch_add(arrival, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == uint32_t(S - 1);
        if (last) __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
        ws.last = last;
    }
    __syncthreads();
    if (!ws.last) return;
    const int tid = threadIdx.x;
    auto load = [](const float* x) { return __hip_atomic_load(x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); };
    auto load2 = [](const float2* x) {
        return __builtin_bit_cast(float2, __hip_atomic_load(reinterpret_cast<const uint64_t*>(x), __ATOMIC_RELAXED,
                                                            __HIP_MEMORY_SCOPE_AGENT));
    };
    if (2 * G * S + 2 * G <= lds_floats) {
        // Stats of the G heads' S splits into LDS (one load each, all in flight),
        // then per head the maximum, the split weights e^(m_s - M) and the sum l.
        float2* w = reinterpret_cast<float2*>(lds);   // [G][S]: (m, l) -> (weight, -)
        float* linv = lds + 2 * G * S;                // [G]: 1 / sum of weighted l
        for (int i = tid; i < G * S; i += kThreads) {
            const int hh = i / S;
            w[i] = load2(&stats[(qh0 + hh) * SS + (i - hh * S)]);
        }
        __syncthreads();
        if (tid < G) {
            float M = -INFINITY, l = 0.0f;
            for (int sp = 0; sp < S; ++sp) M = fmaxf(M, w[tid * S + sp].x);
            for (int sp = 0; sp < S; ++sp) {
                const float2 ms = w[tid * S + sp];
                const float e = ms.x == -INFINITY ? 0.0f : expf(ms.x - M);
                w[tid * S + sp].x = e;
                l = fmaf(ms.y, e, l);
            }
            linv[tid] = 1.0f / l;
        }
        __syncthreads();
        for (int i = tid; i < G * D; i += kThreads) {
            const int hh = i / D, c = i - hh * D;
            const float* src = partial + (qh0 + hh) * size_t(SS) * D + c;
            float acc = 0.0f;
            int sp = 0;
            for (; sp + 8 <= S; sp += 8) {
                float x[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) x[j] = load(src + size_t(sp + j) * D);
#pragma unroll
                for (int j = 0; j < 8; ++j) acc = fmaf(x[j], w[hh * S + sp + j].x, acc);
            }
            for (; sp < S; ++sp) acc = fmaf(load(src + size_t(sp) * D), w[hh * S + sp].x, acc);
            out[(qh0 + hh) * D + c] = acc * linv[hh];
        }
    } else {
        for (int i = tid; i < G * D; i += kThreads) {
            const int hh = i / D, c = i - hh * D;
            const size_t qh = qh0 + hh;
            float M = -INFINITY;
            for (int sp = 0; sp < S; ++sp) M = fmaxf(M, load2(&stats[qh * SS + sp]).x);
            float acc = 0.0f, l = 0.0f;
            for (int sp = 0; sp < S; ++sp) {
                const float2 ms = load2(&stats[qh * SS + sp]);
                const float e = ms.x == -INFINITY ? 0.0f : expf(ms.x - M);
                l = fmaf(ms.y, e, l);
                acc = fmaf(load(&partial[(qh * SS + sp) * D + c]), e, acc);
            }
            out[qh * D + c] = acc / l;
        }
    }
    if (tid == 0) __hip_atomic_store(arrival, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Combine: each wave sums its rows over the group's tiles and over lanes, then
// the four waves' states merge into this split's (partial, stats). comb:
// [kWaves][D][kMaxG] floats in LDS, free for this use.
template <int D, int NCH, int G>
__device__ inline void combine_waves(float* comb, WaveStats& ws, AttnState<D>& st, float* __restrict__ partial,
                                     float2* __restrict__ stats, size_t qh0, int S, int split) {
    constexpr int Gs = Grp<G, D>::Gs;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, n16 = lane & 15, g = lane >> 4;
    // Row partial sums over the tiles of a group and all lanes of a head.
    st.l = lane_allreduce(st.l, Gs, AddOp{});
    st.off = lane_allreduce(st.off, Gs, AddOp{});
    // Accumulator rows 4g + i = (tile, head): sum over the tiles.
#pragma unroll
    for (int mb = 0; mb < D / 16; ++mb)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            st.o[mb][i] = lane_allreduce(st.o[mb][i], 16 * (Gs / 4), AddOp{});
        }
    if (g < Gs / 4) {
#pragma unroll
        for (int mb = 0; mb < D / 16; ++mb)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int hh = 4 * g + i;
                if (hh < G) comb[(wave * D + pv_channel<NCH>(mb, n16)) * kMaxG + hh] = st.o[mb][i];
            }
    }
    if (g == 0 && n16 < G) {
        ws.wm[wave][n16] = st.m;
        ws.wl[wave][n16] = st.l;
        ws.wo[wave][n16] = st.off;
    }
    __syncthreads();
    for (int i = tid; i < G * D; i += kThreads) {
        const int hh = i / D, c = i - hh * D;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) M = fmaxf(M, ws.wm[w][hh]);
        float acc = 0.0f, l = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const float e = ws.wm[w][hh] == -INFINITY ? 0.0f : exp2f(ws.wm[w][hh] - M);
            acc = fmaf(e, comb[(w * D + c) * kMaxG + hh] + ws.wo[w][hh], acc);
            l = fmaf(e, ws.wl[w][hh], l);
        }
        const size_t qh = qh0 + hh;
        // Agent-scope stores (written through to the device coherence point),
        // so that the workgroup merging the splits can read them from any XCD.
        __hip_atomic_store(&partial[(qh * S + split) * D + c], acc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (c == 0) {
            const float2 ml{M * 0.69314718055994531f, l};
            __hip_atomic_store(reinterpret_cast<uint64_t*>(&stats[qh * S + split]), __builtin_bit_cast(uint64_t, ml),
                               __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// --- ASTC split kernel -------------------------------------------------------

// FILLS: room for the fill stage's texels (the split kernel's; the paged
// kernel has no fill stage).
template <int D, int NCH, bool WIDE = false, bool FILLS = true, int MAXB = 0>
struct AstcShared {
    using C = Cfg<D, NCH, WIDE, MAXB>;
    LdsTables tabs;
    union {
        struct {
            BlockDesc<NCH> desc[C::kMaxBlocks];
            uint32_t cv[C::kMaxBlocks][kColourScratchWords];   // header-stage colour values, per lane
            uint8_t fill[kFillSlots];                          // blocks for the fill stage (kInfoFilled)
            FillArea<NCH> fv[FILLS ? 1 : 0];                   // their texels
        } h;
        float comb[kWaves * D * kMaxG];      // final per-wave accumulators
    } u;
    uint32_t so[C::kMaxTok];                 // per-token V scale | offset << 16 (fp16)
    uint32_t tokrow[C::kMaxTok];             // token_row_entry of each chunk token
    uint32_t key_count[kPathKeys];           // blocks per decode-path class (zero between chunks)
    uint32_t nfill;                          // entries of u.h.fill (zero between chunks)
    uint8_t order[C::kMaxBlocks];            // blocks sorted by decode-path class
    uint2 q[2 * C::kKSteps][64];             // Q operands (fp16 high, low)
    WaveStats ws;
};

// The chunk's blocks (one per lane).
__device__ inline uint4 load_block(const uint4* __restrict__ bseq, uint32_t cols, int row0, int nblk, int tid) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(seq_rsrc(bseq + size_t(row0) * cols, uint32_t(nblk) * 16),
                                                         16 * tid, 0, 0);   // lanes past nblk read zero
    return uint4{v[0], v[1], v[2], v[3]};
}

// Texels of one 16-token tile straight into the P.V operand: lane (n16, g)
// decodes tokens t0 + 4g .. + 3 of its texel columns x = n16 + 16 kc. Tokens at
// or past ntok come out zero. RGBA: channel j of column x feeds row block 4kc + j.
// This lane's four tokens of the 16-token tile at t0 (tokens t0 + 4g .. + 3):
// their token_row_entry values.
__device__ inline void tile_rows(const uint32_t* tokrow, int t0, int g, uint32_t (&rows)[4]) {
    const uint4 e4 = *reinterpret_cast<const uint4*>(&tokrow[t0 + 4 * g]);
    rows[0] = e4.x;
    rows[1] = e4.y;
    rows[2] = e4.z;
    rows[3] = e4.w;
}

// Texels of one texel column (block column bcol, x = xin in the block) for
// the four tokens of `rows`.
template <int NCH, bool FILL>
__device__ __attribute__((always_inline)) inline void column_texels(const BlockDesc<NCH>* desc, const LdsTables& L,
                                                                    Footprint f, const uint32_t (&rows)[4], int bcol,
                                                                    int xin, const FillArea<NCH>* fa,
                                                                    uint2 (&tv)[4]) {
    int bk[4], ik[4], xk[4], yk[4];
#pragma unroll
    for (int tk = 0; tk < 4; ++tk) {
        bk[tk] = int(rows[tk] >> 16) + bcol;
        ik[tk] = int(__builtin_amdgcn_ubfe(rows[tk], 8, 8)) + xin;
        xk[tk] = xin;
        yk[tk] = int(rows[tk] & 0xFF);
    }
    texels_fp16<NCH, 4, FILL>(desc, bk, ik, xk, yk, L, f, fa, tv);
}

// Row table of a chunk: token t -> (first block of its block row) << 16 |
// (y * bx) << 8 | y, for a chunk whose first token sits at row offset yoff
// of its first block row (y = (t + yoff) % by). Tokens at or past ntok take
// the entry of the chunk's last token, so that tile padding decodes real
// (finite) texels; their probabilities are zero.
__device__ inline uint32_t token_row_entry(int t, int ntok, uint32_t mag_by, Footprint f, uint32_t cols,
                                           int yoff = 0) {
    const int tl = min(t, ntok - 1) + yoff;
    const int r = int(fdiv(uint32_t(tl), mag_by)), y = tl - r * f.by;
    return (__umul24(uint32_t(r), cols) << 16) | (uint32_t(y * f.bx) << 8) | uint32_t(y);
}

// One column's texels for four tokens -> P.V B operands. RGBA: channel j of
// the column feeds row block j of the group (lane: tokens 4g .. 4g+3 of
// channel j); scalar: one row block.
template <int NCH>
__device__ inline void texel_operands(const uint2 (&tv)[4], half4* va) {
    if constexpr (NCH == 4) {
        const uint32_t sel[2] = {0x05040100u, 0x07060302u};
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
            const uint32_t sl = sel[jj & 1];
            const uint32_t lo = jj < 2 ? __builtin_amdgcn_perm(tv[1].x, tv[0].x, sl) : __builtin_amdgcn_perm(tv[1].y, tv[0].y, sl);
            const uint32_t hi = jj < 2 ? __builtin_amdgcn_perm(tv[3].x, tv[2].x, sl) : __builtin_amdgcn_perm(tv[3].y, tv[2].y, sl);
            va[jj] = __builtin_bit_cast(half4, uint2{lo, hi});
        }
    } else {
        va[0] = __builtin_bit_cast(half4, uint2{tv[0].x | (tv[1].x << 16), tv[2].x | (tv[3].x << 16)});
    }
}

}  // namespace akv_hip
