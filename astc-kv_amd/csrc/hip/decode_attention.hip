// Split-K decode attention over FP16 K and ASTC-compressed V for gfx950, the
// FP16-K/V control, the split merge, and the decode readback kernels.
//
// Reference semantics: metal/attention_gqa_v10.metal:568-674 (one group per
// (kv head, split) holding the G query states of that kv head; online softmax;
// factored token affine acc = sum p*s*u + sum p*o) and :229-253 (exact merge
// of split states).
//
// Split kernel schedule. One 256-lane workgroup per (sequence, kv head,
// split); a split is processed in chunks of whole block rows (at most 144
// blocks and 256 tokens for head dim 64, 128 for head dim 128). Per chunk:
//   1. the partition-pattern words of the chunk's blocks are requested first
//      (the blocks themselves were loaded one chunk ahead), then the chunk's
//      K rows (16-byte loads, in the MFMA operand layout) and the per-token V
//      scale/offset, then the next chunk's blocks;
//   2. header stage, one lane per block: BlockDesc records in LDS;
//   3. each wave takes every fourth 16-token tile of the chunk. A lane decodes
//      the texels of its MFMA operand directly: 4 consecutive tokens of one
//      texel column (RGBA: 4 channels each, so one decode feeds 4 MFMA row
//      blocks; the row blocks therefore hold channels 4x + j, x = texel
//      column, and the output is un-permuted at the end). Then S^T = K.Q^T and
//      O += V^T.P on the matrix cores (v_mfma_f32_16x16x16_f16; q and p are
//      split into fp16 high and low parts so the products keep ~22 bits), the
//      G query heads padded to the 16 MFMA columns, with an online softmax per
//      head, the per-token V scale folded into p and the offset term summed
//      separately.
// At the end the four wave states are combined into the split's state; the
// merge kernel combines the splits.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdint>
#include <map>
#include <mutex>
#include <tuple>

#include "astc_decode_device.h"
#include "astc_format.h"
#include "astc_kv_hip.h"

namespace akv_hip {

constexpr int kWaves = 4;
constexpr int kThreads = 64 * kWaves;
constexpr int kMaxG = 8;   // query heads per kv head
#ifndef AKV_ASTC_WAVES
#define AKV_ASTC_WAVES 3   // waves per SIMD the split kernel is register-limited to
#endif

typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

template <int D, int NCH>
struct Cfg {
    // Blocks per chunk (header stage, one per lane): at head dim 128 the
    // kernel runs two workgroups per CU, which leaves room for a full 256.
    static constexpr int kMaxBlocks = D == 64 ? 160 : 256;
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
    uint32_t chunk_tokens;   // tokens per full chunk (whole block rows for ASTC V)
    uint32_t mag_by, mag_bx; // ceil(2^24 / divisor)
    float qscale;            // log2(e) / sqrt(dim)
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
// (j = 0..3), matching the K row loads. Written by the first wave.
template <int D, int G>
__device__ inline void store_q(const float* __restrict__ qrow, float qscale, uint2* qs) {
    const int lane = threadIdx.x & 63, n16 = lane & 15, g = lane >> 4;
    const int h = n16 % Grp<G, D>::Gs;
#pragma unroll
    for (int ks = 0; ks < D / 16; ++ks) {
        half4 hi, lo;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float v = h < G ? qrow[size_t(h) * D + 32 * (ks / 2) + 8 * g + 4 * (ks % 2) + j] * qscale : 0.0f;
            hi[j] = _Float16(v);
            lo[j] = _Float16(v - float(hi[j]));
        }
        qs[(2 * ks) * 64 + lane] = __builtin_bit_cast(uint2, hi);
        qs[(2 * ks + 1) * 64 + lane] = __builtin_bit_cast(uint2, lo);
    }
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
// kreg[t * D/32 + L] are tile t's K rows; vtile(t, kc, va) produces tile t's
// V operands for row blocks MPB*kc .. MPB*kc + MPB-1 (lane (row, g): tokens
// 4g..4g+3 of the tile), called with kc = 0, 1, ... in order for each tile.
// so: per-token scale | offset << 16 for the chunk (AFFINE).
template <int D, int G, bool AFFINE, int MPB, typename VTile>
__device__ __attribute__((always_inline)) inline void attend_group(const uint4* kreg, const uint2* qs, int ng, int tb0,
                                                                   int ntok, const uint32_t* so, int so_cap,
                                                                   AttnState<D>& st, VTile&& vtile) {
    constexpr int Gs = Grp<G, D>::Gs, TPG = Grp<G, D>::TPG;
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
            const uint4 kk = kreg[t * (D / 32) + ks / 2];
            const half4 ka = __builtin_bit_cast(half4, (ks & 1) ? uint2{kk.z, kk.w} : uint2{kk.x, kk.y});
            sacc[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(ka, qh, sacc[t], 0, 0, 0);
            sacc[t] = __builtin_amdgcn_mfma_f32_16x16x16f16(ka, ql, sacc[t], 0, 0, 0);
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
// launch. No workgroup waits for another. The states are written and read
// with agent-scope atomic accesses (write-through stores, coherent loads), so
// publishing them needs no L2 write-back or invalidation: the stores of every
// wave complete (s_waitcnt 0) before the barrier, and the counter increment
// comes after it.
template <int D, int G>
__device__ inline void merge_if_last(uint32_t* arrival, const float* partial, const float2* stats,
                                     float* __restrict__ out, size_t qh0, int S, WaveStats& ws, float* lds,
                                     int lds_floats) {
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    if (threadIdx.x == 0)
        ws.last = __hip_atomic_fetch_add(arrival, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == uint32_t(S - 1);
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
        for (int i = tid; i < G * S; i += kThreads) w[i] = load2(&stats[qh0 * S + i]);
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
            const float* src = partial + (qh0 + hh) * size_t(S) * D + c;
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
            for (int sp = 0; sp < S; ++sp) M = fmaxf(M, load2(&stats[qh * S + sp]).x);
            float acc = 0.0f, l = 0.0f;
            for (int sp = 0; sp < S; ++sp) {
                const float2 ms = load2(&stats[qh * S + sp]);
                const float e = ms.x == -INFINITY ? 0.0f : expf(ms.x - M);
                l = fmaf(ms.y, e, l);
                acc = fmaf(load(&partial[(qh * S + sp) * D + c]), e, acc);
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

template <int D, int NCH>
struct AstcShared {
    using C = Cfg<D, NCH>;
    LdsTables tabs;
    union {
        struct {
            BlockDesc<NCH> desc[C::kMaxBlocks];
            uint8_t cv[C::kMaxBlocks][20];   // colour values of the header stage, per lane
        } h;
        float comb[kWaves * D * kMaxG];      // final per-wave accumulators
    } u;
    uint32_t so[C::kMaxTok];                 // per-token V scale | offset << 16 (fp16)
    uint32_t tokrow[C::kMaxTok];             // token_row_entry of each chunk token
    uint32_t key_count[kPathKeys];           // blocks per decode-path class (zero between chunks)
    uint32_t key_base[kPathKeys];            // first sorted position of each class
    uint8_t order[C::kMaxBlocks];            // blocks sorted by decode-path class
    uint2 q[2 * C::kKSteps][64];             // Q operands (fp16 high, low)
    WaveStats ws;
};

// The chunk's blocks (one per lane).
__device__ inline uint4 load_block(const uint4* __restrict__ bseq, uint32_t cols, int row0, int nblk, int tid) {
    return tid < nblk ? bseq[size_t(row0) * cols + tid] : uint4{0, 0, 0, 0};
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
template <int NCH>
__device__ __attribute__((always_inline)) inline void column_texels(const BlockDesc<NCH>* desc, const LdsTables& L,
                                                                    Footprint f, const uint32_t (&rows)[4], int bcol,
                                                                    int xin, uint2 (&tv)[4]) {
    int bk[4], ik[4], xk[4], yk[4];
#pragma unroll
    for (int tk = 0; tk < 4; ++tk) {
        bk[tk] = int(rows[tk] >> 16) + bcol;
        ik[tk] = int(__builtin_amdgcn_ubfe(rows[tk], 8, 8)) + xin;
        xk[tk] = xin;
        yk[tk] = int(rows[tk] & 0xFF);
    }
    texels_fp16<NCH, 4>(desc, bk, ik, xk, yk, L, f, tv);
}

// Row table of a chunk: token t -> (first block of its block row) << 16 |
// (y * bx) << 8 | y, y = t % by. Tokens at or past ntok take the entry of the
// chunk's last token, so that tile padding decodes real (finite) texels; their
// probabilities are zero.
__device__ inline uint32_t token_row_entry(int t, int ntok, uint32_t mag_by, Footprint f, uint32_t cols) {
    const int tl = min(t, ntok - 1);
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

template <int D, int NCH, int G, bool DUMP>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(D == 64 ? AKV_ASTC_WAVES : 2))) void astc_attn_kernel(
    KernelArgs a, const float* __restrict__ q, const uint16_t* __restrict__ k, const uint4* __restrict__ vblk,
    const uint16_t* __restrict__ vscale, const uint16_t* __restrict__ voffset, const AkvTables* __restrict__ tab,
    float* partial, float2* stats, uint16_t* __restrict__ dump, float* __restrict__ out, uint32_t* arrivals) {
    using C = Cfg<D, NCH>;
    constexpr int TPG = Grp<G, D>::TPG;
    // K tiles of a wave's first group requested before the header stage (their
    // registers are live through it); the rest right after it.
    constexpr int kKEarly = TPG < 2 ? TPG : 2;
    __shared__ AstcShared<D, NCH> sh;
    const AkvAttnParams& p = a.p;
    const Footprint f = a.fp;
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int n16 = lane & 15, g = lane >> 4;
    const int split = blockIdx.x, kh = blockIdx.y, b = blockIdx.z;
    const int split_begin = split * int(p.tile_tokens);
    const int split_end = min(split_begin + int(p.tile_tokens), int(p.tokens));
    const int CT = int(a.chunk_tokens), by = f.by;
    const uint32_t cols = p.atlas_cols;

    const size_t seq_kv = size_t(b) * p.kv_heads + kh;
    const uint16_t* kseq = DUMP ? nullptr : k + seq_kv * p.tokens * D;
    const uint4* bseq = vblk + seq_kv * p.atlas_rows * cols;
    const uint16_t* sseq = DUMP ? nullptr : vscale + seq_kv * p.tokens;
    const uint16_t* oseq = DUMP ? nullptr : voffset + seq_kv * p.tokens;

    auto chunk_blocks = [&](int c0) { return int((min(CT, split_end - c0) + by - 1) / by * cols); };
    uint4 raw = load_block(bseq, cols, split_begin / by, chunk_blocks(split_begin), tid);
    uint4 pw = tid < chunk_blocks(split_begin) ? partition_words(raw, tab) : uint4{0, 0, 0, 0};
    stage_tables(tab, sh.tabs, tid, kThreads);
    if (tid < kPathKeys) sh.key_count[tid] = 0;

    if constexpr (!DUMP)
        if (wave == 0) store_q<D, G>(q + (size_t(b) * p.query_heads + size_t(kh) * G) * D, a.qscale, &sh.q[0][0]);

    // This lane's texel columns: x = n16 + 16 * kc -> block column and x in block.
    int bcol[C::kColGroups], xin[C::kColGroups];
#pragma unroll
    for (int kc = 0; kc < C::kColGroups; ++kc) {
        const int x = n16 + 16 * kc;
        bcol[kc] = int(fdiv(uint32_t(x), a.mag_bx));
        xin[kc] = x - bcol[kc] * f.bx;
    }

    AttnState<D> st;
    st.m = -INFINITY;
    st.l = st.off = 0.0f;
#pragma unroll
    for (int mb = 0; mb < C::kMBlocks; ++mb) st.o[mb] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

    __syncthreads();   // decode tables and Q operands
    for (int c0 = split_begin; c0 < split_end; c0 += CT) {
        const int ntok = min(CT, split_end - c0);
        const int ntiles = (ntok + 15) >> 4;
        const int nblk = chunk_blocks(c0);
        // 1. Loads (the chunk's blocks and their partition-pattern words were
        // requested during the previous chunk): the first K tiles of this
        // wave's first group, per-token scale/offset, the next chunk's blocks.
        uint4 kreg[TPG * C::kRowLoads];
        const __amdgpu_buffer_rsrc_t krs = seq_rsrc(DUMP ? nullptr : kseq + size_t(c0) * D, DUMP ? 0u : uint32_t(ntok) * D * 2);
        if constexpr (!DUMP) {
#pragma unroll
            for (int t = 0; t < kKEarly; ++t)
                load_k_tile<D>(kreg + t * C::kRowLoads, krs, 16 * (TPG * wave + t), lane);
        }
        // Per-token V scale | offset << 16 for up to two tokens per lane.
        static_assert(C::kMaxTok <= 2 * kThreads, "two scale/offset tokens per lane");
        uint32_t so[2] = {0, 0};
        if constexpr (!DUMP) {
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int t = tid + i * kThreads;
                if (t < ntok) so[i] = uint32_t(sseq[c0 + t]) | (uint32_t(oseq[c0 + t]) << 16);
            }
        }
        const uint4 raw_now = raw;
        if (c0 + CT < split_end) raw = load_block(bseq, cols, (c0 + CT) / by, chunk_blocks(c0 + CT), tid);
        // 2. Block headers, with the chunk's blocks sorted by decode-path class
        // so that the lanes of a wave take the same branches. Each block's raw
        // bits and pattern words wait in its own descriptor slot; the lane that
        // decodes a block reads them from there and overwrites that slot.
        int key = 0, rank = 0;
        if (tid < nblk) {
            key = block_path_key(raw_now, sh.tabs);
            stash_block(sh.u.h.desc[tid], raw_now, pw);
            rank = int(atomicAdd(&sh.key_count[key], 1u));
        }
        // Tokens past the chunk up to the tile edge get scale = offset = 0.
        if constexpr (!DUMP) {
#pragma unroll
            for (int i = 0; i < 2; ++i)
                if (tid + i * kThreads < 16 * ntiles) sh.so[tid + i * kThreads] = so[i];
        }
#pragma unroll
        for (int i = 0; i < 2; ++i)
            if (tid + i * kThreads < C::kMaxTok)
                sh.tokrow[tid + i * kThreads] = token_row_entry(tid + i * kThreads, ntok, a.mag_by, f, cols);
        __syncthreads();
        if (wave == 0) {   // exclusive scan of the class counts (kPathKeys == 64 lanes)
            const uint32_t c = sh.key_count[lane];
            uint32_t incl = c;
#pragma unroll
            for (int d = 1; d < 64; d <<= 1) {
                const uint32_t t = __shfl_up(incl, d, 64);
                if (lane >= d) incl += t;
            }
            sh.key_base[lane] = incl - c;
            sh.key_count[lane] = 0;
        }
        __syncthreads();
        if (tid < nblk) sh.order[sh.key_base[key] + rank] = uint8_t(tid);
        __syncthreads();
        if (tid < nblk) decode_header<NCH>(sh.tabs, sh.u.h.desc[sh.order[tid]], sh.u.h.cv[tid]);
        // The next chunk's pattern words (its blocks have arrived by now).
        if (c0 + CT < split_end) pw = tid < chunk_blocks(c0 + CT) ? partition_words(raw, tab) : uint4{0, 0, 0, 0};
        __syncthreads();
        // 3. This wave's groups of TPG consecutive tiles (every fourth group):
        // S for the whole group, then for each tile its texels straight into
        // MFMA operands and P.V. The next group's K rows are requested as soon
        // as S no longer needs the registers.
        if constexpr (DUMP) {
            uint16_t* dst = dump + (seq_kv * p.tokens + c0) * D;
            for (int t0 = 16 * wave; t0 < ntok; t0 += 16 * kWaves) {
                uint32_t rows[4];
                tile_rows(sh.tokrow, t0, g, rows);
#pragma unroll
                for (int kc = 0; kc < C::kColGroups; ++kc) {
                    uint2 tv[4];
                    column_texels<NCH>(sh.u.h.desc, sh.tabs, f, rows, bcol[kc], xin[kc], tv);
                    const int x = n16 + 16 * kc;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int t = t0 + 4 * g + i;
                        if (t >= ntok) break;
                        if constexpr (NCH == 4) *reinterpret_cast<uint2*>(dst + size_t(t) * D + 4 * x) = tv[i];
                        else dst[size_t(t) * D + x] = uint16_t(tv[i].x);
                    }
                }
            }
        } else {
#pragma unroll
            for (int t = kKEarly; t < TPG; ++t)
                load_k_tile<D>(kreg + t * C::kRowLoads, krs, 16 * (TPG * wave + t), lane);
#pragma unroll 1
            for (int tb0 = 16 * TPG * wave; tb0 < ntok; tb0 += 16 * TPG * kWaves) {
                const int ng = min(TPG, (ntok - tb0 + 15) >> 4);
                uint32_t rows[4];   // token_row_entry of this lane's four tokens of the tile
                attend_group<D, G, true, C::kRowBlocksPerGroup>(
                    kreg, &sh.q[0][0], ng, tb0, ntok, sh.so, C::kMaxTok, st, [&](int t, int kc, half4* va) {
                        if (kc == 0) {
                            if (t == 0) {   // S is done with this group's K rows
                                const int nb0 = tb0 + 16 * TPG * kWaves;
#pragma unroll
                                for (int tt = 0; tt < TPG; ++tt)
                                    load_k_tile<D>(kreg + tt * C::kRowLoads, krs, nb0 + 16 * tt, lane);
                            }
                            tile_rows(sh.tokrow, tb0 + 16 * t, g, rows);
                        }
                        uint2 tv[4];
                        column_texels<NCH>(sh.u.h.desc, sh.tabs, f, rows, bcol[kc], xin[kc], tv);
                        texel_operands<NCH>(tv, va);
                    });
            }
        }
        __syncthreads();   // descriptors and so are rewritten by the next chunk
    }
    if constexpr (DUMP) return;
    const size_t qh0 = size_t(b) * p.query_heads + size_t(kh) * G;
    combine_waves<D, NCH, G>(sh.u.comb, sh.ws, st, partial, stats, qh0, int(p.splits), split);
    if (arrivals)
        merge_if_last<D, G>(arrivals + seq_kv, partial, stats, out, qh0, int(p.splits), sh.ws, sh.u.comb,
                            kWaves * D * kMaxG);
}

// --- FP16-K/V control ----------------------------------------------------------

template <int D>
struct Fp16Shared {
    float comb[kWaves * D * kMaxG];
    uint2 q[2 * D / 16][64];   // Q operands (fp16 high, low)
    WaveStats ws;
};

// V rows of one 16-token tile straight into the P.V operand layout
// (RGBA-style channel order: lane n16 reads channels 4x .. 4x+3 of group
// x = n16 + 16k for tokens t0 + 4 * (lane / 16) + i, 8 bytes per token, so 16
// lanes read 128 contiguous bytes). Tokens at or past ntok read as zero.
template <int D>
__device__ inline void load_v_tile(uint2 (&r)[4][D / 64], __amdgpu_buffer_rsrc_t rs, int t0, int lane) {
    const uint32_t n16 = uint32_t(lane & 15), g = uint32_t(lane >> 4);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int kc = 0; kc < D / 64; ++kc) {
            const uint32_t t = uint32_t(t0) + 4 * g + uint32_t(i);
            const auto v = __builtin_amdgcn_raw_buffer_load_b64(rs, 2 * (t * D + 4 * (n16 + 16 * kc)), 0, 0);
            r[i][kc] = uint2{v[0], v[1]};
        }
}

// FP16-K/V control: each wave streams its groups of TPG tiles of the split
// (every fourth group); the next group's K rows are requested once S is done
// with the registers, and each tile's V rows one tile ahead.
template <int D, int G>
__global__ __launch_bounds__(kThreads) void fp16_attn_kernel(KernelArgs a, const float* __restrict__ q,
                                                             const uint16_t* __restrict__ k,
                                                             const uint16_t* __restrict__ v,
                                                             float* partial, float2* stats,
                                                             float* __restrict__ out, uint32_t* arrivals) {
    using C = Cfg<D, 4>;
    constexpr int TPG = Grp<G, D>::TPG;
    __shared__ Fp16Shared<D> sh;
    const AkvAttnParams& p = a.p;
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int n16 = lane & 15, g = lane >> 4;
    const int split = blockIdx.x, kh = blockIdx.y, b = blockIdx.z;
    const int split_begin = split * int(p.tile_tokens);
    const int ntok = min(int(p.tile_tokens), int(p.tokens) - split_begin);
    const size_t seq_kv = size_t(b) * p.kv_heads + kh;
    const __amdgpu_buffer_rsrc_t krs = seq_rsrc(k + (seq_kv * p.tokens + split_begin) * D, uint32_t(ntok) * D * 2);
    const __amdgpu_buffer_rsrc_t vrs = seq_rsrc(v + (seq_kv * p.tokens + split_begin) * D, uint32_t(ntok) * D * 2);

    if (wave == 0) store_q<D, G>(q + (size_t(b) * p.query_heads + size_t(kh) * G) * D, a.qscale, &sh.q[0][0]);
    AttnState<D> st;
    st.m = -INFINITY;
    st.l = st.off = 0.0f;
#pragma unroll
    for (int mb = 0; mb < C::kMBlocks; ++mb) st.o[mb] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

    constexpr int kStride = 16 * TPG * kWaves;
    uint4 kreg[TPG * C::kRowLoads];
    uint2 vreg[4][D / 64], cur[4][D / 64];
    int tb0 = 16 * TPG * wave;
#pragma unroll
    for (int t = 0; t < TPG; ++t) load_k_tile<D>(kreg + t * C::kRowLoads, krs, tb0 + 16 * t, lane);
    load_v_tile<D>(vreg, vrs, tb0, lane);
    __syncthreads();   // Q operands
#pragma unroll 1
    for (; tb0 < ntok; tb0 += kStride) {
        const int ng = min(TPG, (ntok - tb0 + 15) >> 4);
        attend_group<D, G, false, 4>(kreg, &sh.q[0][0], ng, tb0, ntok, nullptr, 4, st, [&](int t, int kc, half4* va) {
            if (kc == 0) {
                if (t == 0) {
#pragma unroll
                    for (int tt = 0; tt < TPG; ++tt)
                        load_k_tile<D>(kreg + tt * C::kRowLoads, krs, tb0 + kStride + 16 * tt, lane);
                }
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int c = 0; c < D / 64; ++c) cur[i][c] = vreg[i][c];
                // The next tile's V rows (the next group's first tile after the last).
                const int nt = t + 1 < ng ? tb0 + 16 * (t + 1) : tb0 + kStride;
                load_v_tile<D>(vreg, vrs, nt, lane);
            }
            const uint2 tv[4] = {cur[0][kc], cur[1][kc], cur[2][kc], cur[3][kc]};
            texel_operands<4>(tv, va);
        });
    }
    __syncthreads();
    const size_t qh0 = size_t(b) * p.query_heads + size_t(kh) * G;
    combine_waves<D, 4, G>(sh.comb, sh.ws, st, partial, stats, qh0, int(p.splits), split);
    if (arrivals)
        merge_if_last<D, G>(arrivals + seq_kv, partial, stats, out, qh0, int(p.splits), sh.ws, sh.comb,
                            kWaves * D * kMaxG);
}

// --- merge ---------------------------------------------------------------------

// One workgroup per (sequence, query head); wave w takes splits w, w + 4, ...;
// lane = channel (and channel + 64 for dim 128).
__global__ __launch_bounds__(kThreads) void merge_kernel(uint32_t splits, uint32_t dim,
                                                         const float* __restrict__ partial,
                                                         const float2* __restrict__ stats, float* __restrict__ out) {
    __shared__ float red_m[kWaves], red_l[kWaves];
    __shared__ float red_acc[kWaves][128];
    const size_t qh = blockIdx.x;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int S = int(splits), D = int(dim);
    const float2* st = stats + qh * S;
    float M = -INFINITY;
    for (int s = tid; s < S; s += kThreads) M = fmaxf(M, st[s].x);
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) M = fmaxf(M, __shfl_xor(M, o, 64));
    if (lane == 0) red_m[wave] = M;
    __syncthreads();
    M = fmaxf(fmaxf(red_m[0], red_m[1]), fmaxf(red_m[2], red_m[3]));
    const float* base = partial + qh * S * D;
    float acc0 = 0.0f, acc1 = 0.0f, l = 0.0f;
#pragma unroll 4
    for (int s = wave; s < S; s += kWaves) {
        const float2 ms = st[s];
        const float e = ms.x == -INFINITY ? 0.0f : expf(ms.x - M);
        l = fmaf(ms.y, e, l);
        acc0 = fmaf(base[size_t(s) * D + lane], e, acc0);
        if (D == 128) acc1 = fmaf(base[size_t(s) * D + 64 + lane], e, acc1);
    }
    if (lane == 0) red_l[wave] = l;
    red_acc[wave][lane] = acc0;
    if (D == 128) red_acc[wave][64 + lane] = acc1;
    __syncthreads();
    if (tid < D) {
        const float L = red_l[0] + red_l[1] + red_l[2] + red_l[3];
        const float A = red_acc[0][tid] + red_acc[1][tid] + red_acc[2][tid] + red_acc[3][tid];
        out[qh * D + tid] = A / L;
    }
}

// --- standalone block decode -------------------------------------------------------

struct BlocksShared {
    LdsTables tabs;
    BlockDesc<4> desc[kThreads];
    uint8_t cv[kThreads][20];
};

// 256 blocks per workgroup -> FP16 RGBA texels [n][by][bx][4].
__global__ __launch_bounds__(kThreads) void decode_blocks_kernel(const uint4* __restrict__ blocks, size_t n,
                                                                 Footprint f, const AkvTables* __restrict__ tab,
                                                                 uint2* __restrict__ out) {
    __shared__ BlocksShared sh;
    const int tid = threadIdx.x;
    const size_t first = size_t(blockIdx.x) * kThreads;
    const int nblk = int(min(size_t(kThreads), n - first));
    const uint4 raw = tid < nblk ? blocks[first + tid] : uint4{0, 0, 0, 0};
    const uint4 pw = tid < nblk ? partition_words(raw, tab) : uint4{0, 0, 0, 0};
    stage_tables(tab, sh.tabs, tid, kThreads);
    __syncthreads();
    if (tid < nblk) {
        stash_block(sh.desc[tid], raw, pw);
        decode_header<4>(sh.tabs, sh.desc[tid], sh.cv[tid]);
    }
    __syncthreads();
    for (int it = tid; it < nblk * f.ntex; it += kThreads) {
        const int blk = it / f.ntex, i = it - blk * f.ntex;
        const int y = i / f.bx, x = i - y * f.bx;
        out[(first + blk) * f.ntex + i] = texel_fp16<4>(sh.desc[blk], sh.tabs, f, x, y);
    }
}

// ---------------------------------------------------------------------------
// Host side.

namespace {

std::mutex g_mu;
std::map<std::tuple<int, int, int>, AkvTables*> g_tables;  // (device, bx, by)

int device_tables(int bx, int by, const AkvTables** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return int(e);
    std::lock_guard<std::mutex> lock(g_mu);
    auto key = std::make_tuple(dev, bx, by);
    auto it = g_tables.find(key);
    if (it != g_tables.end()) {
        *out = it->second;
        return 0;
    }
    const AkvTables* host = akv::tables_for(bx, by);
    if (!host) return AKV_HIP_ERR_FOOTPRINT;
    AkvTables* d = nullptr;
    e = hipMalloc(reinterpret_cast<void**>(&d), sizeof(AkvTables));
    if (e != hipSuccess) return int(e);
    e = hipMemcpy(d, host, sizeof(AkvTables), hipMemcpyHostToDevice);
    if (e != hipSuccess) {
        (void)hipFree(d);
        return int(e);
    }
    g_tables[key] = d;
    *out = d;
    return 0;
}

uint32_t magic(uint32_t d) { return ((1u << 24) + d - 1) / d; }

int check_common(const AkvAttnParams* p, uint32_t* G) {
    if (!p) return AKV_HIP_ERR_NULL;
    if (p->batch == 0 || p->tokens == 0 || p->kv_heads == 0 || p->query_heads % p->kv_heads) return AKV_HIP_ERR_SHAPE;
    if (p->dim != 64 && p->dim != 128) return AKV_HIP_ERR_SHAPE;
    const uint32_t g = p->query_heads / p->kv_heads;
    if (g != 1 && g != 2 && g != 3 && g != 4 && g != 8) return AKV_HIP_ERR_SHAPE;
    if (p->batch > 65535 || p->kv_heads > 65535) return AKV_HIP_ERR_SHAPE;
    if (p->tile_tokens == 0) return AKV_HIP_ERR_TILE;
    if (p->splits != (p->tokens + p->tile_tokens - 1) / p->tile_tokens || p->splits > 2147483647u)
        return AKV_HIP_ERR_TILE;
    *G = g;
    return 0;
}

Footprint footprint(uint32_t bx, uint32_t by) {
    Footprint f{};
    f.bx = int(bx);
    f.by = int(by);
    f.ntex = int(bx * by);
    f.ds = int((1024 + bx / 2) / (bx - 1));
    f.dt = int((1024 + by / 2) / (by - 1));
    return f;
}

int check_astc(const AkvAttnParams* p) {
    if (p->layout != AKV_LAYOUT_SCALAR && p->layout != AKV_LAYOUT_RGBA) return AKV_HIP_ERR_SHAPE;
    const uint32_t bx = p->block_x, by = p->block_y;
    if (bx < 4 || by < 4 || bx > 12 || by > 12 || bx * by > uint32_t(akv::kMaxTexels)) return AKV_HIP_ERR_FOOTPRINT;
    const uint32_t texcols = p->layout == AKV_LAYOUT_SCALAR ? p->dim : p->dim / 4;
    if (p->atlas_cols != (texcols + bx - 1) / bx) return AKV_HIP_ERR_SHAPE;
    if (p->tile_tokens % by) return AKV_HIP_ERR_TILE;
    if (uint64_t(p->atlas_rows) * by < p->tokens) return AKV_HIP_ERR_SHAPE;
    return 0;
}

// Chunk shape. ASTC V: the most whole block rows whose blocks fit the header
// stage and whose tokens fit a chunk; FP16 control: a whole chunk. Never more
// than one split.
template <int D, int NCH>
int plan_chunks(const AkvAttnParams* p, bool astc, KernelArgs* a) {
    using C = Cfg<D, NCH>;
    uint32_t tokens = C::kMaxTok;
    if (astc) {
        const uint32_t by = p->block_y;
        uint32_t r = uint32_t(C::kMaxBlocks) / p->atlas_cols;
        if (r * by > uint32_t(C::kMaxTok)) r = uint32_t(C::kMaxTok) / by;
        if (r == 0) return AKV_HIP_ERR_SHAPE;
        tokens = r * by;
    }
    a->chunk_tokens = tokens < p->tile_tokens ? tokens : p->tile_tokens;
    return 0;
}

int make_args(const AkvAttnParams* p, bool astc, KernelArgs* a) {
    *a = KernelArgs{};
    a->p = *p;
    if (astc) {
        a->fp = footprint(p->block_x, p->block_y);
        a->mag_by = magic(p->block_y);
        a->mag_bx = magic(p->block_x);
    }
    a->qscale = float(1.4426950408889634 / std::sqrt(double(p->dim)));
    const bool scalar = astc && p->layout == AKV_LAYOUT_SCALAR;
    if (p->dim == 64) return scalar ? plan_chunks<64, 1>(p, astc, a) : plan_chunks<64, 4>(p, astc, a);
    return scalar ? plan_chunks<128, 1>(p, astc, a) : plan_chunks<128, 4>(p, astc, a);
}

struct Ptrs {
    const float* q;
    const uint16_t* k;
    const uint4* vblk;
    const uint16_t* vh;
    const uint16_t* vs;
    const uint16_t* vo;
    const AkvTables* tab;
    float* partial;
    float* stats;
    uint16_t* dump;
    float* out = nullptr;             // with arrivals: the merged output
    uint32_t* arrivals = nullptr;     // non-null: merge in the split kernel
};

template <int D, int NCH, bool DUMP>
hipError_t launch_astc_g(const KernelArgs& a, uint32_t G, const Ptrs& x, hipStream_t st) {
    dim3 grid(a.p.splits, a.p.kv_heads, a.p.batch);
    auto* s2 = reinterpret_cast<float2*>(x.stats);
    if constexpr (DUMP) {
        astc_attn_kernel<D, NCH, 1, true><<<grid, kThreads, 0, st>>>(a, x.q, x.k, x.vblk, x.vs, x.vo, x.tab, x.partial,
                                                                      s2, x.dump, nullptr, nullptr);
        return hipGetLastError();
    }
    switch (G) {
#define AKV_CASE(GG)                                                                                       \
    case GG:                                                                                               \
        astc_attn_kernel<D, NCH, GG, DUMP><<<grid, kThreads, 0, st>>>(a, x.q, x.k, x.vblk, x.vs, x.vo, x.tab, \
                                                                       x.partial, s2, x.dump, x.out,      \
                                                                       x.arrivals);                       \
        break;
        AKV_CASE(1)
        AKV_CASE(2)
        AKV_CASE(3)
        AKV_CASE(4)
        AKV_CASE(8)
#undef AKV_CASE
        default:
            return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

template <bool DUMP>
hipError_t launch_astc(const KernelArgs& a, uint32_t G, const Ptrs& x, hipStream_t st) {
    const bool scalar = a.p.layout == AKV_LAYOUT_SCALAR;
    if (a.p.dim == 64) return scalar ? launch_astc_g<64, 1, DUMP>(a, G, x, st) : launch_astc_g<64, 4, DUMP>(a, G, x, st);
    return scalar ? launch_astc_g<128, 1, DUMP>(a, G, x, st) : launch_astc_g<128, 4, DUMP>(a, G, x, st);
}

template <int D>
hipError_t launch_fp16_g(const KernelArgs& a, uint32_t G, const Ptrs& x, hipStream_t st) {
    dim3 grid(a.p.splits, a.p.kv_heads, a.p.batch);
    auto* s2 = reinterpret_cast<float2*>(x.stats);
    switch (G) {
#define AKV_CASE(GG)                                                                                   \
    case GG:                                                                                           \
        fp16_attn_kernel<D, GG><<<grid, kThreads, 0, st>>>(a, x.q, x.k, x.vh, x.partial, s2, x.out,   \
                                                           x.arrivals);                                 \
        break;
        AKV_CASE(1)
        AKV_CASE(2)
        AKV_CASE(3)
        AKV_CASE(4)
        AKV_CASE(8)
#undef AKV_CASE
        default:
            return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

int as_int(hipError_t e) { return e == hipSuccess ? 0 : int(e); }

hipError_t launch_merge(const AkvAttnParams* p, const float* partial, const float* stats, float* out, hipStream_t st) {
    const uint64_t groups = uint64_t(p->batch) * p->query_heads;
    if (groups > 0x7FFFFFFFu) return hipErrorInvalidValue;
    merge_kernel<<<dim3(uint32_t(groups)), dim3(kThreads), 0, st>>>(p->splits, p->dim, partial,
                                                                    reinterpret_cast<const float2*>(stats), out);
    return hipGetLastError();
}

int run_astc(const AkvAttnParams* p, const float* q, const uint16_t* k, const void* v_blocks, const uint16_t* v_scale,
             const uint16_t* v_offset, float* partial, float* stats, float* out, bool with_merge, uint32_t* arrivals,
             void* stream) {
    uint32_t G = 0;
    if (int rc = check_common(p, &G)) return rc;
    if (int rc = check_astc(p)) return rc;
    if (!q || !k || !v_blocks || !v_scale || !v_offset || !partial || !stats || (with_merge && !out))
        return AKV_HIP_ERR_NULL;
    const AkvTables* tab = nullptr;
    if (int rc = device_tables(int(p->block_x), int(p->block_y), &tab)) return rc;
    KernelArgs a;
    if (int rc = make_args(p, true, &a)) return rc;
    hipStream_t st = static_cast<hipStream_t>(stream);
    Ptrs x{q, k, static_cast<const uint4*>(v_blocks), nullptr, v_scale, v_offset, tab, partial, stats, nullptr};
    if (with_merge && arrivals) {
        x.out = out;
        x.arrivals = arrivals;
    }
    hipError_t e = launch_astc<false>(a, G, x, st);
    if (e == hipSuccess && with_merge && !arrivals) e = launch_merge(p, partial, stats, out, st);
    return as_int(e);
}

}  // namespace
}  // namespace akv_hip

using namespace akv_hip;

extern "C" {

int akv_hip_attention_split(const AkvAttnParams* p, const float* q, const uint16_t* k, const void* v_blocks,
                            const uint16_t* v_scale, const uint16_t* v_offset, float* partial, float* stats,
                            void* stream) {
    return run_astc(p, q, k, v_blocks, v_scale, v_offset, partial, stats, nullptr, false, nullptr, stream);
}

int akv_hip_attention_merge(const AkvAttnParams* p, const float* partial, const float* stats, float* out,
                            void* stream) {
    uint32_t G = 0;
    if (int rc = check_common(p, &G)) return rc;
    if (!partial || !stats || !out) return AKV_HIP_ERR_NULL;
    return as_int(launch_merge(p, partial, stats, out, static_cast<hipStream_t>(stream)));
}

int akv_hip_decode_attention(const AkvAttnParams* p, const float* q, const uint16_t* k, const void* v_blocks,
                             const uint16_t* v_scale, const uint16_t* v_offset, float* partial, float* stats,
                             float* out, void* stream) {
    return run_astc(p, q, k, v_blocks, v_scale, v_offset, partial, stats, out, true, nullptr, stream);
}

int akv_hip_decode_attention_fused(const AkvAttnParams* p, const float* q, const uint16_t* k, const void* v_blocks,
                                   const uint16_t* v_scale, const uint16_t* v_offset, float* partial, float* stats,
                                   float* out, uint32_t* arrivals, void* stream) {
    if (!arrivals) return AKV_HIP_ERR_NULL;
    return run_astc(p, q, k, v_blocks, v_scale, v_offset, partial, stats, out, true, arrivals, stream);
}

int akv_hip_fp16_attention_fused(const AkvAttnParams* p, const float* q, const uint16_t* k, const uint16_t* v,
                                 float* partial, float* stats, float* out, uint32_t* arrivals, void* stream) {
    uint32_t G = 0;
    if (int rc = check_common(p, &G)) return rc;
    if (!q || !k || !v || !partial || !stats || !out) return AKV_HIP_ERR_NULL;
    KernelArgs a;
    if (int rc = make_args(p, false, &a)) return rc;
    hipStream_t st = static_cast<hipStream_t>(stream);
    Ptrs x{q, k, nullptr, v, nullptr, nullptr, nullptr, partial, stats, nullptr};
    x.out = out;
    x.arrivals = arrivals;
    hipError_t e = p->dim == 64 ? launch_fp16_g<64>(a, G, x, st) : launch_fp16_g<128>(a, G, x, st);
    if (e == hipSuccess && !arrivals) e = launch_merge(p, partial, stats, out, st);
    return as_int(e);
}

int akv_hip_fp16_attention(const AkvAttnParams* p, const float* q, const uint16_t* k, const uint16_t* v,
                           float* partial, float* stats, float* out, void* stream) {
    return akv_hip_fp16_attention_fused(p, q, k, v, partial, stats, out, nullptr, stream);
}

int akv_hip_decode_values(const AkvAttnParams* p, const void* v_blocks, uint16_t* u, void* stream) {
    uint32_t G = 0;
    if (int rc = check_common(p, &G)) return rc;
    if (int rc = check_astc(p)) return rc;
    if (!v_blocks || !u) return AKV_HIP_ERR_NULL;
    const AkvTables* tab = nullptr;
    if (int rc = device_tables(int(p->block_x), int(p->block_y), &tab)) return rc;
    KernelArgs a;
    if (int rc = make_args(p, true, &a)) return rc;
    const Ptrs x{nullptr, nullptr, static_cast<const uint4*>(v_blocks), nullptr, nullptr, nullptr, tab, nullptr,
                 nullptr, u};
    return as_int(launch_astc<true>(a, 1, x, static_cast<hipStream_t>(stream)));
}

int akv_hip_decode_blocks(const void* blocks, size_t n, unsigned bx, unsigned by, uint16_t* texels, void* stream) {
    if ((!blocks || !texels) && n) return AKV_HIP_ERR_NULL;
    if (bx < 4 || by < 4 || bx > 12 || by > 12 || bx * by > unsigned(akv::kMaxTexels)) return AKV_HIP_ERR_FOOTPRINT;
    if (n == 0) return 0;
    const AkvTables* tab = nullptr;
    if (int rc = device_tables(int(bx), int(by), &tab)) return rc;
    const Footprint f = footprint(bx, by);
    const size_t groups = (n + kThreads - 1) / kThreads;
    if (groups > 0x7FFFFFFF) return AKV_HIP_ERR_SHAPE;
    decode_blocks_kernel<<<dim3(unsigned(groups)), dim3(kThreads), 0, static_cast<hipStream_t>(stream)>>>(
        static_cast<const uint4*>(blocks), n, f, tab, reinterpret_cast<uint2*>(texels));
    return as_int(hipGetLastError());
}

int akv_hip_task_tokens(const AkvAttnParams* p, int astc) {
    uint32_t G = 0;
    if (int rc = check_common(p, &G)) return rc;
    if (astc)
        if (int rc = check_astc(p)) return rc;
    KernelArgs a;
    if (int rc = make_args(p, astc != 0, &a)) return rc;
    return int(a.chunk_tokens);
}

const char* akv_hip_error_string(int code) {
    switch (code) {
        case 0: return "success";
        case AKV_HIP_ERR_NULL: return "required pointer is NULL";
        case AKV_HIP_ERR_SHAPE: return "unsupported or inconsistent shape";
        case AKV_HIP_ERR_FOOTPRINT: return "unsupported ASTC footprint";
        case AKV_HIP_ERR_TILE: return "tile_tokens/splits inconsistent (tile must be a positive multiple of "
                                      "block_y and splits = ceil(tokens/tile))";
        default: return code > 0 ? hipGetErrorString(hipError_t(code)) : "unknown error";
    }
}

}  // extern "C"
