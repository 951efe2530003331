// Split-K decode attention over FP16 K and ASTC-compressed V for gfx950 on a
// contiguous atlas ([sequence][kv head][block row][block column]), the FP16-K/V
// control, the split merge, the decode readback kernels, and their C-ABI.
//
// Reference semantics: metal/attention_gqa_v10.metal:568-674 (one group per
// (kv head, split) holding the G query states of that kv head; online softmax;
// factored token affine acc = sum p*s*u + sum p*o) and :229-253 (exact merge
// of split states).
//
// Split kernel schedule. One 256-lane workgroup per (sequence, kv head,
// split); a split is processed in chunks of whole block rows (at most 160
// blocks and 320 tokens at head dim 64, 256 blocks and 128 tokens at 128).
// Per chunk:
//   1. loads: the first K tiles of each wave's first tile group, the per-token
//      V scale/offset, the next chunk's blocks (this chunk's blocks and their
//      partition-pattern words were requested during the previous chunk);
//   2. header stage, one lane per block, blocks sorted by decode-path class:
//      BlockDesc records in LDS;
//   3. each wave takes every fourth group of consecutive 16-token tiles
//      (attend_group; in the SPREAD variant a chunk shorter than four whole
//      groups is cut into smaller ones, so that every wave gets tiles): S for
//      the group on the matrix cores, the online softmax, then per tile its
//      texels decoded straight into P.V operands.
// At the end the four wave states are combined into the split's state; the
// last split workgroup of each (sequence, kv head) merges when the caller
// passes arrival counters, otherwise merge_kernel does.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <map>
#include <mutex>
#include <tuple>

#include "astc_decode_device.h"
#include "astc_format.h"
#include "astc_kv_hip.h"
#include "attention_device.h"
#include "host_common.h"

namespace akv_hip {

// Occupancy: three workgroups per CU at head dim 64, two at 128; the wide
// variant runs at most one per CU.
template <int D, int NCH, int G, bool DUMP, bool WIDE, bool SPREAD>
__global__ __launch_bounds__(kThreads)
__attribute__((amdgpu_waves_per_eu(D == 64 && !WIDE ? AKV_ASTC_WAVES : WIDE ? 1 : 2))) void astc_attn_kernel(
    KernelArgs a, const float* __restrict__ q, const uint16_t* __restrict__ k, const uint4* __restrict__ vblk,
    const uint16_t* __restrict__ vscale, const uint16_t* __restrict__ voffset, const AkvTables* __restrict__ tab,
    float* partial, float2* stats, uint16_t* __restrict__ dump, float* __restrict__ out, uint32_t* arrivals) {
    using C = Cfg<D, NCH, WIDE>;
    constexpr int TPG = Grp<G, D>::TPG;
    // K tiles of a wave's first group: the first kKEarly requested with the
    // chunk's other loads, the rest just before the header stage (all arrive
    // during it; issued together they stall the chunk's first phase).
    constexpr int kKEarly = TPG < 2 ? TPG : 2;
    __shared__ AstcShared<D, NCH, WIDE> sh;
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

    // Splits and chunks start at any token, not on block rows: a chunk covers
    // the block rows from row c0 / by, starting at row offset c0 % by (a block
    // row split between two chunks is decoded by both).
    auto chunk_blocks = [&](int c0) { return int((c0 % by + min(CT, split_end - c0) + by - 1) / by * cols); };
    auto k_rsrc = [&](int c0) {
        return seq_rsrc(DUMP ? nullptr : kseq + size_t(c0) * D, DUMP ? 0u : uint32_t(min(CT, split_end - c0)) * D * 2);
    };
    // Prologue: the decode tables and Q (from L2) and the first chunk's
    // blocks, all issued before the first wait.
    TableStage<kThreads> tables;
    tables.load(tab, tid);
    QStage<D, G> qst;
    if constexpr (!DUMP)
        if (wave == 0) qst.load(q + (size_t(b) * p.query_heads + size_t(kh) * G) * D);
    uint4 raw = load_block(bseq, cols, split_begin / by, chunk_blocks(split_begin), tid);
    tables.store(sh.tabs, tid);
    if constexpr (!DUMP)
        if (wave == 0) qst.store(a.qscale, &sh.q[0][0]);
    if (tid < kPathKeys) sh.key_count[tid] = 0;
    if (tid == 0) sh.nfill = 0;
    // Blocks the fill area holds (kFillSlots at most).
    const int fill_slots = min(kFillSlots, FillArea<NCH>::kTexels / f.ntex);

    // This lane's texel columns: x = n16 + 16 * kc -> block column | x in
    // block << 16 (one register each).
    int colpk[C::kColGroups];
#pragma unroll
    for (int kc = 0; kc < C::kColGroups; ++kc) {
        const int x = n16 + 16 * kc;
        const int bc = int(fdiv(uint32_t(x), a.mag_bx));
        colpk[kc] = bc | ((x - bc * f.bx) << 16);
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
        // Tiles per group: TPG, or, in the variant for chunks shorter than a
        // round (TPG tiles for every wave), as many as spread the chunk over
        // all four waves.
        const int gt = SPREAD ? min(TPG, (ntiles + kWaves - 1) / kWaves) : TPG;
        const int nblk = chunk_blocks(c0);
        // 1. Loads. Only the blocks cross chunks (requested one chunk ahead:
        // the header stage needs them first). The rest is requested here and
        // first used after the header stage, which covers its latency: the
        // blocks' partition-pattern words (they depend on the blocks), the
        // per-token scale/offset (two tokens per lane, clamped index), the
        // first K tiles of this wave's first group. Memory waits count loads
        // in issue order, so they are issued in the order of first use.
        const uint4 raw_now = raw;
        const uint4 pat = partition_words(raw_now, tab);
        uint32_t sc[2] = {0, 0}, of[2] = {0, 0};
        static_assert(C::kMaxTok <= 2 * kThreads, "two scale/offset tokens per lane");
        if constexpr (!DUMP) {
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int tc = c0 + min(tid + i * kThreads, ntok - 1);
                sc[i] = sseq[tc];
                of[i] = oseq[tc];
            }
        }
        if (c0 + CT < split_end) raw = load_block(bseq, cols, (c0 + CT) / by, chunk_blocks(c0 + CT), tid);
        uint4 kreg[TPG * C::kRowLoads];
        const __amdgpu_buffer_rsrc_t krs = k_rsrc(c0);
        if constexpr (!DUMP) {
#pragma unroll
            for (int t = 0; t < kKEarly; ++t) load_k_tile<D>(kreg + t * C::kRowLoads, krs, 16 * (gt * wave + t), lane);
        }
        // 2. Block headers, with the chunk's blocks sorted by decode-path class
        // so that the lanes of a wave take the same branches. Each block's raw
        // bits wait in its own descriptor slot; the lane that decodes a block
        // reads them from there and overwrites that slot. A chunk of one
        // wave's blocks gains nothing from the sort: each lane decodes the
        // block it stashed, with no barrier.
        const bool sorted = nblk > 64;
        int key = 0, rank = 0;
        if (tid < nblk) {
            stash_block(sh.u.h.desc[tid], raw_now);
            if (sorted) {
                key = block_path_key(raw_now);
                rank = int(atomicAdd(&sh.key_count[key], 1u));
            }
        }
#pragma unroll
        for (int i = 0; i < 2; ++i)
            if (tid + i * kThreads < C::kMaxTok)
                sh.tokrow[tid + i * kThreads] = token_row_entry(tid + i * kThreads, ntok, a.mag_by, f, cols, c0 % by);
        if (sorted) {
            __syncthreads();   // class counts complete
            static_assert(kPathKeys == 64, "one class per lane");
            place_by_class(sh.key_count, sh.order, key, rank, tid < nblk, tid);
            __syncthreads();   // sorted order complete (and every count read)
            if (wave == 0) sh.key_count[lane] = 0;   // for the next chunk (two barriers away)
        }
        if constexpr (!DUMP) {
#pragma unroll
            for (int t = kKEarly; t < TPG; ++t)
                load_k_tile<D>(kreg + t * C::kRowLoads, krs, 16 * (gt * wave + t), lane);
        }
        // What the texel stage needs besides the headers, written first so
        // that nothing of it stays in registers through the header stage:
        // each lane's own block's partition words (a field the header stage
        // does not touch), and the per-token scale | offset << 16 (zero past
        // the chunk, up to the tile edge).
        if (tid < nblk) {
            const uint4 w = block_part_words(raw_now, pat);
            uint32_t* part = sh.u.h.desc[tid].part;   // 4-byte aligned
            part[0] = w.x;
            part[1] = w.y;
            part[2] = w.z;
            part[3] = w.w;
        }
        if constexpr (!DUMP) {
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const int t = tid + i * kThreads;
                if (t < 16 * ntiles) sh.so[t] = t < ntok ? sc[i] | (of[i] << 16) : 0u;
            }
        }
        if (tid < nblk) {
            const int bi = sorted ? int(sh.order[tid]) : tid;
            decode_header<NCH, D == 128, true, D == 128 && NCH == 1>(sh.tabs, sh.u.h.desc[bi], sh.u.h.cv[tid], f.ntex);
            if (sh.u.h.desc[bi].info & kInfoFilled) {   // a slot of the fill area, or the compute path
                const uint32_t slot = atomicAdd(&sh.nfill, 1u);
                if (slot < uint32_t(fill_slots)) {
                    sh.u.h.fill[slot] = uint8_t(bi);
                    sh.u.h.desc[bi].info |= slot << kInfoFillShift;
                } else {
                    sh.u.h.desc[bi].info &= ~kInfoFilled;
                }
            }
        }
        __syncthreads();
        // 2b. Reduced weight grids: every texel of those blocks computed once,
        // by whole waves, rather than at each texel lookup.
        if (const int nfill = __builtin_amdgcn_readfirstlane(int(sh.nfill))) {
            fill_values<NCH, kThreads>(sh.u.h.desc, sh.tabs, f, sh.u.h.fill, min(nfill, fill_slots), sh.u.h.fv[0], tid);
            __syncthreads();
            if (tid == 0) sh.nfill = 0;   // read by every thread before the barrier above
        }
        // 3. This wave's groups of gt consecutive tiles (every fourth group):
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
                    column_texels<NCH, true>(sh.u.h.desc, sh.tabs, f, rows, colpk[kc] & 0xFFFF, colpk[kc] >> 16, sh.u.h.fv, tv);
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
#pragma unroll 1
            for (int tb0 = 16 * gt * wave; tb0 < ntok; tb0 += 16 * gt * kWaves) {
                const int ng = min(gt, (ntok - tb0 + 15) >> 4);
                uint32_t rows[4];   // token_row_entry of this lane's four tokens of the tile
                attend_group<D, G, true, C::kRowBlocksPerGroup>(
                    Fp16KOperands<D>{kreg}, &sh.q[0][0], ng, tb0, ntok, sh.so, C::kMaxTok, st, [&](int t, int kc, half4* va) {
                        if (kc == 0) {
                            if (t == 0) {   // S is done with this group's K rows
                                const int nb0 = tb0 + 16 * gt * kWaves;
#pragma unroll
                                for (int tt = 0; tt < TPG; ++tt)
                                    load_k_tile<D>(kreg + tt * C::kRowLoads, krs, nb0 + 16 * tt, lane);
                            }
                            tile_rows(sh.tokrow, tb0 + 16 * t, g, rows);
                        }
                        uint2 tv[4];
                        column_texels<NCH, true>(sh.u.h.desc, sh.tabs, f, rows, colpk[kc] & 0xFFFF, colpk[kc] >> 16, sh.u.h.fv, tv);
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
        merge_if_last<D, G>(arrivals + seq_kv, partial, stats, out, qh0, int(p.splits), int(p.splits), sh.ws, sh.u.comb,
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
        attend_group<D, G, false, 4>(Fp16KOperands<D>{kreg}, &sh.q[0][0], ng, tb0, ntok, nullptr, 4, st, [&](int t, int kc, half4* va) {
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
        merge_if_last<D, G>(arrivals + seq_kv, partial, stats, out, qh0, int(p.splits), int(p.splits), sh.ws, sh.comb,
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
    uint32_t cv[kThreads][kColourScratchWords];
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
    const uint4 pw = partition_words(raw, tab);
    stage_tables<kThreads>(tab, sh.tabs, tid);
    __syncthreads();
    if (tid < nblk) {
        stash_block(sh.desc[tid], raw);
        decode_header<4>(sh.tabs, sh.desc[tid], sh.cv[tid]);
        const uint4 w = block_part_words(raw, pw);
        uint32_t* part = sh.desc[tid].part;
        part[0] = w.x;
        part[1] = w.y;
        part[2] = w.z;
        part[3] = w.w;
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
}  // namespace

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

Footprint footprint(uint32_t bx, uint32_t by) {
    Footprint f{};
    f.bx = int(bx);
    f.by = int(by);
    f.ntex = int(bx * by);
    f.ds = int((1024 + bx / 2) / (bx - 1));
    f.dt = int((1024 + by / 2) / (by - 1));
    return f;
}

namespace {

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


int check_astc(const AkvAttnParams* p) {
    if (p->layout != AKV_LAYOUT_SCALAR && p->layout != AKV_LAYOUT_RGBA) return AKV_HIP_ERR_SHAPE;
    const uint32_t bx = p->block_x, by = p->block_y;
    if (bx < 4 || by < 4 || bx > 12 || by > 12 || bx * by > uint32_t(akv::kMaxTexels)) return AKV_HIP_ERR_FOOTPRINT;
    const uint32_t texcols = p->layout == AKV_LAYOUT_SCALAR ? p->dim : p->dim / 4;
    if (p->atlas_cols != (texcols + bx - 1) / bx) return AKV_HIP_ERR_SHAPE;
    if (uint64_t(p->atlas_rows) * by < p->tokens) return AKV_HIP_ERR_SHAPE;
    return 0;
}

// Chunk shape. ASTC V: the most whole block rows whose blocks fit the header
// stage and whose tokens fit a chunk; FP16 control: a whole chunk. Never more
// than one split.
template <int D, int NCH, bool WIDE>
int plan_chunks(const AkvAttnParams* p, bool astc, KernelArgs* a) {
    using C = Cfg<D, NCH, WIDE>;
    uint32_t tokens = C::kMaxTok;
    if (astc) {
        // A chunk starts at c0 = split * tile + k * chunk, where the chunk is
        // the whole split or a multiple of 16 tokens, so every start is a
        // multiple of g = gcd(16, tile, by) and sits at row offset c0 % by <=
        // by - g of its first block row: the most tokens whose block rows fit
        // the header stage at the worst offset, then whole rounds of tile
        // groups (every wave the same number of tiles) where that fits, else
        // whole tiles.
        const uint32_t by = p->block_y;
        auto gcd = [](uint32_t x, uint32_t y) {
            while (y) {
                const uint32_t t = x % y;
                x = y;
                y = t;
            }
            return x;
        };
        const uint32_t g16 = gcd(gcd(16, p->tile_tokens), by);
        const uint32_t rows = uint32_t(C::kMaxBlocks) / p->atlas_cols;
        if (rows * by <= by - g16) return AKV_HIP_ERR_SHAPE;
        tokens = std::min(rows * by - (by - g16), uint32_t(C::kMaxTok));
        const uint32_t G = p->query_heads / p->kv_heads;
        const uint32_t round = 16 * (16 / ((G <= 4 && D <= 64) ? 4 : 8)) * kWaves;
        tokens -= tokens >= round ? tokens % round : tokens % 16;
        if (tokens == 0) return AKV_HIP_ERR_SHAPE;
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
    // At most one workgroup per CU (MI355X: 256 CUs): the wide split kernel.
    a->wide = astc && p->dim == 64 && uint64_t(p->splits) * p->kv_heads * p->batch <= kCUs;
    if (p->dim == 64) {
        if (a->wide) return scalar ? plan_chunks<64, 1, true>(p, astc, a) : plan_chunks<64, 4, true>(p, astc, a);
        return scalar ? plan_chunks<64, 1, false>(p, astc, a) : plan_chunks<64, 4, false>(p, astc, a);
    }
    return scalar ? plan_chunks<128, 1, false>(p, astc, a) : plan_chunks<128, 4, false>(p, astc, a);
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

template <int D, int NCH, bool DUMP, bool WIDE, bool SPREAD>
hipError_t launch_astc_g(const KernelArgs& a, uint32_t G, const Ptrs& x, hipStream_t st) {
    dim3 grid(a.p.splits, a.p.kv_heads, a.p.batch);
    auto* s2 = reinterpret_cast<float2*>(x.stats);
    if constexpr (DUMP) {
        astc_attn_kernel<D, NCH, 1, true, WIDE, SPREAD><<<grid, kThreads, 0, st>>>(a, x.q, x.k, x.vblk, x.vs, x.vo, x.tab, x.partial,
                                                                      s2, x.dump, nullptr, nullptr);
        return hipGetLastError();
    }
    switch (G) {
#define AKV_CASE(GG)                                                                                       \
    case GG:                                                                                               \
        astc_attn_kernel<D, NCH, GG, DUMP, WIDE, SPREAD><<<grid, kThreads, 0, st>>>(a, x.q, x.k, x.vblk, x.vs, x.vo, \
                                                                               x.tab, x.partial, s2, x.dump, x.out, \
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
    // SPREAD: the variant whose tile groups shrink for chunks shorter than a
    // round (TPG tiles for every wave). Scalar layouts (11 or 22 block
    // columns) and the wide variant have such chunks; RGBA ones mostly do not
    // (6x5 at head dim 64 and every footprint at 128 fill whole rounds), and
    // there the fixed group is kept, which the compiler schedules better.
    if (a.p.dim == 64) {
        if (a.wide)
            return scalar ? launch_astc_g<64, 1, DUMP, true, true>(a, G, x, st)
                          : launch_astc_g<64, 4, DUMP, true, true>(a, G, x, st);
        if (scalar) return launch_astc_g<64, 1, DUMP, false, true>(a, G, x, st);
        if constexpr (!DUMP) {
            const uint32_t round = 16u * (G <= 4 ? 4u : 2u) * kWaves;   // tokens
            if (a.chunk_tokens % round) return launch_astc_g<64, 4, false, false, true>(a, G, x, st);
        }
        return launch_astc_g<64, 4, DUMP, false, false>(a, G, x, st);
    }
    return scalar ? launch_astc_g<128, 1, DUMP, false, true>(a, G, x, st)
                  : launch_astc_g<128, 4, DUMP, false, false>(a, G, x, st);
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


hipError_t launch_merge(const AkvAttnParams* p, const float* partial, const float* stats, float* out, hipStream_t st) {
    const uint64_t groups = uint64_t(p->batch) * p->query_heads;
    if (groups > 0x7FFFFFFFu) return hipErrorInvalidValue;
    merge_kernel<<<dim3(uint32_t(groups)), dim3(kThreads), 0, st>>>(p->splits, p->dim, partial,
                                                                    reinterpret_cast<const float2*>(stats), out);
    return hipGetLastError();
}

// `tab`: the footprint's decode tables on the current device, or NULL to use
// (and on first use upload) the library's allocated copy.
int run_astc(const AkvAttnParams* p, const float* q, const uint16_t* k, const void* v_blocks, const uint16_t* v_scale,
             const uint16_t* v_offset, float* partial, float* stats, float* out, bool with_merge, uint32_t* arrivals,
             void* stream, const AkvTables* tab = nullptr) {
    uint32_t G = 0;
    if (int rc = check_common(p, &G)) return rc;
    if (int rc = check_astc(p)) return rc;
    if (!q || !k || !v_blocks || !v_scale || !v_offset || !partial || !stats || (with_merge && !out))
        return AKV_HIP_ERR_NULL;
    if (!aligned16(q) || !aligned16(k) || !aligned16(v_blocks)) return AKV_HIP_ERR_ALIGN;
    if (!tab)
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

// --- the entry point that allocates nothing ----------------------------------
//
// akv_hip_decode_attention_noalloc keeps the one-launch step's workspace in a
// static device array instead of caller memory: the split states (partial,
// stats), the arrival counters and the decode tables of up to four footprints.
// Each GPU holds its own copy for the life of the process. Layout:
//   [0, 256 KiB)           four 64 KiB decode-table slots, one per footprint
//   [256 KiB, 512 KiB)     65,536 arrival counters (uint32), zero between calls
//   [512 KiB, 8.5 MiB)     split states: partial f32 [B][Hq][S][D], then stats
constexpr size_t kNaSlots = 4, kNaSlotBytes = 65536;
constexpr size_t kNaCounters = 65536;
constexpr size_t kNaStateBytes = size_t(8) << 20;
constexpr size_t kNaCounterOff = kNaSlots * kNaSlotBytes;
constexpr size_t kNaStateOff = kNaCounterOff + kNaCounters * sizeof(uint32_t);
constexpr size_t kNaBytes = kNaStateOff + kNaStateBytes;
static_assert(sizeof(AkvTables) <= kNaSlotBytes, "a table slot holds one footprint's tables");

static __device__ __align__(256) unsigned char scratch[kNaBytes];

__global__ void zero_words_kernel(uint32_t* p, uint32_t n) {
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) p[i] = 0u;
}

struct NoAllocDevice {
    unsigned char* base = nullptr;   // the device address of `scratch` on this GPU
    int slot_bx[kNaSlots] = {}, slot_by[kNaSlots] = {};
    int used = 0;
};

std::mutex g_na_mu;
std::map<int, NoAllocDevice> g_na;   // per device

// The current device's scratch address and the table slot of footprint (bx,
// by). The first call on a device looks the address up (hipGetSymbolAddress)
// and clears the arrival counters with a fill kernel on `st`; the first call
// for a footprint copies its tables into a free slot (a blocking copy from
// host memory, no allocation).
int noalloc_setup(int bx, int by, hipStream_t st, unsigned char** base, const AkvTables** tab) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return int(e);
    std::lock_guard<std::mutex> lock(g_na_mu);
    NoAllocDevice& d = g_na[dev];
    if (!d.base) {
        void* ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !ptr) {
            g_na.erase(dev);
            return e != hipSuccess ? int(e) : int(hipErrorInvalidSymbol);
        }
        unsigned char* b = static_cast<unsigned char*>(ptr);
        zero_words_kernel<<<dim3(64), dim3(kThreads), 0, st>>>(reinterpret_cast<uint32_t*>(b + kNaCounterOff),
                                                                uint32_t(kNaCounters));
        e = hipGetLastError();
        if (e != hipSuccess) {
            g_na.erase(dev);
            return int(e);
        }
        d.base = b;
    }
    int slot = -1;
    for (int i = 0; i < d.used; ++i)
        if (d.slot_bx[i] == bx && d.slot_by[i] == by) slot = i;
    if (slot < 0) {
        if (d.used == int(kNaSlots)) return AKV_HIP_ERR_SCRATCH;
        const AkvTables* host = akv::tables_for(bx, by);
        if (!host) return AKV_HIP_ERR_FOOTPRINT;
        e = hipMemcpy(d.base + d.used * kNaSlotBytes, host, sizeof(AkvTables), hipMemcpyHostToDevice);
        if (e != hipSuccess) return int(e);
        slot = d.used++;
        d.slot_bx[slot] = bx;
        d.slot_by[slot] = by;
    }
    *base = d.base;
    *tab = reinterpret_cast<const AkvTables*>(d.base + slot * kNaSlotBytes);
    return 0;
}

}  // namespace
}  // namespace akv_hip

using namespace akv_hip;

extern "C" {

int akv_hip_decode_attention_noalloc(const AkvAttnParams* p, const float* q, const uint16_t* k, const void* v_blocks,
                                     const uint16_t* v_scale, const uint16_t* v_offset, float* out, void* stream) {
    uint32_t G = 0;
    if (int rc = check_common(p, &G)) return rc;
    if (int rc = check_astc(p)) return rc;
    if (!q || !k || !v_blocks || !v_scale || !v_offset || !out) return AKV_HIP_ERR_NULL;
    if (!aligned16(q) || !aligned16(k) || !aligned16(v_blocks)) return AKV_HIP_ERR_ALIGN;
    const uint64_t states = uint64_t(p->batch) * p->query_heads * p->splits * p->dim;
    if ((states + uint64_t(p->batch) * p->query_heads * p->splits * 2) * sizeof(float) > kNaStateBytes ||
        uint64_t(p->batch) * p->kv_heads > kNaCounters)
        return AKV_HIP_ERR_SCRATCH;
    hipStream_t st = static_cast<hipStream_t>(stream);
    unsigned char* base = nullptr;
    const AkvTables* tab = nullptr;
    if (int rc = noalloc_setup(int(p->block_x), int(p->block_y), st, &base, &tab)) return rc;
    float* partial = reinterpret_cast<float*>(base + kNaStateOff);
    float* stats = partial + states;   // states is a multiple of 64: 8-byte aligned
    uint32_t* arrivals = reinterpret_cast<uint32_t*>(base + kNaCounterOff);
    return run_astc(p, q, k, v_blocks, v_scale, v_offset, partial, stats, out, true, arrivals, stream, tab);
}

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
    if (!aligned16(q) || !aligned16(k) || !aligned16(v)) return AKV_HIP_ERR_ALIGN;
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
    if (!aligned16(v_blocks)) return AKV_HIP_ERR_ALIGN;
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
    if (n && !aligned16(blocks)) return AKV_HIP_ERR_ALIGN;
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
        case AKV_HIP_ERR_TILE: return "tile_tokens/splits inconsistent (tile must be positive and "
                                      "splits = ceil(tokens/tile); paged: tile a multiple of 16 and of "
                                      "block_y, at most 62 pages)";
        case AKV_HIP_ERR_ALIGN: return "q, k, v and the V blocks must be 16-byte aligned";
        case AKV_HIP_ERR_SCRATCH: return "request exceeds the static scratch of akv_hip_decode_attention_noalloc "
                                         "(split states batch*query_heads*splits*(dim+2)*4 bytes <= 8 MiB, "
                                         "batch*kv_heads <= 65536, at most 4 footprints per device)";
        default: return code > 0 ? hipGetErrorString(hipError_t(code)) : "unknown error";
    }
}

}  // extern "C"
