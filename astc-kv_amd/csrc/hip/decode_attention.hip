// Split-K decode attention over FP16 K and ASTC-compressed V for gfx950, the
// FP16-K/V control, the split merge, and the decode readback kernels.
//
// Reference semantics: metal/attention_gqa_v10.metal:568-674 (one group per
// (kv head, split) holding the G query states of that kv head; online softmax;
// factored token affine acc = sum p*s*u + sum p*o) and :229-253 (exact merge
// of split states).
//
// Split kernel schedule. One 256-lane workgroup per (sequence, kv head,
// split). A split is processed in chunks of whole block rows (at most 144
// blocks and 240 tokens for head dim 64). Per chunk:
//   1. header stage, one lane per block: BlockDesc records in LDS (the
//      chunk's blocks were loaded one chunk ahead);
//   2. the chunk's K rows are loaded into registers in the MFMA operand
//      layout (16-byte loads) while the texel stage runs, and the next
//      chunk's blocks are requested;
//   3. texel stage, one lane per pair of tokens: u (the exact FP16 values
//      astcenc returns) channel-major into the LDS tile vt;
//   4. each wave takes every fourth 16-token tile: S^T = K.Q^T and O += V^T.P
//      on the matrix cores (v_mfma_f32_16x16x16_f16, q and p split into fp16
//      high and low parts so the products keep ~22 bits), the G query heads
//      padded to the 16 MFMA columns; online softmax per head with the per-token
//      V scale folded into p and the offset term accumulated separately.
// At the end the four wave states are combined into the split's state.
// A second kernel merges the splits.
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

typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

template <int D, int NCH, bool ASTC>
struct Cfg {
    static constexpr int kMaxBlocks = ASTC ? 144 : 1;                // blocks per chunk
    static constexpr int kVtTok = ASTC ? (D == 64 ? 240 : 112) : (D == 64 ? 256 : 128);
    static constexpr int kVtStride = kVtTok + 4;                     // odd multiple of 8 bytes per row
    static constexpr int kMaxTiles = kVtTok / 16;                    // 16-token MFMA tiles per chunk
    static constexpr int kWaveTiles = (kMaxTiles + kWaves - 1) / kWaves;
    static constexpr int kRowLoads = D / 32;                         // 16-byte row loads per lane per tile
    static constexpr int kKSteps = D / 16;
    static constexpr int kMBlocks = D / 16;
    static_assert((kVtStride / 4) % 2 == 1, "vt rows must be an odd multiple of 8 bytes");
};

struct KernelArgs {
    AkvAttnParams p;
    Footprint fp;
    uint32_t chunk_rows, chunk_tokens;   // block rows / tokens per full chunk
    uint32_t mag_by, mag_bx;             // ceil(2^24 / divisor)
    float qscale;                        // log2(e) / sqrt(dim)
};

// a / d with magic = ceil(2^24 / d): exact when a * d < 2^24 (the error term
// a * (magic * d - 2^24) stays below 2^24), which holds for every use below.
__device__ inline uint32_t fdiv(uint32_t a, uint32_t magic) { return (a * magic) >> 24; }
__device__ inline float half_to_float(uint16_t h) { return float(__builtin_bit_cast(_Float16, h)); }

// Order this wave's LDS accesses (a wave's LDS operations complete in order).
__device__ inline void wave_sync() {
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
    __builtin_amdgcn_wave_barrier();
}

template <int D, int NCH, bool ASTC>
struct Shared {
    using C = Cfg<D, NCH, ASTC>;
    union {
        _Float16 vt[D][C::kVtStride];   // u (or fp16 V), channel-major
        float comb[kWaves][D][16];      // final per-wave accumulators
    } u;
    BlockDesc<NCH> desc[C::kMaxBlocks];
    uint32_t cv[5][C::kMaxBlocks];      // colour values of the header stage
    uint32_t so[2][C::kVtTok];          // per-token V scale | offset << 16 (fp16), two chunks
    SmallLuts luts;
    float wm[kWaves][16], wl[kWaves][16], wo[kWaves][16];
};

// 16-byte rows of one wave's tiles in the MFMA A-operand layout: lane holds
// token 16 * tile + lane % 16, dims 32 * L + 8 * (lane / 16) .. + 7. Tokens at
// or past ntok read as zero.
template <int D, int NCH, bool ASTC>
__device__ inline void load_rows(uint4* r, const uint16_t* __restrict__ seq, int c0, int ntok, int wave, int lane) {
    using C = Cfg<D, NCH, ASTC>;
    const int n16 = lane & 15, g = lane >> 4;
#pragma unroll
    for (int j = 0; j < C::kWaveTiles; ++j)
#pragma unroll
        for (int L = 0; L < C::kRowLoads; ++L) {
            const int tok = 16 * (wave + kWaves * j) + n16;
            r[j * C::kRowLoads + L] =
                tok < ntok ? *reinterpret_cast<const uint4*>(seq + size_t(c0 + tok) * D + 32 * L + 8 * g)
                           : uint4{0, 0, 0, 0};
        }
}

// The blocks of the chunk starting at block row `row0` (one per lane).
template <int D, int NCH>
__device__ inline uint4 load_block(const KernelArgs& a, const uint4* __restrict__ bseq, int row0, int nrows, int tid) {
    const int nblk = nrows * int(a.p.atlas_cols);
    return tid < nblk ? bseq[size_t(row0) * a.p.atlas_cols + tid] : uint4{0, 0, 0, 0};
}

// Texel stage: one lane per (texel column, token pair) of the chunk; u into vt.
// Token columns from ntok up to the tile edge are zeroed.
template <int D, int NCH, bool ASTC>
__device__ inline void decode_texels(Shared<D, NCH, ASTC>& sh, const KernelArgs& a, int ntok, int tid) {
    const Footprint& f = a.fp;
    const int cols = int(a.p.atlas_cols);
    constexpr int TC = NCH == 1 ? D : D / 4;   // texel columns holding channels
    const int pairs = 8 * ((ntok + 15) >> 4);
    const uint32_t mag = (0x1000000u + uint32_t(pairs) - 1) / uint32_t(pairs);
    for (int it = tid; it < pairs * TC; it += kThreads) {
        const int x = int(fdiv(uint32_t(it), mag));
        const int t = 2 * (it - x * pairs);
        const int bc = int(fdiv(uint32_t(x), a.mag_bx)), xx = x - bc * f.bx;
        uint2 v[2];
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            v[k] = uint2{0, 0};
            if (t + k < ntok) {
                const int r = int(fdiv(uint32_t(t + k), a.mag_by)), y = t + k - r * f.by;
                v[k] = texel_fp16<NCH>(sh.desc[r * cols + bc], sh.luts, f, xx, y);
            }
        }
        if constexpr (NCH == 1) {
            *reinterpret_cast<uint32_t*>(&sh.u.vt[x][t]) = v[0].x | (v[1].x << 16);
        } else {
            *reinterpret_cast<uint32_t*>(&sh.u.vt[4 * x + 0][t]) = __builtin_amdgcn_perm(v[1].x, v[0].x, 0x05040100u);
            *reinterpret_cast<uint32_t*>(&sh.u.vt[4 * x + 1][t]) = __builtin_amdgcn_perm(v[1].x, v[0].x, 0x07060302u);
            *reinterpret_cast<uint32_t*>(&sh.u.vt[4 * x + 2][t]) = __builtin_amdgcn_perm(v[1].y, v[0].y, 0x05040100u);
            *reinterpret_cast<uint32_t*>(&sh.u.vt[4 * x + 3][t]) = __builtin_amdgcn_perm(v[1].y, v[0].y, 0x07060302u);
        }
    }
}

// FP16 control: transpose this wave's V rows (in registers) into its vt columns.
template <int D, int NCH, bool ASTC>
__device__ inline void stage_fp16_rows(Shared<D, NCH, ASTC>& sh, const uint4* v, int wave, int lane) {
    using C = Cfg<D, NCH, ASTC>;
    const int n16 = lane & 15, g = lane >> 4;
#pragma unroll
    for (int j = 0; j < C::kWaveTiles; ++j)
#pragma unroll
        for (int L = 0; L < C::kRowLoads; ++L) {
            const uint4 x = v[j * C::kRowLoads + L];
            const uint32_t w[4] = {x.x, x.y, x.z, x.w};
            const int tok = 16 * (wave + kWaves * j) + n16, c0 = 32 * L + 8 * g;
            if (tok < C::kVtTok) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    sh.u.vt[c0 + 2 * i][tok] = __builtin_bit_cast(_Float16, uint16_t(w[i]));
                    sh.u.vt[c0 + 2 * i + 1][tok] = __builtin_bit_cast(_Float16, uint16_t(w[i] >> 16));
                }
            }
        }
}

// --- the split kernel --------------------------------------------------------

template <int D, int NCH, int G, bool ASTC, bool DUMP>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(3))) void attn_kernel(
    KernelArgs a, const float* __restrict__ q, const uint16_t* __restrict__ k, const uint4* __restrict__ vblk,
    const uint16_t* __restrict__ vh, const uint16_t* __restrict__ vscale, const uint16_t* __restrict__ voffset,
    const AkvTables* __restrict__ tab, float* __restrict__ partial, float2* __restrict__ stats,
    uint16_t* __restrict__ dump) {
    using C = Cfg<D, NCH, ASTC>;
    __shared__ Shared<D, NCH, ASTC> sh;
    const AkvAttnParams& p = a.p;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int n16 = lane & 15, g = lane >> 4;
    const int split = blockIdx.x, kh = blockIdx.y, b = blockIdx.z;
    const int T = int(p.tokens);
    const int split_begin = split * int(p.tile_tokens);
    const int split_end = min(split_begin + int(p.tile_tokens), T);
    const int CT = int(a.chunk_tokens);

    const size_t seq_kv = size_t(b) * p.kv_heads + kh;
    const uint16_t* kseq = DUMP ? nullptr : k + seq_kv * p.tokens * D;
    const uint16_t* vseq = ASTC ? nullptr : vh + seq_kv * p.tokens * D;
    const uint4* bseq = ASTC ? vblk + seq_kv * p.atlas_rows * p.atlas_cols : nullptr;
    const uint16_t* sseq = (ASTC && !DUMP) ? vscale + seq_kv * p.tokens : nullptr;
    const uint16_t* oseq = (ASTC && !DUMP) ? voffset + seq_kv * p.tokens : nullptr;

    uint4 raw = uint4{0, 0, 0, 0};
    if constexpr (ASTC) {
        const int rows0 = (min(CT, split_end - split_begin) + int(p.block_y) - 1) / int(p.block_y);
        raw = load_block<D, NCH>(a, bseq, split_begin / int(p.block_y), rows0, tid);
        stage_luts(tab, sh.luts, tid, kThreads);
    }

    // Q as the B operand of Q.K^T, split into fp16 high and low parts. k-step
    // ks covers dims 32*(ks/2) + 8*g + 4*(ks%2) + j, matching the K row loads.
    half4 qhi[C::kKSteps], qlo[C::kKSteps];
#pragma unroll
    for (int ks = 0; ks < C::kKSteps; ++ks)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float v = 0.0f;
            if (!DUMP && n16 < G)
                v = q[(size_t(b) * p.query_heads + size_t(kh) * G + n16) * D + 32 * (ks / 2) + 8 * g + 4 * (ks % 2) +
                      j] *
                    a.qscale;
            const _Float16 hi = _Float16(v);
            qhi[ks][j] = hi;
            qlo[ks][j] = _Float16(v - float(hi));
        }

    float m_run = -INFINITY, l_run = 0.0f, off_run = 0.0f;
    floatx4 o[C::kMBlocks];
#pragma unroll
    for (int mb = 0; mb < C::kMBlocks; ++mb) o[mb] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    if constexpr (ASTC) __syncthreads();   // LUTs staged

    int buf = 0;
    for (int c0 = split_begin; c0 < split_end; c0 += CT, buf ^= 1) {
        const int ntok = min(CT, split_end - c0);
        const int ntiles = (ntok + 15) >> 4;
        uint4 kreg[C::kWaveTiles * C::kRowLoads];
        uint4 vreg[ASTC ? 1 : C::kWaveTiles * C::kRowLoads];
        if constexpr (ASTC) {
            // Scale/offset of the chunk's tokens (consumed after the next barrier).
            uint32_t so = 0;
            if (!DUMP && tid < ntok) so = uint32_t(sseq[c0 + tid]) | (uint32_t(oseq[c0 + tid]) << 16);
            // 1. Block headers.
            const int nblk = ((ntok + int(p.block_y) - 1) / int(p.block_y)) * int(p.atlas_cols);
            if (tid < nblk) decode_header<NCH>(raw, tab, sh.luts, sh.desc[tid], &sh.cv[0][tid], C::kMaxBlocks);
            // 2. This chunk's K rows, then the next chunk's blocks.
            if constexpr (!DUMP) load_rows<D, NCH, ASTC>(kreg, kseq, c0, ntok, wave, lane);
            const int cn = c0 + CT;
            if (cn < split_end) {
                const int rows = (min(CT, split_end - cn) + int(p.block_y) - 1) / int(p.block_y);
                raw = load_block<D, NCH>(a, bseq, cn / int(p.block_y), rows, tid);
            }
            if (!DUMP && tid < ntok) sh.so[buf][tid] = so;
            __syncthreads();
            // 3. Texels.
            decode_texels<D, NCH, ASTC>(sh, a, ntok, tid);
            __syncthreads();
        } else {
            load_rows<D, NCH, ASTC>(kreg, kseq, c0, ntok, wave, lane);
            load_rows<D, NCH, ASTC>(vreg, vseq, c0, ntok, wave, lane);
            stage_fp16_rows<D, NCH, ASTC>(sh, vreg, wave, lane);
            wave_sync();
        }
        if constexpr (DUMP) {
            uint16_t* dst = dump + (seq_kv * p.tokens + c0) * D;
            for (int i = tid; i < ntok * D; i += kThreads) {
                const int t = i / D, c = i - t * D;
                dst[i] = __builtin_bit_cast(uint16_t, sh.u.vt[c][t]);
            }
            __syncthreads();
            continue;
        }

        // 4. Scores of this wave's tiles.
        floatx4 s[C::kWaveTiles];
        float mt = -INFINITY;
#pragma unroll
        for (int j = 0; j < C::kWaveTiles; ++j) {
            const int tt = wave + kWaves * j;
            s[j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
            if (tt >= ntiles) continue;
#pragma unroll
            for (int ks = 0; ks < C::kKSteps; ++ks) {
                const uint4 kk = kreg[j * C::kRowLoads + ks / 2];
                const half4 ka = __builtin_bit_cast(half4, (ks & 1) ? uint2{kk.z, kk.w} : uint2{kk.x, kk.y});
                s[j] = __builtin_amdgcn_mfma_f32_16x16x16f16(ka, qhi[ks], s[j], 0, 0, 0);
                s[j] = __builtin_amdgcn_mfma_f32_16x16x16f16(ka, qlo[ks], s[j], 0, 0, 0);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if (16 * tt + 4 * g + i >= ntok) s[j][i] = -INFINITY;
                mt = fmaxf(mt, s[j][i]);
            }
        }
        if (wave < ntiles) {
            mt = fmaxf(mt, __shfl_xor(mt, 16, 64));
            mt = fmaxf(mt, __shfl_xor(mt, 32, 64));
            const float m_new = fmaxf(m_run, mt);
            const float alpha = exp2f(m_run - m_new);
            m_run = m_new;
            l_run *= alpha;
            off_run *= alpha;
#pragma unroll
            for (int mb = 0; mb < C::kMBlocks; ++mb) o[mb] *= alpha;
#pragma unroll
            for (int j = 0; j < C::kWaveTiles; ++j) {
                const int tt = wave + kWaves * j;
                if (tt >= ntiles) break;
                uint4 so4 = uint4{0x3C00u, 0, 0x3C00u, 0};   // FP16 control: scale 1, offset 0
                if constexpr (ASTC) so4 = *reinterpret_cast<const uint4*>(&sh.so[buf][16 * tt + 4 * g]);
                const uint32_t sov[4] = {so4.x, so4.y, so4.z, so4.w};
                half4 phi, plo;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float pr = exp2f(s[j][i] - m_new);
                    l_run += pr;
                    float pv = pr;
                    if constexpr (ASTC) {
                        pv = pr * half_to_float(uint16_t(sov[i]));
                        off_run = fmaf(pr, half_to_float(uint16_t(sov[i] >> 16)), off_run);
                    }
                    const _Float16 h = _Float16(pv);
                    phi[i] = h;
                    plo[i] = _Float16(pv - float(h));
                }
#pragma unroll
                for (int mb = 0; mb < C::kMBlocks; ++mb) {
                    const half4 va = *reinterpret_cast<const half4*>(&sh.u.vt[16 * mb + n16][16 * tt + 4 * g]);
                    o[mb] = __builtin_amdgcn_mfma_f32_16x16x16f16(va, phi, o[mb], 0, 0, 0);
                    o[mb] = __builtin_amdgcn_mfma_f32_16x16x16f16(va, plo, o[mb], 0, 0, 0);
                }
            }
        }
        if constexpr (!ASTC) wave_sync();   // this wave's vt columns are rewritten next chunk
    }
    if constexpr (DUMP) return;

    // Wave state: sums over the four lane groups; accumulators to LDS.
    l_run += __shfl_xor(l_run, 16, 64);
    l_run += __shfl_xor(l_run, 32, 64);
    off_run += __shfl_xor(off_run, 16, 64);
    off_run += __shfl_xor(off_run, 32, 64);
    __syncthreads();   // every wave is done with vt
#pragma unroll
    for (int mb = 0; mb < C::kMBlocks; ++mb)
#pragma unroll
        for (int i = 0; i < 4; ++i) sh.u.comb[wave][16 * mb + 4 * g + i][n16] = o[mb][i];
    if (g == 0) {
        sh.wm[wave][n16] = m_run;
        sh.wl[wave][n16] = l_run;
        sh.wo[wave][n16] = off_run;
    }
    __syncthreads();

    // Combine the four waves -> this split's state.
    const int S = int(p.splits);
    for (int i = tid; i < G * D; i += kThreads) {
        const int h = i / D, c = i - h * D;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) M = fmaxf(M, sh.wm[w][h]);
        float acc = 0.0f, l = 0.0f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const float e = sh.wm[w][h] == -INFINITY ? 0.0f : exp2f(sh.wm[w][h] - M);
            acc = fmaf(e, sh.u.comb[w][c][h] + sh.wo[w][h], acc);
            l = fmaf(e, sh.wl[w][h], l);
        }
        const size_t qh = size_t(b) * p.query_heads + size_t(kh) * G + h;
        partial[(qh * S + split) * D + c] = acc;
        if (c == 0) stats[qh * S + split] = float2{M * 0.69314718055994531f, l};
    }
}

// Merge: one workgroup per (sequence, query head); wave w takes splits
// w, w + 4, ...; lane = channel (and channel + 64 for dim 128).
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

// Standalone block decode: 256 blocks per workgroup -> FP16 RGBA texels.
struct BlocksShared {
    SmallLuts luts;
    BlockDesc<4> desc[kThreads];
    uint32_t cv[5][kThreads];
};

__global__ __launch_bounds__(kThreads) void decode_blocks_kernel(const uint4* __restrict__ blocks, size_t n,
                                                                 Footprint f, const AkvTables* __restrict__ tab,
                                                                 uint2* __restrict__ out) {
    __shared__ BlocksShared sh;
    const int tid = threadIdx.x;
    stage_luts(tab, sh.luts, tid, kThreads);
    __syncthreads();
    const size_t first = size_t(blockIdx.x) * kThreads;
    const int nblk = int(min(size_t(kThreads), n - first));
    if (tid < nblk) decode_header<4>(blocks[first + tid], tab, sh.luts, sh.desc[tid], &sh.cv[0][tid], kThreads);
    __syncthreads();
    for (int it = tid; it < nblk * f.ntex; it += kThreads) {
        const int blk = it / f.ntex, i = it - blk * f.ntex;
        const int y = i / f.bx, x = i - y * f.bx;
        out[(first + blk) * f.ntex + i] = texel_fp16<4>(sh.desc[blk], sh.luts, f, x, y);
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

// Chunk shape: the most block rows whose blocks fit the header stage and whose
// tokens, rounded up to whole 16-token tiles, fit the LDS tile; never more
// than one split. The FP16 control uses whole LDS tiles.
template <int D, int NCH, bool ASTC>
int plan_chunks(const AkvAttnParams* p, KernelArgs* a) {
    using C = Cfg<D, NCH, ASTC>;
    if (!ASTC) {
        a->chunk_rows = 0;
        a->chunk_tokens = C::kVtTok;
    } else {
        const uint32_t cols = p->atlas_cols, by = p->block_y;
        uint32_t r = uint32_t(C::kMaxBlocks) / cols;
        while (r > 0 && (r * by + 15) / 16 * 16 > uint32_t(C::kVtTok)) --r;
        if (r == 0) return AKV_HIP_ERR_SHAPE;
        const uint32_t tile_rows = p->tile_tokens / by;
        if (tile_rows < r) r = tile_rows;
        a->chunk_rows = r;
        a->chunk_tokens = r * by;
    }
    if (a->chunk_tokens > p->tile_tokens) a->chunk_tokens = p->tile_tokens;
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
    if (!astc) return p->dim == 64 ? plan_chunks<64, 4, false>(p, a) : plan_chunks<128, 4, false>(p, a);
    if (p->dim == 64) return scalar ? plan_chunks<64, 1, true>(p, a) : plan_chunks<64, 4, true>(p, a);
    return scalar ? plan_chunks<128, 1, true>(p, a) : plan_chunks<128, 4, true>(p, a);
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
};

template <int D, int NCH, bool ASTC, bool DUMP>
hipError_t launch_g(const KernelArgs& a, uint32_t G, const Ptrs& x, hipStream_t st) {
    dim3 grid(a.p.splits, a.p.kv_heads, a.p.batch);
    auto* s2 = reinterpret_cast<float2*>(x.stats);
    switch (G) {
#define AKV_CASE(GG)                                                                                             \
    case GG:                                                                                                     \
        attn_kernel<D, NCH, GG, ASTC, DUMP><<<grid, kThreads, 0, st>>>(a, x.q, x.k, x.vblk, x.vh, x.vs, x.vo,   \
                                                                        x.tab, x.partial, s2, x.dump);          \
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

template <bool ASTC, bool DUMP>
hipError_t launch(const KernelArgs& a, uint32_t G, const Ptrs& x, hipStream_t st) {
    if constexpr (ASTC) {
        const bool scalar = a.p.layout == AKV_LAYOUT_SCALAR;
        if (a.p.dim == 64)
            return scalar ? launch_g<64, 1, true, DUMP>(a, G, x, st) : launch_g<64, 4, true, DUMP>(a, G, x, st);
        return scalar ? launch_g<128, 1, true, DUMP>(a, G, x, st) : launch_g<128, 4, true, DUMP>(a, G, x, st);
    } else {
        if (a.p.dim == 64) return launch_g<64, 4, false, false>(a, G, x, st);
        return launch_g<128, 4, false, false>(a, G, x, st);
    }
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
             const uint16_t* v_offset, float* partial, float* stats, float* out, bool with_merge, void* stream) {
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
    const Ptrs x{q, k, static_cast<const uint4*>(v_blocks), nullptr, v_scale, v_offset, tab, partial, stats, nullptr};
    hipError_t e = launch<true, false>(a, G, x, st);
    if (e == hipSuccess && with_merge) e = launch_merge(p, partial, stats, out, st);
    return as_int(e);
}

}  // namespace
}  // namespace akv_hip

using namespace akv_hip;

extern "C" {

int akv_hip_attention_split(const AkvAttnParams* p, const float* q, const uint16_t* k, const void* v_blocks,
                            const uint16_t* v_scale, const uint16_t* v_offset, float* partial, float* stats,
                            void* stream) {
    return run_astc(p, q, k, v_blocks, v_scale, v_offset, partial, stats, nullptr, false, stream);
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
    return run_astc(p, q, k, v_blocks, v_scale, v_offset, partial, stats, out, true, stream);
}

int akv_hip_fp16_attention(const AkvAttnParams* p, const float* q, const uint16_t* k, const uint16_t* v,
                           float* partial, float* stats, float* out, void* stream) {
    uint32_t G = 0;
    if (int rc = check_common(p, &G)) return rc;
    if (!q || !k || !v || !partial || !stats || !out) return AKV_HIP_ERR_NULL;
    KernelArgs a;
    if (int rc = make_args(p, false, &a)) return rc;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const Ptrs x{q, k, nullptr, v, nullptr, nullptr, nullptr, partial, stats, nullptr};
    hipError_t e = launch<false, false>(a, G, x, st);
    if (e == hipSuccess) e = launch_merge(p, partial, stats, out, st);
    return as_int(e);
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
    return as_int(launch<true, true>(a, G, x, static_cast<hipStream_t>(stream)));
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
