// Split-K decode attention over FP16 K and ASTC-compressed V for gfx950, the
// FP16-K/V control, the split merge, and the decode readback kernels.
//
// Reference semantics: metal/attention_gqa_v10.metal:568-674 (one group per
// (kv head, split) holding G query states; online softmax; factored token
// affine acc = sum p*s*u + sum p*o) and :229-253 (exact merge of split states).
//
// Schedule of the split kernel: one 256-lane workgroup per (sequence, kv head,
// split). It
//   1. issues the split's K loads (16-byte fp16 loads, 32 KB per workgroup)
//      into registers first, so HBM latency overlaps the V decode;
//   2. decodes the split's V blocks into an LDS tile u[tile][dim] (fp16,
//      exactly the values astcenc returns), one lane per block header, then
//      one lane per texel;
//   3. Q.K for all G query heads of the kv head from the staged registers
//      (each K and V byte is read once per kv head, not once per query head);
//   4. the split's softmax statistics per head (one wave per head), folding the
//      per-token V scale into the probabilities;
//   5. P.V from the LDS tile, reduced across token groups.
// The merge kernel then combines splits exactly.
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

constexpr int kThreads = 256;
constexpr int kTileElems = 16384;  // tile_tokens * dim per workgroup (32 KB of fp16 K)

template <int NCH>
struct ChunkCap {
    static constexpr int blocks = NCH == 4 ? 192 : 256;
};

// Per-launch constants derived on the host.
struct KernelArgs {
    AkvAttnParams p;
    uint32_t G;        // query heads per kv head
    int ds, dt;        // weight infill steps
    uint32_t mag_bx, mag_by, mag_cols;  // ceil(65536 / divisor)
    float qscale;      // log2(e) / sqrt(dim)
    uint32_t sub_tokens;  // tokens per in-kernel sub-tile (<= 16384/dim, multiple of block_y)
};

__device__ inline uint32_t fdiv(uint32_t a, uint32_t magic) { return (a * magic) >> 16; }

__device__ inline float half_to_float(uint16_t h) { return float(__builtin_bit_cast(_Float16, h)); }

__device__ inline float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}
__device__ inline float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

template <int D, int NCH, int G>
struct SplitShared {
    static constexpr int kMaxTile = kTileElems / D;
    static constexpr int kCP = D / 2;             // channel pairs
    static constexpr int kTG = kThreads / kCP;    // PV token groups
    _Float16 vt[kTileElems];                      // u[tile][D]
    float sc[G][kMaxTile];                        // scores, then p * scale
    float qs[G][D];
    float mlo[G][3];                              // running max, sum, offset term
    float alpha[G];                               // rescale of the running state
    SmallLuts luts;
    union {
        struct {
            BlockDesc<NCH> desc[ChunkCap<NCH>::blocks];
            uint32_t cv[5][kThreads];
        } dec;
        float red[kTG][G][D];
    } u;
};

// Stage 2 of the V decode for one chunk of block rows: every texel of the
// chunk that maps to a token < nt is written into vt.
template <int D, int NCH, int G>
__device__ inline void decode_chunk_texels(SplitShared<D, NCH, G>& sh, const KernelArgs& a, int tid, int chunk_row0,
                                           int nrows, int nt) {
    constexpr int TC = NCH == 1 ? D : D / 4;  // texel columns holding channels
    const int by = int(a.p.block_y), bx = int(a.p.block_x), cols = int(a.p.atlas_cols);
    const int items = nrows * by * TC;
    for (int it = tid; it < items; it += kThreads) {
        const int tl = it / TC, xc = it - tl * TC;
        const int t_tile = chunk_row0 * by + tl;
        if (t_tile >= nt) continue;
        const int brow = int(fdiv(uint32_t(tl), a.mag_by)), y = tl - brow * by;
        const int bcol = int(fdiv(uint32_t(xc), a.mag_bx)), x = xc - bcol * bx;
        uint32_t C[NCH];
        decode_texel<NCH>(sh.u.dec.desc[brow * cols + bcol], sh.luts, x, y, bx, a.ds, a.dt, C);
        if constexpr (NCH == 1) {
            sh.vt[t_tile * D + xc] = __builtin_bit_cast(_Float16, uint16_t(pack_fp16_rtz(C[0], 0) & 0xFFFF));
        } else {
            uint2 h{pack_fp16_rtz(C[0], C[1]), pack_fp16_rtz(C[2], C[3])};
            *reinterpret_cast<uint2*>(&sh.vt[t_tile * D + 4 * xc]) = h;
        }
    }
}

// ASTC: decode V rows of this split into sh.vt. FP16: copy V rows.
template <int D, int NCH, int G, bool ASTC>
__device__ inline void stage_v(SplitShared<D, NCH, G>& sh, const KernelArgs& a, const uint4* __restrict__ vblk,
                               const uint16_t* __restrict__ vh, const AkvTables* __restrict__ tab, int b, int kh,
                               int t0, int nt, int tid) {
    const AkvAttnParams& p = a.p;
    if constexpr (ASTC) {
        const int by = int(p.block_y), cols = int(p.atlas_cols);
        const int rows = (nt + by - 1) / by;
        const int row0 = t0 / by;
        const int chunk_rows = ChunkCap<NCH>::blocks / cols;
        const uint4* base = vblk + (size_t(b) * p.kv_heads + kh) * p.atlas_rows * cols;
        for (int cr = 0; cr < rows; cr += chunk_rows) {
            const int nrows = min(chunk_rows, rows - cr);
            const int nblk = nrows * cols;
            __syncthreads();
            if (tid < nblk) {
                const int r = int(fdiv(uint32_t(tid), a.mag_cols));
                const int c = tid - r * cols;
                uint4 raw = base[size_t(row0 + cr + r) * cols + c];
                decode_header<NCH>(raw, tab, sh.luts, sh.u.dec.desc[tid], &sh.u.dec.cv[0][tid], kThreads);
            }
            __syncthreads();
            decode_chunk_texels<D, NCH, G>(sh, a, tid, cr, nrows, nt);
        }
    } else {
        const uint4* src = reinterpret_cast<const uint4*>(vh + ((size_t(b) * p.kv_heads + kh) * p.tokens + t0) * D);
        uint4* dst = reinterpret_cast<uint4*>(sh.vt);
        for (int i = tid; i < nt * D / 8; i += kThreads) dst[i] = src[i];
    }
    __syncthreads();
}

template <int D, int NCH, int G, bool ASTC, bool DUMP>
__global__ __launch_bounds__(kThreads) void split_kernel(KernelArgs a, const float* __restrict__ q,
                                                         const uint16_t* __restrict__ k,
                                                         const uint4* __restrict__ vblk,
                                                         const uint16_t* __restrict__ vh,
                                                         const uint16_t* __restrict__ vscale,
                                                         const uint16_t* __restrict__ voffset,
                                                         const AkvTables* __restrict__ tab,
                                                         float* __restrict__ partial, float2* __restrict__ stats,
                                                         uint16_t* __restrict__ dump) {
    using Sh = SplitShared<D, NCH, G>;
    __shared__ Sh sh;
    const AkvAttnParams& p = a.p;
    const int tid = threadIdx.x;
    const int split = blockIdx.x, kh = blockIdx.y, b = blockIdx.z;
    const int t_begin = split * int(p.tile_tokens);
    const int t_end = min(t_begin + int(p.tile_tokens), int(p.tokens));

    constexpr int LPT = D / 8;                 // lanes per token: 8 fp16 channels each
    constexpr int TPR = kThreads / LPT;        // tokens per round
    constexpr int ROUNDS = Sh::kMaxTile / TPR;
    constexpr int CP = Sh::kCP, TG = Sh::kTG;
    const int tok_lane = tid / LPT, c8 = tid % LPT;
    const int cp = tid % CP, tg = tid / CP;
    const int wave = tid >> 6, lane = tid & 63;

    if constexpr (!DUMP) {
        for (int i = tid; i < G * D; i += kThreads)
            sh.qs[i / D][i % D] = q[(size_t(b) * p.query_heads + size_t(kh) * G) * D + i] * a.qscale;
        if (tid < G) {
            sh.mlo[tid][0] = -INFINITY;
            sh.mlo[tid][1] = 0.0f;
            sh.mlo[tid][2] = 0.0f;
        }
    }
    if constexpr (ASTC) stage_luts(tab, sh.luts, tid, kThreads);
    float acc[G][2];
#pragma unroll
    for (int h = 0; h < G; ++h) acc[h][0] = acc[h][1] = 0.0f;

    // Sub-tiles of at most kMaxTile tokens (a multiple of the block height);
    // softmax statistics and accumulators are rescaled online across them.
    for (int s0 = t_begin; s0 < t_end; s0 += int(a.sub_tokens)) {
        const int nt = min(int(a.sub_tokens), t_end - s0);
        uint4 kreg[ROUNDS];
        if constexpr (!DUMP) {
            const uint16_t* kb = k + ((size_t(b) * p.kv_heads + kh) * p.tokens + s0) * D + c8 * 8;
#pragma unroll
            for (int r = 0; r < ROUNDS; ++r) {
                const int t = r * TPR + tok_lane;
                kreg[r] = t < nt ? *reinterpret_cast<const uint4*>(kb + size_t(t) * D) : uint4{0, 0, 0, 0};
            }
        }
        __syncthreads();  // previous sub-tile's readers of vt/sc are done
        stage_v<D, NCH, G, ASTC>(sh, a, vblk, vh, tab, b, kh, s0, nt, tid);

        if constexpr (DUMP) {
            uint16_t* dst = dump + ((size_t(b) * p.kv_heads + kh) * p.tokens + s0) * D;
            const uint16_t* src = reinterpret_cast<const uint16_t*>(sh.vt);
            for (int i = tid; i < nt * D; i += kThreads) dst[i] = src[i];
            continue;
        }

        // Q.K from the staged registers.
        {
            float qv[G][8];
#pragma unroll
            for (int h = 0; h < G; ++h)
#pragma unroll
                for (int j = 0; j < 8; ++j) qv[h][j] = sh.qs[h][c8 * 8 + j];
#pragma unroll
            for (int r = 0; r < ROUNDS; ++r) {
                const int t = r * TPR + tok_lane;
                const uint32_t kw[4] = {kreg[r].x, kreg[r].y, kreg[r].z, kreg[r].w};
                float kf[8];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    kf[2 * j] = half_to_float(uint16_t(kw[j] & 0xFFFF));
                    kf[2 * j + 1] = half_to_float(uint16_t(kw[j] >> 16));
                }
#pragma unroll
                for (int h = 0; h < G; ++h) {
                    float s = 0.0f;
#pragma unroll
                    for (int j = 0; j < 8; ++j) s = fmaf(qv[h][j], kf[j], s);
#pragma unroll
                    for (int o = 1; o < LPT; o <<= 1) s += __shfl_xor(s, o, 64);
                    if (c8 == 0 && t < nt) sh.sc[h][t] = s;
                }
            }
        }
        __syncthreads();

        // Online softmax update per head; fold the per-token V scale into p.
        const size_t meta = (size_t(b) * p.kv_heads + kh) * p.tokens + s0;
        for (int h = wave; h < G; h += kThreads / 64) {
            float m = -INFINITY;
            for (int t = lane; t < nt; t += 64) m = fmaxf(m, sh.sc[h][t]);
            const float m_old = sh.mlo[h][0];
            const float m_new = fmaxf(m_old, wave_max(m));
            float l = 0.0f, off = 0.0f;
            for (int t = lane; t < nt; t += 64) {
                const float pr = exp2f(sh.sc[h][t] - m_new);
                l += pr;
                if constexpr (ASTC) {
                    sh.sc[h][t] = pr * half_to_float(vscale[meta + t]);
                    off = fmaf(pr, half_to_float(voffset[meta + t]), off);
                } else {
                    sh.sc[h][t] = pr;
                }
            }
            l = wave_sum(l);
            off = wave_sum(off);
            if (lane == 0) {
                const float alpha = exp2f(m_old - m_new);
                sh.alpha[h] = alpha;
                sh.mlo[h][0] = m_new;
                sh.mlo[h][1] = fmaf(sh.mlo[h][1], alpha, l);
                sh.mlo[h][2] = fmaf(sh.mlo[h][2], alpha, off);
            }
        }
        __syncthreads();

        // P.V over the LDS tile: lane = channel pair, token groups reduced at the end.
#pragma unroll
        for (int h = 0; h < G; ++h) {
            const float alpha = sh.alpha[h];
            acc[h][0] *= alpha;
            acc[h][1] *= alpha;
        }
        for (int t = tg; t < nt; t += TG) {
            const uint32_t u2 = *reinterpret_cast<const uint32_t*>(&sh.vt[t * D + 2 * cp]);
            const float u0 = half_to_float(uint16_t(u2 & 0xFFFF)), u1 = half_to_float(uint16_t(u2 >> 16));
#pragma unroll
            for (int h = 0; h < G; ++h) {
                const float w = sh.sc[h][t];
                acc[h][0] = fmaf(w, u0, acc[h][0]);
                acc[h][1] = fmaf(w, u1, acc[h][1]);
            }
        }
    }
    if constexpr (DUMP) return;

    // The decode scratch is dead now; reuse it for the token-group reduction.
    __syncthreads();
#pragma unroll
    for (int h = 0; h < G; ++h) {
        sh.u.red[tg][h][2 * cp] = acc[h][0];
        sh.u.red[tg][h][2 * cp + 1] = acc[h][1];
    }
    __syncthreads();
    const int S = int(p.splits);
    for (int i = tid; i < G * D; i += kThreads) {
        const int h = i / D, dd = i % D;
        float s = 0.0f;
#pragma unroll
        for (int g = 0; g < TG; ++g) s += sh.u.red[g][h][dd];
        const size_t qh = size_t(b) * p.query_heads + size_t(kh) * G + h;
        partial[(qh * S + split) * D + dd] = s + sh.mlo[h][2];
    }
    if (tid < G) {
        const size_t qh = size_t(b) * p.query_heads + size_t(kh) * G + tid;
        // Natural-log max for drop-in statistics: m2 * ln(2).
        stats[qh * S + split] = float2{sh.mlo[tid][0] * 0.69314718055994531f, sh.mlo[tid][1]};
    }
}

__global__ void merge_kernel(uint32_t splits, uint32_t dim, const float* __restrict__ partial,
                             const float2* __restrict__ stats, float* __restrict__ out) {
    const size_t qh = blockIdx.x;
    const int d = threadIdx.x;
    if (d >= int(dim)) return;
    const float2* st = stats + qh * splits;
    float m = -INFINITY;
    for (uint32_t s = 0; s < splits; ++s) m = fmaxf(m, st[s].x);
    float acc = 0.0f, l = 0.0f;
    for (uint32_t s = 0; s < splits; ++s) {
        const float w = st[s].x == -INFINITY ? 0.0f : expf(st[s].x - m);
        l = fmaf(st[s].y, w, l);
        acc = fmaf(partial[(qh * splits + s) * dim + d], w, acc);
    }
    out[qh * dim + d] = acc / l;
}

// Standalone block decode: 192 blocks per workgroup -> FP16 RGBA texels.
struct BlocksShared {
    SmallLuts luts;
    BlockDesc<4> desc[ChunkCap<4>::blocks];
    uint32_t cv[5][kThreads];
};

__global__ __launch_bounds__(kThreads) void decode_blocks_kernel(const uint4* __restrict__ blocks, size_t n,
                                                                 int bx, int by, int ds, int dt,
                                                                 const AkvTables* __restrict__ tab,
                                                                 uint2* __restrict__ out) {
    __shared__ BlocksShared sh;
    constexpr int NB = ChunkCap<4>::blocks;
    const int tid = threadIdx.x;
    const size_t first = size_t(blockIdx.x) * NB;
    const int nblk = int(min(size_t(NB), n - first));
    stage_luts(tab, sh.luts, tid, kThreads);
    __syncthreads();
    if (tid < nblk) decode_header<4>(blocks[first + tid], tab, sh.luts, sh.desc[tid], &sh.cv[0][tid], kThreads);
    __syncthreads();
    const int per = bx * by;
    for (int it = tid; it < nblk * per; it += kThreads) {
        const int blk = it / per, i = it - blk * per;
        const int y = i / bx, x = i - y * bx;
        uint32_t C[4];
        decode_texel<4>(sh.desc[blk], sh.luts, x, y, bx, ds, dt, C);
        out[(first + blk) * per + i] = uint2{pack_fp16_rtz(C[0], C[1]), pack_fp16_rtz(C[2], C[3])};
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

uint32_t magic(uint32_t d) { return (65536u + d - 1) / d; }

int check_common(const AkvAttnParams* p, uint32_t* G) {
    if (!p) return AKV_HIP_ERR_NULL;
    if (p->batch == 0 || p->tokens == 0 || p->kv_heads == 0 || p->query_heads % p->kv_heads) return AKV_HIP_ERR_SHAPE;
    if (p->dim != 64 && p->dim != 128) return AKV_HIP_ERR_SHAPE;
    const uint32_t g = p->query_heads / p->kv_heads;
    if (g != 1 && g != 2 && g != 3 && g != 4 && g != 8) return AKV_HIP_ERR_SHAPE;
    if (p->batch > 65535 || p->kv_heads > 65535) return AKV_HIP_ERR_SHAPE;
    if (p->tile_tokens == 0) return AKV_HIP_ERR_TILE;
    if (p->splits != (p->tokens + p->tile_tokens - 1) / p->tile_tokens) return AKV_HIP_ERR_TILE;
    *G = g;
    return 0;
}

int check_astc(const AkvAttnParams* p) {
    if (p->layout != AKV_LAYOUT_SCALAR && p->layout != AKV_LAYOUT_RGBA) return AKV_HIP_ERR_SHAPE;
    const uint32_t bx = p->block_x, by = p->block_y;
    if (bx < 4 || by < 4 || bx > 12 || by > 12 || bx * by > uint32_t(akv::kMaxTexels)) return AKV_HIP_ERR_FOOTPRINT;
    const uint32_t texcols = p->layout == AKV_LAYOUT_SCALAR ? p->dim : p->dim / 4;
    if (p->atlas_cols != (texcols + bx - 1) / bx) return AKV_HIP_ERR_SHAPE;
    const uint32_t cap = p->layout == AKV_LAYOUT_SCALAR ? ChunkCap<1>::blocks : ChunkCap<4>::blocks;
    if (p->atlas_cols > cap) return AKV_HIP_ERR_SHAPE;
    if (p->tile_tokens % by) return AKV_HIP_ERR_TILE;
    if (uint64_t(p->atlas_rows) * by < p->tokens) return AKV_HIP_ERR_SHAPE;
    return 0;
}

KernelArgs make_args(const AkvAttnParams* p, uint32_t G) {
    KernelArgs a{};
    a.p = *p;
    a.G = G;
    const int bx = int(p->block_x ? p->block_x : 4), by = int(p->block_y ? p->block_y : 4);
    a.ds = (1024 + bx / 2) / (bx - 1);
    a.dt = (1024 + by / 2) / (by - 1);
    a.mag_bx = magic(uint32_t(bx));
    a.mag_by = magic(uint32_t(by));
    a.mag_cols = magic(p->atlas_cols ? p->atlas_cols : 1);
    a.qscale = float(1.4426950408889634 / std::sqrt(double(p->dim)));
    const uint32_t max_tile = uint32_t(kTileElems) / p->dim;
    a.sub_tokens = max_tile / uint32_t(by) * uint32_t(by);
    return a;
}

template <int D, int NCH, bool ASTC, bool DUMP>
hipError_t launch_split_g(const KernelArgs& a, const float* q, const uint16_t* k, const uint4* vblk,
                          const uint16_t* vh, const uint16_t* vs, const uint16_t* vo, const AkvTables* tab,
                          float* partial, float* stats, uint16_t* dump, hipStream_t st) {
    dim3 grid(a.p.splits, a.p.kv_heads, a.p.batch);
    auto* s2 = reinterpret_cast<float2*>(stats);
    switch (a.G) {
#define AKV_CASE(GG)                                                                                      \
    case GG:                                                                                              \
        split_kernel<D, NCH, GG, ASTC, DUMP><<<grid, kThreads, 0, st>>>(a, q, k, vblk, vh, vs, vo, tab,   \
                                                                         partial, s2, dump);              \
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
hipError_t launch_split(const KernelArgs& a, const float* q, const uint16_t* k, const uint4* vblk,
                        const uint16_t* vh, const uint16_t* vs, const uint16_t* vo, const AkvTables* tab,
                        float* partial, float* stats, uint16_t* dump, hipStream_t st) {
    const bool rgba = a.p.layout == AKV_LAYOUT_RGBA;
    if (a.p.dim == 64)
        return rgba || !ASTC ? launch_split_g<64, 4, ASTC, DUMP>(a, q, k, vblk, vh, vs, vo, tab, partial, stats, dump, st)
                             : launch_split_g<64, 1, ASTC, DUMP>(a, q, k, vblk, vh, vs, vo, tab, partial, stats, dump, st);
    return rgba || !ASTC ? launch_split_g<128, 4, ASTC, DUMP>(a, q, k, vblk, vh, vs, vo, tab, partial, stats, dump, st)
                         : launch_split_g<128, 1, ASTC, DUMP>(a, q, k, vblk, vh, vs, vo, tab, partial, stats, dump, st);
}

int as_int(hipError_t e) { return e == hipSuccess ? 0 : int(e); }

}  // namespace
}  // namespace akv_hip

using namespace akv_hip;

extern "C" {

int akv_hip_attention_split(const AkvAttnParams* p, const float* q, const uint16_t* k, const void* v_blocks,
                            const uint16_t* v_scale, const uint16_t* v_offset, float* partial, float* stats,
                            void* stream) {
    uint32_t G = 0;
    if (int rc = check_common(p, &G)) return rc;
    if (int rc = check_astc(p)) return rc;
    if (!q || !k || !v_blocks || !v_scale || !v_offset || !partial || !stats) return AKV_HIP_ERR_NULL;
    const AkvTables* tab = nullptr;
    if (int rc = device_tables(int(p->block_x), int(p->block_y), &tab)) return rc;
    KernelArgs a = make_args(p, G);
    return as_int(launch_split<true, false>(a, q, k, static_cast<const uint4*>(v_blocks), nullptr, v_scale, v_offset,
                                            tab, partial, stats, nullptr, static_cast<hipStream_t>(stream)));
}

int akv_hip_attention_merge(const AkvAttnParams* p, const float* partial, const float* stats, float* out,
                            void* stream) {
    uint32_t G = 0;
    if (int rc = check_common(p, &G)) return rc;
    if (!partial || !stats || !out) return AKV_HIP_ERR_NULL;
    merge_kernel<<<dim3(p->batch * p->query_heads), dim3(p->dim), 0, static_cast<hipStream_t>(stream)>>>(
        p->splits, p->dim, partial, reinterpret_cast<const float2*>(stats), out);
    return as_int(hipGetLastError());
}

int akv_hip_decode_attention(const AkvAttnParams* p, const float* q, const uint16_t* k, const void* v_blocks,
                             const uint16_t* v_scale, const uint16_t* v_offset, float* partial, float* stats,
                             float* out, void* stream) {
    if (!out) return AKV_HIP_ERR_NULL;
    if (int rc = akv_hip_attention_split(p, q, k, v_blocks, v_scale, v_offset, partial, stats, stream)) return rc;
    return akv_hip_attention_merge(p, partial, stats, out, stream);
}

int akv_hip_fp16_attention(const AkvAttnParams* p, const float* q, const uint16_t* k, const uint16_t* v,
                           float* partial, float* stats, float* out, void* stream) {
    uint32_t G = 0;
    if (int rc = check_common(p, &G)) return rc;
    if (!q || !k || !v || !partial || !stats || !out) return AKV_HIP_ERR_NULL;
    KernelArgs a = make_args(p, G);
    hipStream_t st = static_cast<hipStream_t>(stream);
    hipError_t e = launch_split<false, false>(a, q, k, nullptr, v, nullptr, nullptr, nullptr, partial, stats, nullptr, st);
    if (e != hipSuccess) return int(e);
    return akv_hip_attention_merge(p, partial, stats, out, stream);
}

int akv_hip_decode_values(const AkvAttnParams* p, const void* v_blocks, uint16_t* u, void* stream) {
    uint32_t G = 0;
    if (int rc = check_common(p, &G)) return rc;
    if (int rc = check_astc(p)) return rc;
    if (!v_blocks || !u) return AKV_HIP_ERR_NULL;
    const AkvTables* tab = nullptr;
    if (int rc = device_tables(int(p->block_x), int(p->block_y), &tab)) return rc;
    KernelArgs a = make_args(p, G);
    return as_int(launch_split<true, true>(a, nullptr, nullptr, static_cast<const uint4*>(v_blocks), nullptr, nullptr,
                                           nullptr, tab, nullptr, nullptr, u, static_cast<hipStream_t>(stream)));
}

int akv_hip_decode_blocks(const void* blocks, size_t n, unsigned bx, unsigned by, uint16_t* texels, void* stream) {
    if ((!blocks || !texels) && n) return AKV_HIP_ERR_NULL;
    if (bx < 4 || by < 4 || bx > 12 || by > 12 || bx * by > unsigned(akv::kMaxTexels)) return AKV_HIP_ERR_FOOTPRINT;
    if (n == 0) return 0;
    const AkvTables* tab = nullptr;
    if (int rc = device_tables(int(bx), int(by), &tab)) return rc;
    const int ds = int((1024 + bx / 2) / (bx - 1)), dt = int((1024 + by / 2) / (by - 1));
    const size_t groups = (n + ChunkCap<4>::blocks - 1) / ChunkCap<4>::blocks;
    if (groups > 0x7FFFFFFF) return AKV_HIP_ERR_SHAPE;
    decode_blocks_kernel<<<dim3(unsigned(groups)), dim3(kThreads), 0, static_cast<hipStream_t>(stream)>>>(
        static_cast<const uint4*>(blocks), n, int(bx), int(by), ds, dt, tab, reinterpret_cast<uint2*>(texels));
    return as_int(hipGetLastError());
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
