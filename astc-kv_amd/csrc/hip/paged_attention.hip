// Split-K decode attention over a paged, ragged batch for gfx950: K (FP16 or
// 4-bit in groups of 32 channels) and ASTC V live in page pools addressed
// through per-sequence block tables; an optional FP16 V tail holds each
// sequence's tokens past its last full page. One launch per step: the last
// split workgroup of each (sequence, kv head) merges.
//
// The schedule is the contiguous split kernel's (decode_attention.hip): chunks
// of whole block rows, a header stage of one lane per block sorted by
// decode-path class, groups of 16-token tiles on the matrix cores. What
// changes is addressing: every block row, K row and scale/offset is found
// through the split's pages (cached in LDS), chunks and tiles are aligned to
// 16 tokens so that a tile never straddles a page, and tiles past the last
// full page read V from the FP16 tail with scale 1 and offset 0. At head dim
// 128 with a scalar layout the kernel runs three workgroups per CU (PagedCfg).
//
// Reference semantics: metal/attention_gqa_v10.metal:568-674 and :229-253 (as
// the contiguous kernel); 4-bit K as affine_quantize(axis="token", group=32),
// astc_kv/codec.py:218-250. The reference has no paged kernel; its paged
// format is a plan (docs/representation_v0.1.md:47-50, :84-95).
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>

#include "astc_decode_device.h"
#include "astc_format.h"
#include "astc_kv_hip.h"
#include "attention_device.h"
#include "host_common.h"

namespace akv_hip {
namespace {

constexpr int kMaxSplitPages = 64;   // pages one split may touch

struct PagedArgs {
    AkvPagedParams p;
    Footprint fp;
    uint32_t chunk_tokens;             // a multiple of 16 and of block_y
    uint32_t rows_per_page;            // page_tokens / block_y
    uint32_t mag_by, mag_bx, mag_cols, mag_page, mag_rpp;   // ceil(2^24 / divisor)
    float qscale;
};

// Head dim 128, scalar layout: three workgroups per CU rather than two, for
// a kernel that waits on header-stage latency most of its cycles. That fits
// with one tile per group (168 VGPRs) and chunks of at most 192 blocks (52 KB
// of LDS; scalar 6x6 chunks are 176 blocks either way). Ragged 64-sequence
// batch, D128, 4-bit K + scalar 6x6 V at quality 50: 2.02 -> 1.53 ms.
template <int D, int NCH>
struct PagedCfg {
    static constexpr bool kThree = D == 128 && NCH == 1;
    static constexpr int kMaxBlocks = kThree ? 192 : 0;   // 0: Cfg's own
    static constexpr int kWavesPerSimd = D == 64 ? AKV_ASTC_WAVES : kThree ? 3 : 2;
};

template <int D, int NCH>
struct PagedShared {
    AstcShared<D, NCH, false, false, PagedCfg<D, NCH>::kMaxBlocks> a;
    int32_t pages[kMaxSplitPages];     // the split's pages, from its first
};

// V of one texel column group from the FP16 tail, in the texel operand order
// (RGBA: channels 4x .. 4x+3 of column x; scalar: channel x), for the four
// tokens tail rows r[0..3].
template <int D, int NCH>
__device__ inline void tail_texels(const uint16_t* __restrict__ tail, const int (&r)[4], int x, uint2 (&tv)[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        if constexpr (NCH == 4) tv[i] = *reinterpret_cast<const uint2*>(tail + size_t(r[i]) * D + 4 * x);
        else tv[i] = uint2{uint32_t(tail[size_t(r[i]) * D + x]), 0u};
    }
}

template <int D, int NCH, int G, bool KU4>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(PagedCfg<D, NCH>::kWavesPerSimd))) void
paged_attn_kernel(PagedArgs a, const float* __restrict__ q, const void* __restrict__ kpool,
                  const uint16_t* __restrict__ kmeta, const uint4* __restrict__ vpool,
                  const uint16_t* __restrict__ vscale, const uint16_t* __restrict__ voffset,
                  const int32_t* __restrict__ table, const int32_t* __restrict__ lens,
                  const uint16_t* __restrict__ vtail, const AkvTables* __restrict__ tab, float* partial,
                  float2* stats, float* __restrict__ out, uint32_t* arrivals) {
    using C = Cfg<D, NCH, false, PagedCfg<D, NCH>::kMaxBlocks>;
    constexpr int TPG = PagedCfg<D, NCH>::kThree ? 1 : Grp<G, D>::TPG;   // tiles per group
    constexpr int kKEarly = TPG < 2 ? TPG : 2;
    // Per tile and lane: FP16 K, D/32 16-byte row pieces; 4-bit K, D/32 code
    // dwords and D/32 (offset, scale) dwords.
    constexpr int kKWords = KU4 ? D / 16 : 4 * (D / 32);
    __shared__ PagedShared<D, NCH> shp;
    AstcShared<D, NCH, false, false, PagedCfg<D, NCH>::kMaxBlocks>& sh = shp.a;
    const AkvPagedParams& p = a.p;
    const Footprint f = a.fp;
    const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), lane = tid & 63;
    const int n16 = lane & 15, g = lane >> 4;
    // Grid (kv head, sequence, split): workgroups are dispatched to the XCDs
    // round robin in linear order, and with the split slowest every XCD gets
    // an equal share of each split index. (With the split fastest and a
    // power-of-two split count, split s of every sequence lands on XCD s % 8,
    // and in a ragged batch the XCDs holding the late splits of only the
    // long sequences idle while the others work: up to 2x slower.)
    const int kh = blockIdx.x, b = blockIdx.y, split = blockIdx.z;
    // Lengths come from device memory: a length past max_tokens is read as
    // max_tokens (the launched splits cover exactly that many, and the merge
    // counts the splits of the clamped length); a sequence of no tokens gets
    // zeros from its first split and no merge.
    const int len = min(lens[b], int(p.max_tokens));
    const int P = int(p.page_tokens);
    const size_t qh0 = size_t(b) * p.query_heads + size_t(kh) * G;
    if (len <= 0) {
        if (split == 0)
            for (int i = tid; i < G * D; i += kThreads) out[qh0 * D + i] = 0.0f;
        return;
    }
    const int split_begin = split * int(p.tile_tokens);
    if (split_begin >= len) return;   // this sequence has fewer splits (uniform, before any barrier)
    const int split_end = min(split_begin + int(p.tile_tokens), len);
    const int full = vtail ? len - len % P : len;   // tokens whose V is in ASTC pages
    const int page0 = split_begin / P, base_tok = page0 * P;
    const int npages = (split_end - 1) / P - page0 + 1;
    const int CT = int(a.chunk_tokens), by = f.by;
    const int cols = int(p.atlas_cols), rpp = int(a.rows_per_page), Hkv = int(p.kv_heads);
    const int32_t* seq_table = table + size_t(b) * p.max_pages + page0;
    const uint16_t* tail = vtail ? vtail + (size_t(b) * Hkv + kh) * P * D : nullptr;
    // Page ids come from device memory too: an id outside [0, num_pages) is
    // read as page 0 (nothing outside the pools is touched) and poisons the
    // sequence, whose output becomes NaN.
    auto page_id = [&](int32_t id) { return uint32_t(id) < p.num_pages ? int(id) : 0; };

    // Page of a token: (page id, token within the page); t_abs - base_tok < tile + page.
    auto page_of = [&](int t_abs, int& pid, int& pos) {
        const int rel = t_abs - base_tok;
        const int pg = int(fdiv(uint32_t(rel), a.mag_page));
        pid = shp.pages[pg];
        pos = rel - pg * P;
    };
    auto chunk_astc = [&](int c0) { return max(0, min(full - c0, min(CT, split_end - c0))); };
    auto chunk_blocks = [&](int c0) { return (chunk_astc(c0) + by - 1) / by * cols; };
    // This lane's block of the chunk at c0 (nblk blocks); the first chunk reads
    // its page ids from the block table, later ones from LDS.
    auto load_blk = [&](int c0, int nblk, bool from_table) -> uint4 {
        if (tid >= nblk) return uint4{0, 0, 0, 0};
        // Recomputed per call: hoisted out of the chunk loop, the lane's
        // 64-bit column address stayed live through the header stage and was
        // spilled there.
        int lt = tid;
        asm volatile("" : "+v"(lt));
        const int r = int(fdiv(uint32_t(lt), a.mag_cols)), col = lt - r * cols;
        // (c0 - base_tok) / by can exceed the 8-bit quotients fdiv is exact
        // for; c0 and base_tok are uniform, so this is one scalar division.
        const int grow = (c0 - base_tok) / by + r;
        const int pg = int(fdiv(uint32_t(grow), a.mag_rpp)), prow = grow - pg * rpp;
        const int pid = from_table ? page_id(seq_table[pg]) : shp.pages[pg];
        return vpool[((size_t(pid) * Hkv + kh) * rpp + prow) * cols + col];
    };

    // Prologue: the decode tables and Q (from L2), the split's page ids and
    // the first chunk's blocks, all issued before the first wait.
    TableStage<kThreads> tables;
    tables.load(tab, tid);
    QStage<D, G> qst;
    if (wave == 0) qst.load(q + (size_t(b) * p.query_heads + size_t(kh) * G) * D);
    uint4 raw = load_blk(split_begin, chunk_blocks(split_begin), true);
    int bad_page = 0;
    if (tid < npages) {
        const int32_t id = seq_table[tid];
        bad_page = uint32_t(id) >= p.num_pages;
        shp.pages[tid] = page_id(id);
    }
    tables.store(sh.tabs, tid);
    if (wave == 0) qst.store(a.qscale, &sh.q[0][0]);
    if (tid < kPathKeys) sh.key_count[tid] = 0;

    // (block column | x in block << 16, one register each).
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

    // K rows of the 16-token tile at chunk token t0 of the chunk at c0 (rows
    // past the split read its last token; their scores are never used).
    uint32_t kw[TPG * kKWords];
    auto load_k = [&](uint32_t* r, int c0, int t0) {
        int pid, pos;
        page_of(min(c0 + t0 + n16, split_end - 1), pid, pos);
        const size_t row = (size_t(pid) * Hkv + kh) * P + pos;
        if constexpr (KU4) {
            const uint8_t* codes = static_cast<const uint8_t*>(kpool) + row * (D / 2);
#pragma unroll
            for (int L = 0; L < D / 32; ++L) {
                r[L] = *reinterpret_cast<const uint32_t*>(codes + 16 * L + 4 * g);
                r[D / 32 + L] = *reinterpret_cast<const uint32_t*>(kmeta + (row * (D / 32) + L) * 2);
            }
        } else {
            const uint16_t* k16 = static_cast<const uint16_t*>(kpool) + row * D;
#pragma unroll
            for (int L = 0; L < D / 32; ++L) {
                const uint4 v = *reinterpret_cast<const uint4*>(k16 + 32 * L + 8 * g);
                r[4 * L] = v.x;
                r[4 * L + 1] = v.y;
                r[4 * L + 2] = v.z;
                r[4 * L + 3] = v.w;
            }
        }
    };

    const bool poisoned = __syncthreads_or(bad_page);   // pages, decode tables and Q operands
    for (int c0 = split_begin; c0 < split_end; c0 += CT) {
        const int ntok = min(CT, split_end - c0);
        const int ntiles = (ntok + 15) >> 4;
        // Tiles per group: TPG, or as many as spread a chunk of less than a
        // round (TPG tiles for every wave) over all four waves.
        const int gt = min(TPG, (ntiles + kWaves - 1) / kWaves);
        const int nastc = chunk_astc(c0);
        const int nblk = chunk_blocks(c0);
        // 1. Loads. Only the blocks cross chunks (requested one chunk ahead:
        // the header stage needs them first). The rest is requested here and
        // first used after the header stage, which covers its latency: the
        // blocks' partition-pattern words, the per-token scale/offset (two
        // tokens per lane; every token of the split has a page, so a clamped
        // index reads in bounds), the first K tiles of this wave's first
        // group. Memory waits count loads in issue order, so they are issued
        // in the order of first use.
        const uint4 raw_now = raw;
        const uint4 pat = partition_words(raw_now, tab);
        static_assert(C::kMaxTok <= 2 * kThreads, "two scale/offset tokens per lane");
        uint32_t sc[2], of[2];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            int pid, pos;
            page_of(c0 + min(tid + i * kThreads, ntok - 1), pid, pos);
            const size_t at = (size_t(pid) * Hkv + kh) * P + pos;
            sc[i] = vscale[at];
            of[i] = voffset[at];
        }
        if (c0 + CT < split_end) raw = load_blk(c0 + CT, chunk_blocks(c0 + CT), false);
#pragma unroll
        for (int t = 0; t < kKEarly; ++t)
            if (t < gt) load_k(kw + t * kKWords, c0, 16 * (gt * wave + t));
        // 2. Block headers (the blocks of the chunk's ASTC tokens), sorted by
        // decode-path class.
        int key = 0, rank = 0;
        if (tid < nblk) {
            key = block_path_key(raw_now);
            stash_block(sh.u.h.desc[tid], raw_now);
            rank = int(atomicAdd(&sh.key_count[key], 1u));
        }
#pragma unroll
        for (int i = 0; i < 2; ++i)
            if (tid + i * kThreads < C::kMaxTok)
                sh.tokrow[tid + i * kThreads] =
                    token_row_entry(tid + i * kThreads, max(nastc, 1), a.mag_by, f, uint32_t(cols));
        __syncthreads();   // class counts complete
        static_assert(kPathKeys == 64, "one class per lane");
        place_by_class(sh.key_count, sh.order, key, rank, tid < nblk, tid);
        __syncthreads();   // sorted order complete (and every count read)
        if (wave == 0) sh.key_count[lane] = 0;   // for the next chunk (two barriers away)
        // Each lane's own block's partition words (a field the header stage
        // does not touch), and the per-token scale | offset << 16 (tail
        // tokens: fp16 1.0 and 0; zero past the chunk, up to the tile edge),
        // written first so that nothing of them stays in registers through
        // the header stage.
        if (tid < nblk) {
            const uint4 w = block_part_words(raw_now, pat);
            uint32_t* part = sh.u.h.desc[tid].part;   // 4-byte aligned
            part[0] = w.x;
            part[1] = w.y;
            part[2] = w.z;
            part[3] = w.w;
        }
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int t = tid + i * kThreads;
            if (t < 16 * ntiles) sh.so[t] = t >= ntok ? 0u : c0 + t < full ? sc[i] | (of[i] << 16) : 0x3C00u;
        }
        if (tid < nblk) {
            const int bi = sh.order[tid];
            decode_header<NCH, false, false, D == 128 && NCH == 1, true>(sh.tabs, sh.u.h.desc[bi], sh.u.h.cv[tid]);
        }
        __syncthreads();
        // 3. Tile groups; tiles at or past `full` read V from the FP16 tail.
#pragma unroll
        for (int t = kKEarly; t < TPG; ++t)
            if (t < gt) load_k(kw + t * kKWords, c0, 16 * (gt * wave + t));
#pragma unroll 1
        for (int tb0 = 16 * gt * wave; tb0 < ntok; tb0 += 16 * gt * kWaves) {
            const int ng = min(gt, (ntok - tb0 + 15) >> 4);
            uint32_t rows[4];
            int trow[4];
            bool in_tail = false;
            auto vtile = [&](int t, int kc, half4* va) {
                if (kc == 0) {
                    if (t == 0) {   // S is done with this group's K rows
                        const int nb0 = tb0 + 16 * gt * kWaves;
#pragma unroll
                        for (int tt = 0; tt < TPG; ++tt)
                            if (tt < gt) load_k(kw + tt * kKWords, c0, nb0 + 16 * tt);
                    }
                    in_tail = c0 + tb0 + 16 * t >= full;
                    if (in_tail) {
#pragma unroll
                        for (int i = 0; i < 4; ++i) trow[i] = min(c0 + tb0 + 16 * t + 4 * g + i, split_end - 1) - full;
                    } else {
                        tile_rows(sh.tokrow, tb0 + 16 * t, g, rows);
                    }
                }
                uint2 tv[4];
                if (in_tail) tail_texels<D, NCH>(tail, trow, n16 + 16 * kc, tv);
                else column_texels<NCH, false>(sh.u.h.desc, sh.tabs, f, rows, colpk[kc] & 0xFFFF, colpk[kc] >> 16, nullptr, tv);
                texel_operands<NCH>(tv, va);
            };
            if constexpr (KU4)
                attend_group<D, G, true, C::kRowBlocksPerGroup, TPG>(U4KOperands<D>{kw}, &sh.q[0][0], ng, tb0, ntok,
                                                                 sh.so, C::kMaxTok, st, vtile);
            else
                attend_group<D, G, true, C::kRowBlocksPerGroup, TPG>(
                    Fp16KOperands<D>{reinterpret_cast<const uint4*>(kw)}, &sh.q[0][0], ng, tb0, ntok, sh.so,
                    C::kMaxTok, st, vtile);
        }
        __syncthreads();   // descriptors and so are rewritten by the next chunk
    }
    const int S = int(p.splits), Sb = (len + int(p.tile_tokens) - 1) / int(p.tile_tokens);
    if (poisoned) st.l = __builtin_nanf("");   // a NaN sum of weights reaches every merge of this sequence
    combine_waves<D, NCH, G>(sh.u.comb, sh.ws, st, partial, stats, qh0, S, split);
    merge_if_last<D, G>(arrivals + size_t(b) * Hkv + kh, partial, stats, out, qh0, Sb, S, sh.ws, sh.u.comb,
                        kWaves * D * kMaxG);
}

// --- append and page commit ----------------------------------------------------

// fp16 bits of the largest float16 <= x and of the smallest float16 >= x (x
// finite): round to nearest even, then one step toward -inf / +inf where that
// rounded past x, as np.nextafter on float16 (from +-0 the step is to -+2^-24;
// from -2^-24 up it is to -0).
__device__ inline uint16_t fp16_floor_bits(float x) {
    const _Float16 h = _Float16(x);
    uint16_t b = __builtin_bit_cast(uint16_t, h);
    if (float(h) > x) b = (b & 0x7FFF) == 0 ? uint16_t(0x8001) : (b & 0x8000) ? uint16_t(b + 1) : uint16_t(b - 1);
    return b;
}

__device__ inline uint16_t fp16_ceil_bits(float x) {
    const _Float16 h = _Float16(x);
    uint16_t b = __builtin_bit_cast(uint16_t, h);
    if (float(h) < x) b = (b & 0x7FFF) == 0 ? uint16_t(0x0001) : (b & 0x8000) ? uint16_t(b - 1) : uint16_t(b + 1);
    return b;
}

__device__ inline float fp16_value(uint16_t b) { return float(__builtin_bit_cast(_Float16, b)); }

// One new token per sequence into the pools, at row seq_len % P of page
// block_table[b][seq_len / P]: K as fp16, or as 4-bit codes with the fp16
// (offset, scale) of its group of 32 channels (affine_quantize(axis="token",
// group=32), codec.py:218-250, all in fp32: o = fp16_floor(min), s =
// fp16_ceil(max((max - o) / 15, 2^-24)), code = clip(rint((x - o) / s), 0, 15),
// two codes per byte, low nibble = even channel), and V as fp16 into the tail
// at the same row. One workgroup per (kv head, sequence), one lane per
// channel (a group of 32 channels is half a wave). A sequence whose slot has
// no valid page is left unchanged.
template <int D, bool KU4>
__global__ __launch_bounds__(128) void paged_append_kernel(AkvPagedParams p, const float* __restrict__ knew,
                                                           const float* __restrict__ vnew, void* __restrict__ kpool,
                                                           uint16_t* __restrict__ kmeta,
                                                           const int32_t* __restrict__ table,
                                                           const int32_t* __restrict__ lens,
                                                           uint16_t* __restrict__ vtail) {
    const int c = int(threadIdx.x), kh = int(blockIdx.x), b = int(blockIdx.y);
    const int Hkv = int(p.kv_heads), P = int(p.page_tokens);
    const int n = lens[b];
    if (n < 0 || n / P >= int(p.max_pages)) return;   // uniform over the workgroup
    const int pid = table[size_t(b) * p.max_pages + n / P];
    if (pid < 0 || pid >= int(p.num_pages)) return;
    const int pos = n % P;
    const size_t src = (size_t(b) * Hkv + kh) * D + c;
    const size_t row = (size_t(pid) * Hkv + kh) * P + pos;
    const float x = knew[src];
    if constexpr (!KU4) {
        static_cast<uint16_t*>(kpool)[row * D + c] = __builtin_bit_cast(uint16_t, _Float16(x));
    } else {
        float mn = x, mx = x;
#pragma unroll
        for (int o = 16; o >= 1; o >>= 1) {
            mn = fminf(mn, __shfl_xor(mn, o, 32));
            mx = fmaxf(mx, __shfl_xor(mx, o, 32));
        }
        const uint16_t ob = fp16_floor_bits(mn);
        const float o32 = fp16_value(ob);
        const uint16_t sb = fp16_ceil_bits(fmaxf((mx - o32) / 15.0f, 0x1p-24f));
        const float s32 = fp16_value(sb);
        const int code = int(fminf(fmaxf(rintf((x - o32) / s32), 0.0f), 15.0f));
        const int odd = __shfl_xor(code, 1, 32);
        if ((c & 1) == 0) static_cast<uint8_t*>(kpool)[row * (D / 2) + c / 2] = uint8_t(code | (odd << 4));
        if ((c & 31) == 0) {
            kmeta[(row * (D / 32) + c / 32) * 2] = ob;
            kmeta[(row * (D / 32) + c / 32) * 2 + 1] = sb;
        }
    }
    vtail[((size_t(b) * Hkv + kh) * P + pos) * D + c] = __builtin_bit_cast(uint16_t, _Float16(vnew[src]));
}

// Encoded V pages into their pool slots: staging page i (blocks
// [n][kv_heads][P/block_y][atlas_cols], scale and offset fp16 [n][kv_heads][P])
// -> pool page ids[i], as 16-byte words. Out-of-range ids are skipped.
__global__ __launch_bounds__(kThreads) void paged_commit_kernel(const int32_t* __restrict__ ids, uint32_t num_pages,
                                                                const uint4* __restrict__ blocks,
                                                                const uint4* __restrict__ scale,
                                                                const uint4* __restrict__ offset, uint32_t block_words,
                                                                uint32_t meta_words, uint4* __restrict__ vblocks,
                                                                uint4* __restrict__ vscale,
                                                                uint4* __restrict__ voffset) {
    const uint32_t i = blockIdx.y;
    const int pid = ids[i];
    if (pid < 0 || uint32_t(pid) >= num_pages) return;
    const uint32_t total = block_words + 2 * meta_words;
    for (uint32_t w = blockIdx.x * kThreads + threadIdx.x; w < total; w += gridDim.x * kThreads) {
        if (w < block_words) {
            vblocks[size_t(pid) * block_words + w] = blocks[size_t(i) * block_words + w];
        } else if (w < block_words + meta_words) {
            const uint32_t m = w - block_words;
            vscale[size_t(pid) * meta_words + m] = scale[size_t(i) * meta_words + m];
        } else {
            const uint32_t m = w - block_words - meta_words;
            voffset[size_t(pid) * meta_words + m] = offset[size_t(i) * meta_words + m];
        }
    }
}

// --- host ---------------------------------------------------------------------

// The pools' geometry (what the append and commit entry points need too).
int check_pool(const AkvPagedParams* p) {
    if (!p) return AKV_HIP_ERR_NULL;
    if (p->batch == 0 || p->kv_heads == 0 || (p->dim != 64 && p->dim != 128)) return AKV_HIP_ERR_SHAPE;
    if (p->batch > 65535 || p->kv_heads > 65535 || p->num_pages == 0 || p->max_pages == 0) return AKV_HIP_ERR_SHAPE;
    if (p->k_format != AKV_K_FP16 && p->k_format != AKV_K_U4G32) return AKV_HIP_ERR_SHAPE;
    if (p->layout != AKV_LAYOUT_SCALAR && p->layout != AKV_LAYOUT_RGBA) return AKV_HIP_ERR_SHAPE;
    const uint32_t bx = p->block_x, by = p->block_y;
    if (bx < 4 || by < 4 || bx > 12 || by > 12 || bx * by > uint32_t(akv::kMaxTexels)) return AKV_HIP_ERR_FOOTPRINT;
    const uint32_t texcols = p->layout == AKV_LAYOUT_SCALAR ? p->dim : p->dim / 4;
    if (p->atlas_cols != (texcols + bx - 1) / bx) return AKV_HIP_ERR_SHAPE;
    const uint32_t P = p->page_tokens;
    if (P == 0 || P % 16 || P % by) return AKV_HIP_ERR_SHAPE;
    // The smallest legal tile, lcm(16, block_y) tokens, must pass check_paged's
    // 24-bit bound on split-relative offsets (P <= 4080 for block_y = 4 or 8).
    uint32_t step = 16;
    while (step % by) step += 16;
    if (uint64_t(step + P) * P >= (1u << 24)) return AKV_HIP_ERR_SHAPE;
    return 0;
}

int check_paged(const AkvPagedParams* p, uint32_t* G) {
    if (int rc = check_pool(p)) return rc;
    if (p->max_tokens == 0 || p->query_heads % p->kv_heads) return AKV_HIP_ERR_SHAPE;
    const uint32_t g = p->query_heads / p->kv_heads;
    if (g != 1 && g != 2 && g != 3 && g != 4 && g != 8) return AKV_HIP_ERR_SHAPE;
    const uint32_t by = p->block_y, P = p->page_tokens;
    if (uint64_t(p->max_pages) * P < p->max_tokens) return AKV_HIP_ERR_SHAPE;
    const uint32_t T = p->tile_tokens;
    if (T == 0 || T % 16 || T % by) return AKV_HIP_ERR_TILE;
    if (p->splits != (p->max_tokens + T - 1) / T || p->splits > 65535) return AKV_HIP_ERR_TILE;   // grid z
    // Pages a split touches; split-relative offsets times the divisors fit 24 bits.
    if ((T + P - 1) / P + 1 > uint32_t(kMaxSplitPages) || uint64_t(T + P) * P >= (1u << 24))
        return AKV_HIP_ERR_TILE;
    *G = g;
    return 0;
}

// Chunk: the most 16-token-aligned whole block rows (a multiple of
// lcm(16, block_y) tokens) whose blocks fit the header stage.
template <int D, int NCH>
int plan_paged(const AkvPagedParams* p, PagedArgs* a) {
    using C = Cfg<D, NCH, false, PagedCfg<D, NCH>::kMaxBlocks>;
    const uint32_t by = p->block_y;
    uint32_t step = 16;
    while (step % by) step += 16;
    uint32_t rows = uint32_t(C::kMaxBlocks) / p->atlas_cols;
    uint32_t tokens = rows * by;
    if (tokens > uint32_t(C::kMaxTok)) tokens = uint32_t(C::kMaxTok);
    tokens -= tokens % step;
    if (tokens == 0) return AKV_HIP_ERR_SHAPE;
    a->chunk_tokens = tokens < p->tile_tokens ? tokens : p->tile_tokens;
    return 0;
}

int make_paged_args(const AkvPagedParams* p, PagedArgs* a) {
    *a = PagedArgs{};
    a->p = *p;
    a->fp = footprint(p->block_x, p->block_y);
    a->rows_per_page = p->page_tokens / p->block_y;
    a->mag_by = magic(p->block_y);
    a->mag_bx = magic(p->block_x);
    a->mag_cols = magic(p->atlas_cols);
    a->mag_page = magic(p->page_tokens);
    a->mag_rpp = magic(a->rows_per_page);
    a->qscale = float(1.4426950408889634 / std::sqrt(double(p->dim)));
    const bool scalar = p->layout == AKV_LAYOUT_SCALAR;
    if (p->dim == 64) return scalar ? plan_paged<64, 1>(p, a) : plan_paged<64, 4>(p, a);
    return scalar ? plan_paged<128, 1>(p, a) : plan_paged<128, 4>(p, a);
}

struct PagedPtrs {
    const float* q;
    const void* k;
    const uint16_t* kmeta;
    const uint4* v;
    const uint16_t* vs;
    const uint16_t* vo;
    const int32_t* table;
    const int32_t* lens;
    const uint16_t* tail;
    const AkvTables* tab;
    float* partial;
    float2* stats;
    float* out;
    uint32_t* arrivals;
};

template <int D, int NCH, bool KU4>
hipError_t launch_paged_g(const PagedArgs& a, uint32_t G, const PagedPtrs& x, hipStream_t st) {
    dim3 grid(a.p.kv_heads, a.p.batch, a.p.splits);
    switch (G) {
#define AKV_CASE(GG)                                                                                          \
    case GG:                                                                                                  \
        paged_attn_kernel<D, NCH, GG, KU4><<<grid, kThreads, 0, st>>>(a, x.q, x.k, x.kmeta, x.v, x.vs, x.vo,  \
                                                                      x.table, x.lens, x.tail, x.tab,        \
                                                                      x.partial, x.stats, x.out, x.arrivals); \
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

template <bool KU4>
hipError_t launch_paged(const PagedArgs& a, uint32_t G, const PagedPtrs& x, hipStream_t st) {
    const bool scalar = a.p.layout == AKV_LAYOUT_SCALAR;
    if (a.p.dim == 64)
        return scalar ? launch_paged_g<64, 1, KU4>(a, G, x, st) : launch_paged_g<64, 4, KU4>(a, G, x, st);
    return scalar ? launch_paged_g<128, 1, KU4>(a, G, x, st) : launch_paged_g<128, 4, KU4>(a, G, x, st);
}

}  // namespace
}  // namespace akv_hip

using namespace akv_hip;

extern "C" {

int akv_hip_paged_decode_attention(const AkvPagedParams* p, const float* q, const void* k_pages,
                                   const uint16_t* k_meta, const void* v_blocks, const uint16_t* v_scale,
                                   const uint16_t* v_offset, const int32_t* block_table, const int32_t* seq_lens,
                                   const uint16_t* v_tail, float* partial, float* stats, float* out,
                                   uint32_t* arrivals, void* stream) {
    uint32_t G = 0;
    if (int rc = check_paged(p, &G)) return rc;
    if (!q || !k_pages || !v_blocks || !v_scale || !v_offset || !block_table || !seq_lens || !partial || !stats ||
        !out || !arrivals || (p->k_format == AKV_K_U4G32 && !k_meta))
        return AKV_HIP_ERR_NULL;
    if (!aligned16(q) || !aligned16(k_pages) || !aligned16(v_blocks) || (v_tail && !aligned16(v_tail)))
        return AKV_HIP_ERR_ALIGN;
    const AkvTables* tab = nullptr;
    if (int rc = device_tables(int(p->block_x), int(p->block_y), &tab)) return rc;
    PagedArgs a;
    if (int rc = make_paged_args(p, &a)) return rc;
    const PagedPtrs x{q, k_pages, k_meta, static_cast<const uint4*>(v_blocks), v_scale, v_offset, block_table,
                      seq_lens, v_tail, tab, partial, reinterpret_cast<float2*>(stats), out, arrivals};
    hipStream_t st = static_cast<hipStream_t>(stream);
    return as_int(p->k_format == AKV_K_U4G32 ? launch_paged<true>(a, G, x, st) : launch_paged<false>(a, G, x, st));
}

int akv_hip_paged_append(const AkvPagedParams* p, const float* k_new, const float* v_new, void* k_pages,
                         uint16_t* k_meta, const int32_t* block_table, const int32_t* seq_lens, uint16_t* v_tail,
                         void* stream) {
    if (int rc = check_pool(p)) return rc;
    const bool u4 = p->k_format == AKV_K_U4G32;
    if (!k_new || !v_new || !k_pages || !block_table || !seq_lens || !v_tail || (u4 && !k_meta))
        return AKV_HIP_ERR_NULL;
    const dim3 grid(p->kv_heads, p->batch), block(p->dim);
    hipStream_t st = static_cast<hipStream_t>(stream);
    void* kp = k_pages;
    if (p->dim == 64) {
        if (u4) paged_append_kernel<64, true><<<grid, block, 0, st>>>(*p, k_new, v_new, kp, k_meta, block_table, seq_lens, v_tail);
        else paged_append_kernel<64, false><<<grid, block, 0, st>>>(*p, k_new, v_new, kp, k_meta, block_table, seq_lens, v_tail);
    } else {
        if (u4) paged_append_kernel<128, true><<<grid, block, 0, st>>>(*p, k_new, v_new, kp, k_meta, block_table, seq_lens, v_tail);
        else paged_append_kernel<128, false><<<grid, block, 0, st>>>(*p, k_new, v_new, kp, k_meta, block_table, seq_lens, v_tail);
    }
    return as_int(hipGetLastError());
}

int akv_hip_paged_commit_pages(const AkvPagedParams* p, uint32_t n, const int32_t* page_ids, const void* blocks,
                               const uint16_t* scale, const uint16_t* offset, void* v_blocks, uint16_t* v_scale,
                               uint16_t* v_offset, void* stream) {
    if (int rc = check_pool(p)) return rc;
    if (n == 0) return 0;
    if (n > 65535) return AKV_HIP_ERR_SHAPE;
    if (!page_ids || !blocks || !scale || !offset || !v_blocks || !v_scale || !v_offset) return AKV_HIP_ERR_NULL;
    if (!aligned16(blocks) || !aligned16(scale) || !aligned16(offset) || !aligned16(v_blocks) ||
        !aligned16(v_scale) || !aligned16(v_offset))
        return AKV_HIP_ERR_ALIGN;
    const uint64_t bw = uint64_t(p->kv_heads) * (p->page_tokens / p->block_y) * p->atlas_cols;
    const uint64_t mw = uint64_t(p->kv_heads) * p->page_tokens / 8;   // fp16 x P, P a multiple of 16
    if (bw + 2 * mw > 0xFFFFFFFFull) return AKV_HIP_ERR_SHAPE;
    const uint32_t total = uint32_t(bw + 2 * mw);
    const dim3 grid(std::min<uint32_t>((total + kThreads - 1) / kThreads, 64u), n);
    paged_commit_kernel<<<grid, kThreads, 0, static_cast<hipStream_t>(stream)>>>(
        page_ids, p->num_pages, static_cast<const uint4*>(blocks), reinterpret_cast<const uint4*>(scale),
        reinterpret_cast<const uint4*>(offset), uint32_t(bw), uint32_t(mw), static_cast<uint4*>(v_blocks),
        reinterpret_cast<uint4*>(v_scale), reinterpret_cast<uint4*>(v_offset));
    return as_int(hipGetLastError());
}

int akv_hip_paged_task_tokens(const AkvPagedParams* p) {
    uint32_t G = 0;
    if (int rc = check_paged(p, &G)) return rc;
    PagedArgs a;
    if (int rc = make_paged_args(p, &a)) return rc;
    return int(a.chunk_tokens);
}

}  // extern "C"
