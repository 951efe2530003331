/*
 * astc_kv_hip.h — gfx950 decode-attention C-ABI (libastckv_hip.so).
 *
 * The reference has no library boundary for its GPU path: its host program
 * (metal/probe_gqa_v10.mm) encodes Metal dispatches of the kernels in
 * metal/attention_gqa_v10.metal with a 60-byte Params block
 * (probe_gqa_v10.mm:20-25, attention_gqa_v10.metal:15-31) and buffer slots
 * 0-10 (attention_gqa_v10.metal:101-115). These entry points replace those
 * dispatches:
 *   akv_hip_decode_attention  split (attention_split_gqa3, :568-674) + merge
 *                             (attention_merge, :229-253), ASTC V
 *   akv_hip_decode_attention_fused  the same in one launch (merge by the
 *                             last split workgroup; caller-owned counters)
 *   akv_hip_attention_split   the split pass alone
 *   akv_hip_attention_merge   the merge pass alone
 *   akv_hip_fp16_attention    the FP16 K/V control (fp16_buffer variant,
 *                             probe_gqa_v10.mm:569, :682)
 *   akv_hip_decode_values     correctness readback of normalised V through the
 *                             attention kernel's own decode stage
 *                             (decode_compact_texture, :273-290)
 *   akv_hip_decode_blocks     standalone block decode to FP16 RGBA texels
 *                             (decode_texture, :257-269)
 *
 * Conventions: every pointer is a device pointer owned by the caller; q, k, v
 * and the V blocks (and the paged pools) are 16-byte aligned; `stream`
 * is a hipStream_t (NULL = default stream); calls are stream-ordered and never
 * synchronise the host, except the first call for a footprint on a device,
 * which uploads that footprint's decode tables (a blocking copy). Return 0 on
 * success, a negative AKV_HIP_* code for rejected arguments (nothing is
 * launched), or a positive hipError_t.
 *
 * Layouts (one decode step, one query token per sequence):
 *   q        float32 [batch][query_heads][dim]
 *   k        fp16    [batch][kv_heads][tokens][dim]
 *   v_blocks 16-byte ASTC blocks [batch][kv_heads][atlas_rows][atlas_cols]:
 *            block row r holds tokens r*block_y .. r*block_y+block_y-1; the
 *            scalar layout puts channel c at texel x=c, the rgba layout puts
 *            channels 4x..4x+3 in the RGBA of texel x
 *   v_scale, v_offset  fp16 [batch][kv_heads][tokens]: V = u*scale + offset
 *   v (FP16 control)   fp16 [batch][kv_heads][tokens][dim], restored values
 *   partial  float32 [batch][query_heads][splits][dim] (unnormalised)
 *   stats    float32 [batch][query_heads][splits][2] = (max logit, sum of
 *            exp(logit - max)), natural-log units as in the reference
 *   out      float32 [batch][query_heads][dim]
 * query head h uses kv head h / (query_heads / kv_heads).
 */
#ifndef ASTC_KV_HIP_H
#define ASTC_KV_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    AKV_HIP_ERR_NULL = -1,        /* a required pointer is NULL */
    AKV_HIP_ERR_SHAPE = -2,       /* unsupported or inconsistent shape */
    AKV_HIP_ERR_FOOTPRINT = -3,   /* unsupported ASTC footprint */
    AKV_HIP_ERR_TILE = -4,        /* tile_tokens/splits inconsistent */
    AKV_HIP_ERR_ALIGN = -5,       /* q, k, v or the V blocks not 16-byte aligned */
    AKV_HIP_ERR_SCRATCH = -6      /* beyond the static scratch of the no-allocation entry point */
};

enum { AKV_LAYOUT_SCALAR = 0, AKV_LAYOUT_RGBA = 1 };

/* Mirrors the reference Params (tokens, query_heads, kv_heads, dim,
   page_tokens, tile_tokens, splits, components<->layout, width/height<->
   atlas_cols/atlas_rows) plus the batch and the footprint. */
typedef struct AkvAttnParams {
    uint32_t batch;
    uint32_t tokens;        /* T: keys per sequence */
    uint32_t query_heads;
    uint32_t kv_heads;
    uint32_t dim;           /* 64 or 128 */
    uint32_t page_tokens;   /* atlas padding unit (informational) */
    uint32_t tile_tokens;   /* tokens per split, any positive count as in the reference
                               (probe_gqa_v10.mm:466; splits need not start on a block row,
                               a shared row is decoded by both) */
    uint32_t splits;        /* ceil(tokens / tile_tokens) */
    uint32_t layout;        /* AKV_LAYOUT_SCALAR or AKV_LAYOUT_RGBA */
    uint32_t block_x;
    uint32_t block_y;
    uint32_t atlas_rows;    /* block rows per (sequence, kv head), >= ceil(T/block_y) */
    uint32_t atlas_cols;    /* blocks per row = ceil(texel columns / block_x) */
} AkvAttnParams;

int akv_hip_decode_attention(const AkvAttnParams* p, const float* q, const uint16_t* k, const void* v_blocks,
                             const uint16_t* v_scale, const uint16_t* v_offset, float* partial, float* stats,
                             float* out, void* stream);

/* As akv_hip_decode_attention in one launch: the last split workgroup of each
   (sequence, kv head) to finish merges that kv head's query heads (no second
   pass; results equal the merge pass up to summation order). `arrivals`:
   caller workspace of batch * kv_heads uint32 counters, zero before the first
   call; every call leaves them zero. Concurrent calls must not share it. No
   counterpart in the reference, whose merge is always a second dispatch
   (probe_gqa_v10.mm:648-681). */
int akv_hip_decode_attention_fused(const AkvAttnParams* p, const float* q, const uint16_t* k, const void* v_blocks,
                                   const uint16_t* v_scale, const uint16_t* v_offset, float* partial, float* stats,
                                   float* out, uint32_t* arrivals, void* stream);

/* As akv_hip_decode_attention_fused, allocating nothing. No counterpart in
   the reference; for callers that cannot allocate device memory (code under
   HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).
   The split states, arrival counters and decode tables live in a static
   device array of the library, 8.5 MiB per GPU, held until the process ends:
   limits batch * query_heads * splits * (dim + 2) * 4 bytes <= 8 MiB,
   batch * kv_heads <= 65536 and at most 4 footprints per device (else
   AKV_HIP_ERR_SCRATCH, nothing launched). The first call on a device clears
   the counters with a fill kernel on `stream`; the first call per footprint
   and device copies that footprint's decode tables (blocking): make those
   first calls outside graph capture. Every call leaves the counters zero.
   All calls on one GPU share the array: calls that overlap in time on one
   GPU (concurrent streams, threads) race. */
int akv_hip_decode_attention_noalloc(const AkvAttnParams* p, const float* q, const uint16_t* k, const void* v_blocks,
                                     const uint16_t* v_scale, const uint16_t* v_offset, float* out, void* stream);

int akv_hip_attention_split(const AkvAttnParams* p, const float* q, const uint16_t* k, const void* v_blocks,
                            const uint16_t* v_scale, const uint16_t* v_offset, float* partial, float* stats,
                            void* stream);

int akv_hip_attention_merge(const AkvAttnParams* p, const float* partial, const float* stats, float* out,
                            void* stream);

/* FP16 control: same schedule, V read from restored fp16 values. Uses
   batch, tokens, query_heads, kv_heads, dim, tile_tokens and splits only. */
int akv_hip_fp16_attention(const AkvAttnParams* p, const float* q, const uint16_t* k, const uint16_t* v,
                           float* partial, float* stats, float* out, void* stream);

/* The FP16 control with the merge in the split launch, as
   akv_hip_decode_attention_fused (arrivals may be NULL: two launches). */
int akv_hip_fp16_attention_fused(const AkvAttnParams* p, const float* q, const uint16_t* k, const uint16_t* v,
                                 float* partial, float* stats, float* out, uint32_t* arrivals, void* stream);

/* Normalised V exactly as the attention kernel decodes it: FP16 bit patterns
   [batch][kv_heads][tokens][dim]. */
int akv_hip_decode_values(const AkvAttnParams* p, const void* v_blocks, uint16_t* u, void* stream);

/* n blocks of a bx x by footprint -> FP16 RGBA bit patterns [n][by][bx][4]. */
int akv_hip_decode_blocks(const void* blocks, size_t n, unsigned bx, unsigned by, uint16_t* texels,
                          void* stream);

/* Host-side planning query, no GPU work: tokens per chunk (the whole block
   rows a workgroup decodes and attends at once; a split of tile_tokens is
   processed in ceil(tile/chunk) chunks) for these parameters with ASTC V
   (astc != 0) or for the FP16 control, or a negative AKV_HIP_* code. */
int akv_hip_task_tokens(const AkvAttnParams* p, int astc);

/* --- Paged, ragged batches ---------------------------------------------------
 *
 * Sequences of different lengths whose K and V live in page pools addressed
 * through per-sequence block tables (the paged format the reference plans,
 * docs/representation_v0.1.md:47-50, :84-95). A page holds page_tokens tokens
 * of every kv head. Pools, for num_pages pages:
 *   k_pages   AKV_K_FP16: fp16 [num_pages][kv_heads][page_tokens][dim]
 *             AKV_K_U4G32: 4-bit codes [num_pages][kv_heads][page_tokens][dim/2]
 *             (two per byte, low nibble = even channel), with
 *   k_meta    fp16 [num_pages][kv_heads][page_tokens][dim/32][2] = (offset,
 *             scale) per group of 32 channels: k = code * scale + offset
 *             (affine_quantize(axis="token", group=32), codec.py:218-250)
 *   v_blocks  16-byte ASTC blocks [num_pages][kv_heads][page_tokens/block_y][atlas_cols]
 *   v_scale, v_offset  fp16 [num_pages][kv_heads][page_tokens]
 *   block_table int32 [batch][max_pages]: page of each page_tokens tokens
 *   seq_lens  int32 [batch], 1 .. max_tokens
 *   v_tail    NULL, or fp16 [batch][kv_heads][page_tokens][dim]: the last
 *             seq_len % page_tokens tokens of each sequence take V from here
 *             (the fresh tail not yet encoded; their pages' V blocks are not
 *             read), tail token i at row i.
 * Split states partial/stats are laid out as in the contiguous API with
 * `splits` = ceil(max_tokens / tile_tokens); sequence b uses its first
 * ceil(seq_len / tile_tokens). `arrivals`: batch * kv_heads zeroed counters,
 * as akv_hip_decode_attention_fused (the merge always runs in the split
 * launch here). No reference counterpart: the reference only sketches pages. */
#define AKV_K_FP16 0u
#define AKV_K_U4G32 1u

typedef struct AkvPagedParams {
    uint32_t batch;
    uint32_t max_tokens;    /* longest sequence */
    uint32_t query_heads;
    uint32_t kv_heads;
    uint32_t dim;           /* 64 or 128 */
    uint32_t page_tokens;   /* a multiple of 16 and of block_y */
    uint32_t max_pages;     /* block_table row length, >= ceil(max_tokens / page_tokens) */
    uint32_t num_pages;     /* pages in each pool */
    uint32_t tile_tokens;   /* tokens per split: a multiple of 16 and of block_y */
    uint32_t splits;        /* ceil(max_tokens / tile_tokens), at most 65535 */
    uint32_t layout;        /* AKV_LAYOUT_SCALAR or AKV_LAYOUT_RGBA */
    uint32_t block_x;
    uint32_t block_y;
    uint32_t atlas_cols;    /* blocks per page row */
    uint32_t k_format;      /* AKV_K_FP16 or AKV_K_U4G32 */
} AkvPagedParams;

int akv_hip_paged_decode_attention(const AkvPagedParams* p, const float* q, const void* k_pages,
                                   const uint16_t* k_meta, const void* v_blocks, const uint16_t* v_scale,
                                   const uint16_t* v_offset, const int32_t* block_table, const int32_t* seq_lens,
                                   const uint16_t* v_tail, float* partial, float* stats, float* out,
                                   uint32_t* arrivals, void* stream);

/* Appending to the paged cache (the active path the reference plans: an FP16
   fresh tail read by the same split-K, and on page completion a GPU upload of
   the encoded blocks with no re-encode, docs/representation_v0.1.md:84-95).

   akv_hip_paged_append writes one new token per sequence: k_new, v_new f32
   [batch][kv_heads][dim] go to row seq_lens[b] % page_tokens of page
   block_table[b][seq_lens[b] / page_tokens]: K as fp16 (AKV_K_FP16, round to
   nearest even) or as 4-bit codes plus k_meta computed on the GPU exactly as
   affine_quantize(axis="token", group=32) in fp32 (AKV_K_U4G32), V as fp16
   into v_tail (required). seq_lens holds the lengths before the append and is
   not modified (the caller advances it). A sequence whose slot has no valid
   page (seq_lens[b] / page_tokens >= max_pages, or an id outside
   [0, num_pages)) is left unchanged. Uses the pool fields of p (batch,
   kv_heads, dim, page_tokens, max_pages, num_pages, layout, block_x, block_y,
   atlas_cols, k_format); inputs finite.

   akv_hip_paged_commit_pages copies n pages the host has encoded (blocks
   [n][kv_heads][page_tokens/block_y][atlas_cols] 16-byte ASTC blocks, scale
   and offset fp16 [n][kv_heads][page_tokens], device memory) into the V pool
   pages page_ids[0..n) (device int32; ids outside [0, num_pages) are
   skipped), in one launch. A sequence whose length reaches a multiple of
   page_tokens needs its completed page committed before the next decode step
   reads it, and before the next append overwrites its tail. */
int akv_hip_paged_append(const AkvPagedParams* p, const float* k_new, const float* v_new, void* k_pages,
                         uint16_t* k_meta, const int32_t* block_table, const int32_t* seq_lens, uint16_t* v_tail,
                         void* stream);

int akv_hip_paged_commit_pages(const AkvPagedParams* p, uint32_t n, const int32_t* page_ids, const void* blocks,
                               const uint16_t* scale, const uint16_t* offset, void* v_blocks, uint16_t* v_scale,
                               uint16_t* v_offset, void* stream);

/* Host-side planning query for the paged kernel (no GPU work): tokens per
   chunk, or a negative AKV_HIP_* code. */
int akv_hip_paged_task_tokens(const AkvPagedParams* p);

/* Text for a return code of the functions above. */
const char* akv_hip_error_string(int code);

#ifdef __cplusplus
}
#endif
#endif
