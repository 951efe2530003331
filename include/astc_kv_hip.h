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
 * Conventions: every pointer is a device pointer owned by the caller; `stream`
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
    AKV_HIP_ERR_TILE = -4         /* tile_tokens/splits inconsistent */
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
    uint32_t tile_tokens;   /* tokens per split (any positive multiple of block_y) */
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

/* Text for a return code of the functions above. */
const char* akv_hip_error_string(int code);

#ifdef __cplusplus
}
#endif
#endif
