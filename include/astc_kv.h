/*
 * astc_kv.h — CPU ASTC codec bridge (libakv_astc.so).
 *
 * Drop-in replacement for the reference's astcenc bridge. The five akv_*
 * entry points keep the reference signatures and semantics, as bound by
 * ctypes in astc_kv/codec.py:27-33:
 *   akv_create   astc_kv/bridge.cpp:7-15
 *   akv_destroy  astc_kv/bridge.cpp:16
 *   akv_error    astc_kv/bridge.cpp:17
 *   akv_encode   astc_kv/bridge.cpp:18-26
 *   akv_decode   astc_kv/bridge.cpp:27-35
 * Images are float32 RGBA, row-major [h][w][4]; payloads are row-major 16-byte
 * blocks, ceil(w/bx)*ceil(h/by) of them. The caller owns every buffer. One
 * context must not be used by two threads at once (the reference creates
 * one astcenc thread per context). Return value 0 means success; other codes
 * map to text through akv_error.
 *
 * The encoder is this library's own (astcenc is not available); decoding is
 * ASTC LDR with astcenc's float output contract: texels are FP16 values,
 * UNORM16 c -> 1.0 when c == 0xFFFF, else c/65536 truncated to FP16.
 * HDR profiles are not supported (akv_create reports AKV_ERR_BAD_PROFILE).
 */
#ifndef ASTC_KV_H
#define ASTC_KV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    AKV_SUCCESS = 0,
    AKV_ERR_OUT_OF_MEM = 1,
    AKV_ERR_BAD_PARAM = 2,
    AKV_ERR_BAD_BLOCK_SIZE = 3,
    AKV_ERR_BAD_PROFILE = 4,
    AKV_ERR_BAD_QUALITY = 5,
    AKV_ERR_BAD_CONTEXT = 6,
    AKV_ERR_BAD_BUFFER = 7
};

/* astc_kv/bridge.cpp:7-15. Returns NULL and sets *error on failure. */
void* akv_create(unsigned bx, unsigned by, float quality, int hdr, int* error);
/* astc_kv/bridge.cpp:16. NULL is ignored. */
void akv_destroy(void* ctx);
/* astc_kv/bridge.cpp:17. Static string; the caller does not free it. */
const char* akv_error(int code);
/* astc_kv/bridge.cpp:18-26. pixels: float32 [h][w][4] in [0,1]; compressed:
   `bytes` >= ceil(w/bx)*ceil(h/by)*16. */
int akv_encode(void* ctx, float* pixels, unsigned w, unsigned h, uint8_t* compressed, size_t bytes);
/* astc_kv/bridge.cpp:27-35. pixels: float32 [h][w][4] written by the call. */
int akv_decode(void* ctx, const uint8_t* compressed, size_t bytes, float* pixels, unsigned w, unsigned h);

/* Additions with no counterpart in the reference bridge (used by the atlas
   builder and the tests; the reference encodes whole images only):
   akv_encode_blocks: texels float32 [n][by][bx][4] -> n 16-byte blocks.
   akv_decode_blocks_fp16: n blocks -> FP16 bit patterns [n][by][bx][4]; kinds
   (optional) receives 0 normal, 1 void extent, 2 error block per block. */
int akv_encode_blocks(void* ctx, const float* texels, size_t n, uint8_t* blocks);
int akv_decode_blocks_fp16(unsigned bx, unsigned by, const uint8_t* blocks, size_t n, uint16_t* texels,
                           int32_t* kinds);

/* akv_block_classes: the decode-path class of each of n blocks of a bx x by
   footprint (what decides its decode cost), one word per block:
   bits 0-1 kind (AKV_CLASS_NORMAL / VOID / ERROR, by the same rules as
   akv_decode_blocks_fp16's kinds), 2-3 partitions - 1, 4 dual plane,
   5 weight grid the size of the block, 6-11 weight levels, 12-15 endpoint
   mode of the first partition, 16 one endpoint mode shared by every
   partition. The normal-block fields are zero for void-extent and error
   blocks. No counterpart in the reference: a diagnostic for atlases. */
enum { AKV_CLASS_NORMAL = 0, AKV_CLASS_VOID = 1, AKV_CLASS_ERROR = 2 };
int akv_block_classes(unsigned bx, unsigned by, const uint8_t* blocks, size_t n, uint32_t* out);

#ifdef __cplusplus
}
#endif
#endif
