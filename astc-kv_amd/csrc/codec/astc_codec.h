// CPU ASTC LDR codec behind the akv_* bridge (libakv_astc.so). Replaces the
// reference's astcenc binding (astc_kv/bridge.cpp) with an encoder and a
// table-driven decoder of our own.
#pragma once
#include <cstddef>
#include <cstdint>

#include "astc_format.h"

namespace akv {

enum BlockKind : int { kBlockNormal = 0, kBlockVoid = 1, kBlockError = 2 };

// Decode one 16-byte block into UNORM16 RGBA texels [by][bx][4].
int decode_block_unorm16(const AkvTables& t, const uint8_t* block, uint16_t* texels);

// Decode one block into FP16 bit patterns [by][bx][4].
int decode_block_fp16(const AkvTables& t, const uint8_t* block, uint16_t* texels);

struct EncoderOptions {
    float quality = 98.0f;   // 0..100: search effort (refinement passes, candidates)
};

// Encode one block of float RGBA texels in [0,1], [by][bx][4] row-major.
void encode_block(const AkvTables& t, const float* texels, const EncoderOptions& opt, uint8_t* out);

// Whole-image helpers with astcenc image semantics: row-major block payload,
// partial edge blocks replicate the last row/column.
int encode_image(const AkvTables& t, const float* rgba, unsigned w, unsigned h, const EncoderOptions& opt,
                 uint8_t* out, size_t bytes);
int decode_image(const AkvTables& t, const uint8_t* data, size_t bytes, float* rgba, unsigned w, unsigned h);

}  // namespace akv
