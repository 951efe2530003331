// akv_* C-ABI of libakv_astc.so (declared in include/astc_kv.h).
#include "astc_kv.h"

#include <new>

#include "astc_codec.h"

namespace {

struct Context {
    const akv::AkvTables* tables;
    akv::EncoderOptions options;
    unsigned bx, by;
};

size_t payload_bytes(const Context* c, unsigned w, unsigned h) {
    return size_t((w + c->bx - 1) / c->bx) * ((h + c->by - 1) / c->by) * 16;
}

}  // namespace

extern "C" {

void* akv_create(unsigned bx, unsigned by, float quality, int hdr, int* error) {
    int dummy = 0;
    if (!error) error = &dummy;
    if (hdr) {
        *error = AKV_ERR_BAD_PROFILE;
        return nullptr;
    }
    if (!(quality >= 0.0f && quality <= 100.0f)) {
        *error = AKV_ERR_BAD_QUALITY;
        return nullptr;
    }
    const akv::AkvTables* t = akv::tables_for(int(bx), int(by));
    if (!t) {
        *error = AKV_ERR_BAD_BLOCK_SIZE;
        return nullptr;
    }
    Context* c = new (std::nothrow) Context{t, akv::EncoderOptions{}, bx, by};
    if (!c) {
        *error = AKV_ERR_OUT_OF_MEM;
        return nullptr;
    }
    c->options.quality = quality;
    *error = AKV_SUCCESS;
    return c;
}

void akv_destroy(void* ctx) { delete static_cast<Context*>(ctx); }

const char* akv_error(int code) {
    switch (code) {
        case AKV_SUCCESS: return "ASTC-KV success";
        case AKV_ERR_OUT_OF_MEM: return "ASTC-KV out of memory";
        case AKV_ERR_BAD_PARAM: return "ASTC-KV bad parameter";
        case AKV_ERR_BAD_BLOCK_SIZE: return "ASTC-KV unsupported block size (2D, 4..12 per side, <= 64 texels)";
        case AKV_ERR_BAD_PROFILE: return "ASTC-KV unsupported profile (LDR only)";
        case AKV_ERR_BAD_QUALITY: return "ASTC-KV quality outside [0, 100]";
        case AKV_ERR_BAD_CONTEXT: return "ASTC-KV null context";
        case AKV_ERR_BAD_BUFFER: return "ASTC-KV buffer size does not match the image";
        default: return "ASTC-KV unknown error";
    }
}

int akv_encode(void* ctx, float* pixels, unsigned w, unsigned h, uint8_t* compressed, size_t bytes) {
    Context* c = static_cast<Context*>(ctx);
    if (!c) return AKV_ERR_BAD_CONTEXT;
    if (!pixels || !compressed || w == 0 || h == 0) return AKV_ERR_BAD_PARAM;
    if (bytes < payload_bytes(c, w, h)) return AKV_ERR_BAD_BUFFER;
    return akv::encode_image(*c->tables, pixels, w, h, c->options, compressed, bytes) ? AKV_ERR_BAD_BUFFER
                                                                                      : AKV_SUCCESS;
}

int akv_decode(void* ctx, const uint8_t* compressed, size_t bytes, float* pixels, unsigned w, unsigned h) {
    Context* c = static_cast<Context*>(ctx);
    if (!c) return AKV_ERR_BAD_CONTEXT;
    if (!pixels || !compressed || w == 0 || h == 0) return AKV_ERR_BAD_PARAM;
    if (bytes < payload_bytes(c, w, h)) return AKV_ERR_BAD_BUFFER;
    return akv::decode_image(*c->tables, compressed, bytes, pixels, w, h) ? AKV_ERR_BAD_BUFFER : AKV_SUCCESS;
}

int akv_encode_blocks(void* ctx, const float* texels, size_t n, uint8_t* blocks) {
    Context* c = static_cast<Context*>(ctx);
    if (!c) return AKV_ERR_BAD_CONTEXT;
    if ((!texels || !blocks) && n) return AKV_ERR_BAD_PARAM;
    const size_t per = size_t(c->bx) * c->by * 4;
    for (size_t i = 0; i < n; ++i) akv::encode_block(*c->tables, texels + i * per, c->options, blocks + 16 * i);
    return AKV_SUCCESS;
}

int akv_decode_blocks_fp16(unsigned bx, unsigned by, const uint8_t* blocks, size_t n, uint16_t* texels,
                           int32_t* kinds) {
    const akv::AkvTables* t = akv::tables_for(int(bx), int(by));
    if (!t) return AKV_ERR_BAD_BLOCK_SIZE;
    if ((!blocks || !texels) && n) return AKV_ERR_BAD_PARAM;
    const size_t per = size_t(bx) * by * 4;
    for (size_t i = 0; i < n; ++i) {
        int k = akv::decode_block_fp16(*t, blocks + 16 * i, texels + i * per);
        if (kinds) kinds[i] = k;
    }
    return AKV_SUCCESS;
}

}  // extern "C"
