// akv_* C-ABI of libakv_astc.so (declared in include/astc_kv.h).
#include "astc_kv.h"

#include <algorithm>
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

int akv_block_classes(unsigned bx, unsigned by, const uint8_t* blocks, size_t n, uint32_t* out) {
    const akv::AkvTables* t = akv::tables_for(int(bx), int(by));
    if (!t) return AKV_ERR_BAD_BLOCK_SIZE;
    if ((!blocks || !out) && n) return AKV_ERR_BAD_PARAM;
    auto bits = [](const uint8_t* b, int start, int count) {   // little-endian bit field, count <= 24
        uint32_t v = 0;
        for (int k = 0; k < count; ++k) v |= uint32_t((b[(start + k) >> 3] >> ((start + k) & 7)) & 1) << k;
        return v;
    };
    for (size_t i = 0; i < n; ++i) {
        const uint8_t* b = blocks + 16 * i;
        const uint32_t mode = bits(b, 0, 11);
        if ((mode & 0x1FF) == 0x1FC) {
            // Void extent: LDR only, and the extent either all ones or ordered.
            const uint32_t s0 = bits(b, 12, 13), s1 = bits(b, 25, 13), t0 = bits(b, 38, 13), t1 = bits(b, 51, 13);
            const bool all_ones = s0 == 0x1FFF && s1 == 0x1FFF && t0 == 0x1FFF && t1 == 0x1FFF;
            out[i] = (bits(b, 9, 1) || (!all_ones && (s0 >= s1 || t0 >= t1))) ? AKV_CLASS_ERROR : AKV_CLASS_VOID;
            continue;
        }
        const uint32_t md = t->block_mode[mode];
        const uint32_t parts = bits(b, 11, 2) + 1;
        if (!md || (akv::mode_dual(md) && parts == 4)) {
            out[i] = AKV_CLASS_ERROR;
            continue;
        }
        uint32_t cem[4] = {0, 0, 0, 0}, shared = 1;
        int below = 128 - int(akv::mode_wbits(md)), config_start = 17;
        if (parts == 1) {
            cem[0] = bits(b, 13, 4);
        } else {
            config_start = 29;
            const uint32_t field = bits(b, 23, 6);
            if ((field & 3) == 0) {
                for (uint32_t p = 0; p < parts; ++p) cem[p] = field >> 2;
            } else {
                shared = 0;
                const int extra = 3 * int(parts) - 4;
                below -= extra;
                const uint32_t enc = field | bits(b, below, extra) << 6;
                const uint32_t base = (enc & 3) - 1;
                for (uint32_t p = 0; p < parts; ++p)
                    cem[p] = (base + ((enc >> (2 + p)) & 1)) << 2 | ((enc >> (2 + parts + 2 * p)) & 3);
            }
        }
        if (akv::mode_dual(md)) below -= 2;
        int pairs = 0;
        for (uint32_t p = 0; p < parts; ++p) pairs += int(cem[p] >> 2) + 1;
        const int avail = below - config_start;
        // Colour values must fit (at most 18) with at least 6 levels (range 4).
        if (pairs > 9 || avail <= 0 || t->color_range[pairs][std::min(avail, 127)] < 4) {
            out[i] = AKV_CLASS_ERROR;
            continue;
        }
        out[i] = AKV_CLASS_NORMAL | (parts - 1) << 2 | akv::mode_dual(md) << 4 | akv::mode_identity(md) << 5 |
                 uint32_t(t->weight_levels[akv::mode_range(md)]) << 6 | cem[0] << 12 | shared << 16;
    }
    return AKV_SUCCESS;
}

}  // extern "C"
