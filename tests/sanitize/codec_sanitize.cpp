// Drives the CPU codec (libakv_astc sources) and the oracle's C decoder
// through every entry point on random and encoder-produced blocks, for a
// build with AddressSanitizer and UndefinedBehaviorSanitizer
// (tests/test_sanitizers.py compiles and runs it). Exits non-zero on any
// decoder disagreement; the sanitizers abort on any memory or UB error.
#include <cstdio>
#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <random>
#include <vector>

#include "astc_kv.h"

extern "C" {
void oracle_decode_blocks_fp16(const uint8_t* blocks, long n, int bx, int by, uint16_t* out, int* kinds);
int oracle_decode_image(const uint8_t* data, long bytes, int bx, int by, int w, int h, float* img);
}

static int check(int rc, const char* what) {
    if (rc != AKV_SUCCESS) std::fprintf(stderr, "%s: %s\n", what, akv_error(rc));
    return rc != AKV_SUCCESS;
}

int main(int argc, char** argv) {
    const int nrand = argc > 1 ? std::atoi(argv[1]) : 20000;
    const int fp[][2] = {{4, 4}, {5, 4}, {5, 5}, {6, 5}, {6, 6}, {8, 5}, {8, 6}, {8, 8}, {10, 5}, {10, 6}, {12, 5}};
    std::mt19937_64 rng(20261202);
    int bad = 0;
    for (const auto& f : fp) {
        const int bx = f[0], by = f[1], nt = bx * by;
        // Random 128-bit blocks (every mode, void extents, errors): product
        // decoder against the oracle, and the block classes.
        std::vector<uint8_t> blocks(size_t(nrand) * 16);
        for (auto& b : blocks) b = uint8_t(rng());
        for (int i = 0; i < nrand / 20; ++i) {
            blocks[16 * i] = 0xFC;
            blocks[16 * i + 1] = uint8_t((blocks[16 * i + 1] & 0xF0) | 0x0D);
        }
        std::vector<uint16_t> got(size_t(nrand) * nt * 4), exp(got.size());
        std::vector<int32_t> kg(nrand);
        std::vector<int> ke(nrand);
        std::vector<uint32_t> cls(nrand);
        bad += check(akv_decode_blocks_fp16(bx, by, blocks.data(), nrand, got.data(), kg.data()), "decode_blocks");
        oracle_decode_blocks_fp16(blocks.data(), nrand, bx, by, exp.data(), ke.data());
        bad += check(akv_block_classes(bx, by, blocks.data(), nrand, cls.data()), "block_classes");
        for (int i = 0; i < nrand; ++i)
            if (kg[i] != ke[i] || int(cls[i] & 3) != ke[i] ||
                std::memcmp(&got[size_t(i) * nt * 4], &exp[size_t(i) * nt * 4], size_t(nt) * 8)) {
                if (bad < 5) std::fprintf(stderr, "%dx%d block %d differs\n", bx, by, i);
                ++bad;
            }
        // Encoder round trip on an image whose edge blocks are partial, at two
        // qualities; akv_decode against the oracle's image decode.
        for (float quality : {10.0f, 98.0f}) {
            int err = 0;
            void* ctx = akv_create(bx, by, quality, 0, &err);
            if (!ctx) { bad += check(err, "create"); continue; }
            const unsigned w = 3 * bx + 1, h = 2 * by + 3;
            std::vector<float> img(size_t(w) * h * 4), dec(img.size()), ref(img.size());
            std::uniform_real_distribution<float> u(0.0f, 1.0f);
            for (auto& v : img) v = u(rng);
            const size_t nb = size_t((w + bx - 1) / bx) * ((h + by - 1) / by);
            std::vector<uint8_t> payload(nb * 16);
            bad += check(akv_encode(ctx, img.data(), w, h, payload.data(), payload.size()), "encode");
            bad += check(akv_decode(ctx, payload.data(), payload.size(), dec.data(), w, h), "decode");
            oracle_decode_image(payload.data(), long(payload.size()), bx, by, int(w), int(h), ref.data());
            if (std::memcmp(dec.data(), ref.data(), dec.size() * sizeof(float))) {
                std::fprintf(stderr, "%dx%d q%g image decode differs\n", bx, by, quality);
                ++bad;
            }
            // The scalar layout's images (grey RGB, alpha 1: luminance
            // endpoint modes, and at quality 90+ the endpoint polish).
            for (size_t i = 0; i < img.size(); i += 4) img[i + 1] = img[i + 2] = img[i], img[i + 3] = 1.0f;
            bad += check(akv_encode(ctx, img.data(), w, h, payload.data(), payload.size()), "encode grey");
            bad += check(akv_decode(ctx, payload.data(), payload.size(), dec.data(), w, h), "decode grey");
            oracle_decode_image(payload.data(), long(payload.size()), bx, by, int(w), int(h), ref.data());
            if (std::memcmp(dec.data(), ref.data(), dec.size() * sizeof(float))) {
                std::fprintf(stderr, "%dx%d q%g grey image decode differs\n", bx, by, quality);
                ++bad;
            }
            // Texel blocks straight through akv_encode_blocks.
            std::vector<float> tex(size_t(8) * nt * 4);
            for (auto& v : tex) v = u(rng);
            std::vector<uint8_t> eb(8 * 16);
            bad += check(akv_encode_blocks(ctx, tex.data(), 8, eb.data()), "encode_blocks");
            // Refusals: short buffers and null pointers come back as errors.
            if (akv_encode(ctx, img.data(), w, h, payload.data(), payload.size() - 1) == AKV_SUCCESS) ++bad;
            if (akv_decode(ctx, payload.data(), payload.size() - 1, dec.data(), w, h) == AKV_SUCCESS) ++bad;
            akv_destroy(ctx);
        }
    }
    // Footprints past 64 texels are refused, not decoded.
    {
        int err = 0;
        uint8_t blk[16] = {};
        uint16_t tex[10 * 10 * 4];
        uint32_t c = 0;
        if (akv_create(10, 10, 50.0f, 0, &err) != nullptr || err != AKV_ERR_BAD_BLOCK_SIZE) ++bad;
        if (akv_decode_blocks_fp16(10, 10, blk, 1, tex, nullptr) != AKV_ERR_BAD_BLOCK_SIZE) ++bad;
        if (akv_block_classes(10, 10, blk, 1, &c) != AKV_ERR_BAD_BLOCK_SIZE) ++bad;
    }
    akv_destroy(nullptr);
    std::printf("sanitized codec run: %d problems\n", bad);
    return bad ? 1 : 0;
}
