// 128-bit block helpers for the CPU codec.
#pragma once
#include <cstdint>
#include <cstring>

namespace akv {

struct Bits128 {
    uint64_t lo = 0, hi = 0;

    static Bits128 load(const uint8_t* p) {
        Bits128 b;
        std::memcpy(&b.lo, p, 8);
        std::memcpy(&b.hi, p + 8, 8);
        return b;
    }
    void store(uint8_t* p) const {
        std::memcpy(p, &lo, 8);
        std::memcpy(p + 8, &hi, 8);
    }
    // Bits [pos, pos+n) as an integer, n <= 64; bits at or beyond 128 read 0.
    uint64_t get(int pos, int n) const {
        if (n <= 0 || pos >= 128) return 0;
        uint64_t v;
        if (pos == 0) v = lo;
        else if (pos < 64) v = (lo >> pos) | (hi << (64 - pos));
        else v = hi >> (pos - 64);
        return n >= 64 ? v : v & ((uint64_t(1) << n) - 1);
    }
    void put(int pos, int n, uint64_t v) {
        for (int i = 0; i < n; ++i) {
            int p = pos + i;
            if (p >= 128) break;
            uint64_t bit = (v >> i) & 1;
            if (p < 64) lo |= bit << p;
            else hi |= bit << (p - 64);
        }
    }
    Bits128 reversed() const {
        Bits128 r;
        r.lo = rev64(hi);
        r.hi = rev64(lo);
        return r;
    }
    static uint64_t rev64(uint64_t x) {
        x = ((x >> 1) & 0x5555555555555555ull) | ((x & 0x5555555555555555ull) << 1);
        x = ((x >> 2) & 0x3333333333333333ull) | ((x & 0x3333333333333333ull) << 2);
        x = ((x >> 4) & 0x0F0F0F0F0F0F0F0Full) | ((x & 0x0F0F0F0F0F0F0F0Full) << 4);
        return __builtin_bswap64(x);
    }
};

}  // namespace akv
