// ASTC LDR format tables shared by the CPU codec (libakv_astc.so) and the
// gfx950 decode kernels (libastckv_hip.so uploads one AkvTables per footprint
// to device memory). Everything here is plain data so the same struct is read
// by host code and by device code.
//
// The decode these tables drive is the one astcenc 5.7.0 performs behind the
// reference bridge (astc_kv/bridge.cpp:27-35): block mode -> weight grid,
// integer-sequence (BISE) unpacking, endpoint and weight unquantisation, the
// partition hash, and UNORM16 -> FP16 truncation of the interpolated texel.
#pragma once
#include <cstddef>
#include <cstdint>

namespace akv {

constexpr int kMaxTexels = 64;     // footprints up to 8x8 (codec.py allows 4/6/8)
constexpr int kNumRanges = 21;     // ISE ranges: 2,3,4,5,6,8,...,192,256 levels
constexpr int kRange6 = 4;         // lowest range allowed for colour endpoints

// Integer-sequence ranges, in the order of the ASTC range index: {plain bits,
// trit?, quint?}; levels = (1 + 2*trit + 4*quint) << bits. Weight ranges are
// indices 0..11, colour ranges 4..20.
struct IseRange {
    uint8_t bits, trit, quint;
};
inline constexpr IseRange kIse[kNumRanges] = {
    {1, 0, 0}, {0, 1, 0}, {2, 0, 0}, {0, 0, 1}, {1, 1, 0}, {3, 0, 0}, {1, 0, 1},
    {2, 1, 0}, {4, 0, 0}, {2, 0, 1}, {3, 1, 0}, {5, 0, 0}, {3, 0, 1}, {4, 1, 0},
    {6, 0, 0}, {4, 0, 1}, {5, 1, 0}, {7, 0, 0}, {5, 0, 1}, {6, 1, 0}, {8, 0, 0}};

// Packed block-mode descriptor (AkvTables::block_mode), 0 for an invalid or
// reserved mode and for a void-extent selector.
//   bits 0-3 grid width, 4-7 grid height, 8 dual plane, 9-12 weight range,
//   13-19 weight bit count, 20 grid equals footprint, 31 valid.
constexpr uint32_t kModeValid = 1u << 31;
inline constexpr uint32_t mode_gw(uint32_t m) { return m & 15u; }
inline constexpr uint32_t mode_gh(uint32_t m) { return (m >> 4) & 15u; }
inline constexpr uint32_t mode_dual(uint32_t m) { return (m >> 8) & 1u; }
inline constexpr uint32_t mode_range(uint32_t m) { return (m >> 9) & 15u; }
inline constexpr uint32_t mode_wbits(uint32_t m) { return (m >> 13) & 127u; }
inline constexpr uint32_t mode_identity(uint32_t m) { return (m >> 20) & 1u; }

struct AkvTables {
    // --- leading kLdsTableBytes bytes: the per-block decode tables, which the
    // --- GPU kernels copy into LDS as one contiguous block.
    uint32_t block_mode[2048];
    // Unquantised colour value 0..255 for each range and ISE value.
    uint8_t color_unq[kNumRanges][256];
    // Highest colour range whose ISE sequence of 2*pairs values fits in the
    // available bits, or -1. Index [pairs 1..9][bits 0..127].
    int8_t color_range[10][128];
    // 8-bit trit block -> five trits, trit j in bits 2j..2j+1.
    uint16_t trit[256];
    // 7-bit quint block -> three quints, quint j in bits 3j..3j+2.
    uint16_t quint[128];
    // Per ISE range: low 8 bits = plain bit count, bit 8 = trit, bit 9 = quint.
    uint16_t ise[kNumRanges];
    uint16_t pad0;
    // Unquantised weight 0..64 for each weight range (0..11) and ISE value.
    uint8_t weight_unq[12][32];
    // Number of values of each weight range (2, 3, 4, 5, 6, 8, ..., 32).
    uint8_t weight_levels[12];
    uint8_t pad1[8];
    // --- end of the LDS block.
    // Partition of each texel for 2, 3 and 4 partitions and every 10-bit seed:
    // texel i occupies bits 2*(i%16) of word i/16.
    uint32_t partition[3][1024][4];
    uint32_t block_x, block_y;
};

constexpr size_t kLdsTableBytes = offsetof(AkvTables, partition);
static_assert(kLdsTableBytes % 16 == 0, "LDS table block must be a whole number of 16-byte copies");

// ISE helpers.
int ise_bits(int range);        // plain bits per value
bool ise_trit(int range);
bool ise_quint(int range);
int ise_levels(int range);
int ise_sequence_bits(int count, int range);

// Spec formulations used to build the tables (also used by the encoder).
uint32_t decode_block_mode(uint32_t mode, int bx, int by);
int partition_of(int seed, int x, int y, int count, bool small_block);
void trits_from_block(unsigned T, int t[5]);
void quints_from_block(unsigned Q, int q[3]);
int unquant_color(int range, int value);
int unquant_weight(int range, int value);

// Fill `t` for a bx x by footprint. Returns false for unsupported footprints
// (bx, by in 4..12, bx*by <= kMaxTexels).
bool build_tables(int bx, int by, AkvTables* t);

// Cached, immutable tables for a footprint (thread-safe); nullptr if unsupported.
const AkvTables* tables_for(int bx, int by);

// UNORM16 interpolation result -> FP16 bit pattern: 0xFFFF -> 1.0, otherwise
// c/65536 truncated toward zero.
uint16_t unorm16_to_fp16_bits(uint32_t c);

}  // namespace akv
