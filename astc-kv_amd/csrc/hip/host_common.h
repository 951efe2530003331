// Host-side pieces shared by the kernel translation units of libastckv_hip.
#pragma once
#include <hip/hip_runtime.h>

#include <cstdint>

#include "astc_decode_device.h"

namespace akv_hip {

// Device copy of the decode tables for footprint (bx, by) on the current
// device; the first call per (device, footprint) uploads them (blocking).
int device_tables(int bx, int by, const akv::AkvTables** out);

// ceil(2^24 / d): a / d == fdiv(a, magic(d)) whenever a * d < 2^24.
uint32_t magic(uint32_t d);

// Footprint shape and weight-infill steps.
Footprint footprint(uint32_t bx, uint32_t by);

inline int as_int(hipError_t e) { return e == hipSuccess ? 0 : int(e); }

// The kernels read Q, K, V and the V blocks with 16-byte vector loads.
inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace akv_hip
