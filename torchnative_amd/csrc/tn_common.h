// Shared helpers for the tnhip library: status plumbing, launch accounting,
// exact reduced-float conversions usable on host and device.
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <string>

#include "../../include/tnhip.h"

namespace tn {

// ---- status / errors -------------------------------------------------------

void set_error(const std::string& msg);
tn_status fail(tn_status code, const std::string& msg);
tn_status hip_fail(hipError_t e, const char* what);

struct Counters {
    std::atomic<uint64_t> dispatches{0};
    std::atomic<uint64_t> bytes_uploaded{0};
    std::atomic<uint64_t> host_downloads{0};
    std::atomic<uint64_t> bytes_downloaded{0};
    std::atomic<uint64_t> refusals{0};
    std::atomic<uint64_t> workspace_bytes{0};
};
Counters& counters();

// Grow-only device workspace, one per (device, stream). Calls on one stream
// are ordered, so reuse across them is safe.
tn_status workspace(hipStream_t stream, size_t bytes, void** out);
// Workgroups of `kernel` (block threads, lds dynamic bytes) that the current
// device holds at once: the size of a persistent grid, all of whose
// workgroups must be resident from the start. Cached per (device, kernel,
// block, lds).
tn_status resident_workgroups(const void* kernel, int block, size_t lds, int* out);

// Decode attention (sdpa.hip), shared with the decode step: argument checks,
// and the launch with caller-provided split partials (B*Hq*ceil(max_len/256)
// rows of D floats and as many (m, l) pairs). The grid depends on max_len
// only; each workgroup reads its sequence's length from `lens` on the device.
tn_status decode_check(int dtype, int64_t B, int64_t Hq, int64_t Hkv, int64_t cap, int64_t D, int64_t max_len);
tn_status decode_launch(hipStream_t st, int dtype, const void* q, const void* k_cache, const void* v_cache,
                        int64_t B, int64_t Hq, int64_t Hkv, int64_t cap, int64_t D, const int32_t* lens,
                        int64_t max_len, double scale, void* out, float* lse, float* part_o, float2* part_ml);
constexpr int DECODE_SPLIT_KEYS = 256;  // keys per split of the decode attention

#define TN_HIP(call)                                              \
    do {                                                          \
        hipError_t e_ = (call);                                   \
        if (e_ != hipSuccess) return ::tn::hip_fail(e_, #call);  \
    } while (0)

#define TN_LAUNCHED()                                              \
    do {                                                           \
        ::tn::counters().dispatches.fetch_add(1);                  \
        hipError_t e_ = hipGetLastError();                         \
        if (e_ != hipSuccess) return ::tn::hip_fail(e_, "launch"); \
    } while (0)

// ---- reduced floats (exact, identical on host and device) ---------------

// f32 -> f16 round-to-nearest-even with subnormals and overflow to inf: the
// IEEE conversion of half 2.7.1's f16::from_f32, which stores every Q4_0 and
// Q8_0 block scale in the reference.
__host__ __device__ inline uint16_t f16_from_f32(float f) {
    uint32_t x = __builtin_bit_cast(uint32_t, f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xffu;
    uint32_t man = x & 0x7fffffu;
    if (exp == 0xffu) return (uint16_t)(sign | 0x7c00u | (man ? (0x0200u | (man >> 13)) : 0u));
    int32_t e = (int32_t)exp - 112;  // -127 + 15
    if (e >= 0x1f) return (uint16_t)(sign | 0x7c00u);
    if (e <= 0) {
        if (14 - e > 24) return (uint16_t)sign;
        uint32_t m = man | 0x800000u;
        uint32_t shift = (uint32_t)(14 - e);
        uint32_t hm = m >> shift;
        uint32_t rb = 1u << (shift - 1);
        if ((m & rb) && (m & (3u * rb - 1u))) hm += 1;
        return (uint16_t)(sign | hm);
    }
    uint32_t h = sign | ((uint32_t)e << 10) | (man >> 13);
    if ((man & 0x1000u) && (man & 0x2fffu)) h += 1;
    return (uint16_t)h;
}

__host__ __device__ inline float f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t exp = ((uint32_t)h >> 10) & 0x1fu;
    uint32_t man = (uint32_t)h & 0x3ffu;
    if (exp == 0x1fu) return __builtin_bit_cast(float, sign | 0x7f800000u | (man << 13));
    if (exp == 0) {
        // subnormal or zero: man * 2^-24 is exact in f32
        float v = (float)man * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    return __builtin_bit_cast(float, sign | ((exp + 112u) << 23) | (man << 13));
}

// f32 -> bf16 round-to-nearest-even, NaN quieted (reduced.rs:161-218).
__host__ __device__ inline uint16_t bf16_from_f32(float f) {
    uint32_t x = __builtin_bit_cast(uint32_t, f);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
    return (uint16_t)((x + 0x7fffu + ((x >> 16) & 1u)) >> 16);
}

__host__ __device__ inline float bf16_to_f32(uint16_t h) {
    return __builtin_bit_cast(float, (uint32_t)h << 16);
}

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

}  // namespace tn
