// Pieces shared by the attention kernels (sdpa.hip, flash64.hip): the
// 16-bit formats and their MFMA, LDS transposed reads, the LDS DMA load, the
// mask reader, small wave reductions and waits.
#pragma once

#include "tn_common.h"

namespace tn {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

constexpr float LOG2E = 1.4426950408889634f;
constexpr float LN2 = 0.69314718055994531f;
constexpr float RESCALE_SLACK = 8.0f;  // log2 of the largest unnormalised probability

// over lanes l, l ^ 16, l ^ 32, l ^ 48
__device__ inline float wave_xor_max(float v) { return xor32_max(xor16_max(v)); }
__device__ inline float wave_xor_sum(float v) { return xor32_sum(xor16_sum(v)); }

// two f32 -> packed bf16 pair, RNE (v_cvt_pk_bf16_f32); used for the
// probabilities, which are finite and non-negative
__device__ inline uint32_t pack2_bf16_hw(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, bf16x2));
}

// the same narrowing spelled out (reduced.rs:161-218: RNE, NaN quieted), for outputs
__device__ inline uint32_t pack2_bf16(float a, float b) {
    return (uint32_t)bf16_from_f32(a) | ((uint32_t)bf16_from_f32(b) << 16);
}

typedef float f32x16 __attribute__((ext_vector_type(16)));

// The 16-bit storage formats of the prefill kernel: bf16 or f16 inputs, the
// f32-accumulating MFMA of that type, the narrowing of the probabilities to
// it between the two products, and the narrowing of the output (RNE; f16 with
// subnormals and overflow to inf, bf16 with NaN quieted).
template <bool F16>
struct El;
template <>
struct El<false> {
    typedef __bf16 v8 __attribute__((ext_vector_type(8)));
    static __device__ inline f32x16 mfma(v8 a, v8 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
    }
    static __device__ inline uint32_t pack_p(float a, float b) { return pack2_bf16_hw(a, b); }
    static __device__ inline uint32_t pack_out(float a, float b) { return pack2_bf16(a, b); }
    // pack_out's bits through v_cvt_pk_bf16_f32 (round to nearest even, as
    // bf16_from_f32 for every number), with a NaN given bf16_from_f32's
    // quieted payload
    static __device__ inline uint32_t pack_out_hw(float a, float b) {
        uint32_t r = pack2_bf16_hw(a, b);
        if (a != a) r = (r & 0xffff0000u) | ((__float_as_uint(a) >> 16) | 0x40u);
        if (b != b) r = (r & 0xffffu) | (((__float_as_uint(b) >> 16) | 0x40u) << 16);
        return r;
    }
    static __device__ inline float widen(uint16_t h) { return bf16_to_f32(h); }
    static __device__ inline f32x4 mfma16(v8 a, v8 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
    // the low and high element of a packed pair, widened (exact)
    static __device__ inline float lo(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
    static __device__ inline float hi(uint32_t w) { return __builtin_bit_cast(float, w & 0xffff0000u); }
};
template <>
struct El<true> {
    typedef _Float16 v8 __attribute__((ext_vector_type(8)));
    typedef _Float16 v2 __attribute__((ext_vector_type(2)));
    static __device__ inline f32x16 mfma(v8 a, v8 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
    }
    // v_cvt_f16_f32 rounds to nearest even (equal to f16_from_f32 for every float)
    static __device__ inline uint32_t pack_p(float a, float b) {
        return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, v2));
    }
    static __device__ inline uint32_t pack_out(float a, float b) {
        return (uint32_t)f16_from_f32(a) | ((uint32_t)f16_from_f32(b) << 16);
    }
    // pack_out's bits through v_cvt_f16_f32 (equal to f16_from_f32 for every
    // number, subnormals and overflow included), with a NaN given
    // f16_from_f32's quieted payload
    static __device__ inline uint32_t pack_out_hw(float a, float b) {
        uint32_t r = pack_p(a, b);
        if (a != a) r = (r & 0xffff0000u) | f16_from_f32(a);
        if (b != b) r = (r & 0xffffu) | ((uint32_t)f16_from_f32(b) << 16);
        return r;
    }
    static __device__ inline float widen(uint16_t h) { return f16_to_f32(h); }
    static __device__ inline f32x4 mfma16(v8 a, v8 b, f32x4 c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
    static __device__ inline float lo(uint32_t w) { return f16_bits_hw((uint16_t)(w & 0xffffu)); }
    static __device__ inline float hi(uint32_t w) { return f16_bits_hw((uint16_t)(w >> 16)); }
};
typedef short i16x4 __attribute__((ext_vector_type(4)));

// ds_read_b64_tr_b16: within each 16-lane group, lane i receives element
// (i % 4) of the 8-byte rows that lanes i/4, 4 + i/4, 8 + i/4 and 12 + i/4
// point at -- a 4-key x 16-column block read out column-wise.
__device__ inline uint2 lds_read_tr16(const uint16_t* p) {
#if __HIP_DEVICE_COMPILE__
    typedef __attribute__((address_space(3))) i16x4 lds_i16x4;
    return __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4*)(p)));
#else
    (void)p;
    return make_uint2(0, 0);
#endif
}

// s_waitcnt vmcnt(n) for a compile-time n (expcnt and lgkmcnt left open)
template <int N>
__device__ inline void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xf << 8));
}

// An attention mask as the kernels read it, broadcast by strides: element
// (b, h, i, j) sits at p[b*sb + h*sh + i*sl + j*sk] (element strides; a zero
// stride repeats that dim, as aten.rs:10293-10303 broadcasts the mask onto
// the scores). The kernels' MASK parameter names its format:
//   1 f32 additive; 2 additive in the 16-bit (or f64) query format;
//   3 bool (one byte, nonzero = attend), read as where(mask, 0, -inf), which
//     is the additive mask F.sdpa builds from a bool one
//     (bootstrap.py:12918-12925, :13065-13066).
struct MaskRef {
    const void* p;
    int64_t sb, sh, sl, sk;
};

// The additive value of mask element `off` in natural units.
template <int MASK, bool F16>
__device__ __attribute__((always_inline)) inline float mask_val(const void* p, int64_t off) {
    if constexpr (MASK == 1) return reinterpret_cast<const float*>(p)[off];
    else if constexpr (MASK == 3) return reinterpret_cast<const uint8_t*>(p)[off] ? 0.0f : -INFINITY;
    else if constexpr (F16) return f16_bits_hw(reinterpret_cast<const uint16_t*>(p)[off]);  // exact (tn_common.h)
    else return bf16_to_f32(reinterpret_cast<const uint16_t*>(p)[off]);
}

// Four consecutive keys key .. key+3 of one mask row (row = the row's element
// offset); keys at or past S read as 0. One 16-, 8- or 4-byte load when the
// key dim is dense and the quad is aligned, else four element loads.
template <int MASK, bool F16>
__device__ __attribute__((always_inline)) inline f32x4 mask_quad(const MaskRef m, int64_t row, int key, int S) {
    constexpr int ES = MASK == 1 ? 4 : MASK == 3 ? 1 : 2;  // element bytes
    const int64_t off = row + (int64_t)key * m.sk;
    const char* a = reinterpret_cast<const char*>(m.p) + off * ES;
    if (m.sk == 1 && key + 3 < S && (reinterpret_cast<uintptr_t>(a) & (4 * ES - 1)) == 0) {
        if constexpr (MASK == 1) {
            const float4 v = *reinterpret_cast<const float4*>(a);
            return (f32x4){v.x, v.y, v.z, v.w};
        } else if constexpr (MASK == 3) {
            const uint32_t v = *reinterpret_cast<const uint32_t*>(a);
            return (f32x4){(v & 0xffu) ? 0.0f : -INFINITY, (v & 0xff00u) ? 0.0f : -INFINITY,
                           (v & 0xff0000u) ? 0.0f : -INFINITY, (v & 0xff000000u) ? 0.0f : -INFINITY};
        } else {
            const uint2 v = *reinterpret_cast<const uint2*>(a);
            auto w = [](uint32_t h) { return F16 ? f16_bits_hw((uint16_t)h) : bf16_to_f32((uint16_t)h); };
            return (f32x4){w(v.x & 0xffffu), w(v.x >> 16), w(v.y & 0xffffu), w(v.y >> 16)};
        }
    }
    const float r0 = key < S ? mask_val<MASK, F16>(m.p, off) : 0.0f;
    const float r1 = key + 1 < S ? mask_val<MASK, F16>(m.p, off + m.sk) : 0.0f;
    const float r2 = key + 2 < S ? mask_val<MASK, F16>(m.p, off + 2 * m.sk) : 0.0f;
    const float r3 = key + 3 < S ? mask_val<MASK, F16>(m.p, off + 3 * m.sk) : 0.0f;
    return (f32x4){r0, r1, r2, r3};
}



// 16 bytes per lane from a raw buffer straight into LDS (buffer_load_dwordx4
// ... lds): lane l's bytes land at lds_wave_base + 16*l, which must be
// wave-uniform.
__device__ inline void lds_direct16(buf_rsrc rsrc, uint32_t voffset, void* lds_wave_base) {
#if __HIP_DEVICE_COMPILE__
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void*)lds_wave_base, 16,
                                             voffset, 0, 0, 0);
#else
    (void)rsrc;
    (void)voffset;
    (void)lds_wave_base;
#endif
}

// v_max3_f32 (IEEE maxNum twice): written out because fmaxf on values the
// compiler cannot prove quiet costs an extra canonicalising v_max per operand
__device__ inline float max3f(float a, float b, float c) {
    float r;
    asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
    return r;
}

}  // namespace
}  // namespace tn
