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
// Per-(device, stream) array of n uint32 counters, zero when first handed out
// (cleared on the stream at allocation). A kernel that takes tickets from it
// must leave every counter at zero again when it ends.
tn_status tickets(hipStream_t stream, size_t n, uint32_t** out);
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
// The bf16 / f16 prefill at head dim 64 (flash64.hip): one workgroup per
// (batch, head, 64-query block), no split rows, nothing allocated. mk is the
// mask kind (0 none, 1 f32, 2 the input format, 3 bool) with the mask's
// element strides over (B, Hq, L, S); scale >= 0, folded into sl2 =
// scale * log2(e).
tn_status flash64_launch(hipStream_t st, bool f16, int mk, const void* mask, int64_t msb, int64_t msh, int64_t msl,
                         int64_t msk, const uint16_t* q, const uint16_t* k, const uint16_t* v, int64_t B, int64_t Hq,
                         int64_t Hkv, int64_t L, int64_t S, float sl2, int causal, uint16_t* out, float* lse);

#define TN_HIP(call)                                              \
    do {                                                          \
        hipError_t e_ = (call);                                   \
        if (e_ != hipSuccess) return ::tn::hip_fail(e_, #call);  \
    } while (0)

#define TN_TRY(call)                \
    do {                            \
        tn_status e_ = (call);      \
        if (e_ != TN_OK) return e_; \
    } while (0)

#define TN_LAUNCHED()                                              \
    do {                                                           \
        ::tn::counters().dispatches.fetch_add(1);                  \
        hipError_t e_ = hipGetLastError();                         \
        if (e_ != hipSuccess) return ::tn::hip_fail(e_, "launch"); \
    } while (0)

// ---- raw buffer access ------------------------------------------------------

// Raw buffer descriptor over `bytes` bytes at `base`: offsets at or past the
// end read as zero. Word 3 selects a 32-bit data format (any non-zero format
// enables the access); all else is zero.
#if __HIP_DEVICE_COMPILE__
typedef __amdgpu_buffer_rsrc_t buf_rsrc;
#else
typedef struct { uint32_t w[4]; } buf_rsrc;  // the host pass never emits kernel code
#endif

__device__ inline buf_rsrc make_rsrc(const void* base, uint32_t bytes) {
#if __HIP_DEVICE_COMPILE__
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
#else
    (void)base;
    (void)bytes;
    return buf_rsrc{};
#endif
}

// Unconditional loads through a descriptor: an offset at or past its end
// reads zero without a memory access, so a kernel can issue the same loads
// on every path and the compiler counts the loads in flight exactly (a load
// behind a branch makes every later wait on an older load a full wait).
template <int AUX = 0>  // cache policy bits
__device__ inline float4 buf_load_f4(buf_rsrc r, uint32_t off) {
#if __HIP_DEVICE_COMPILE__
    typedef uint32_t u4 __attribute__((ext_vector_type(4)));
    const u4 v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, AUX);
    return make_float4(__uint_as_float(v[0]), __uint_as_float(v[1]), __uint_as_float(v[2]), __uint_as_float(v[3]));
#else
    (void)r, (void)off;
    return float4{};
#endif
}
template <int AUX = 0>  // cache policy bits
__device__ inline float2 buf_load_f2(buf_rsrc r, uint32_t off) {
#if __HIP_DEVICE_COMPILE__
    typedef uint32_t u2 __attribute__((ext_vector_type(2)));
    const u2 v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, AUX);
    return make_float2(__uint_as_float(v[0]), __uint_as_float(v[1]));
#else
    (void)r, (void)off;
    return float2{};
#endif
}
template <int AUX = 0>  // cache policy bits
__device__ inline float buf_load_f(buf_rsrc r, uint32_t off) {
#if __HIP_DEVICE_COMPILE__
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, AUX));
#else
    (void)r, (void)off;
    return 0.0f;
#endif
}
constexpr uint32_t BUF_OOB = 0x80000000u;  // an offset past every descriptor of under 2^31 bytes

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

// The same two conversions through the hardware (v_cvt_f16_f32 under the
// default round-to-nearest-even mode with f16 denormals, v_cvt_f32_f16): one
// instruction each, equal to f16_from_f32 / f16_to_f32 for every input but
// the payload bits of a NaN (compared over all 2^32 floats and all 65536
// halves on gfx950).
__device__ inline float f16_round_hw(float f) { return (float)(_Float16)f; }
__device__ inline float f16_bits_hw(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }

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

// Sum of one float per thread over a 256-thread workgroup, in one fixed order
// (each 16-lane row, then rows r + (r ^ 1), then halves, then the four waves
// as (w0 + w1) + (w2 + w3)). Every kernel that normalises a row uses this, so
// a fused RMSNorm gives the bits of the separate one. `red` is 4 floats of
// LDS, used once per kernel (there is no barrier after the final reads, so a
// second call on the same `red` could overwrite it early); all threads call.
__device__ inline float block_sum256(float v, float* red);

// One DPP-routed copy of v (a VALU op, no LDS round trip). The patterns used
// here read within each 16-lane row, so every lane has a source:
//   0xB1 lane ^ 1, 0x4E lane ^ 2 (quad_perm), 0x141 the mirror lane within
//   each 8 (row_half_mirror), 0x140 the mirror lane within each 16 (row_mirror).
template <int CTRL>
__device__ inline int dpp_i(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
template <int CTRL>
__device__ inline float dpp_f(float v) {
    return __int_as_float(dpp_i<CTRL>(__float_as_int(v)));
}

// Reductions over aligned groups of 8 or 16 lanes; every lane of a group gets
// the same bits (each step combines a value with its partner's, and the
// partner computes b + a for a + b). All lanes of a group must be active.
__device__ inline float group8_max(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    return fmaxf(v, dpp_f<0x141>(v));
}
__device__ inline int group8_sum(int v) {
    v = v + dpp_i<0xB1>(v);
    v = v + dpp_i<0x4E>(v);
    return v + dpp_i<0x141>(v);
}
__device__ inline float row16_sum(float v) {
    v = v + dpp_f<0xB1>(v);
    v = v + dpp_f<0x4E>(v);
    v = v + dpp_f<0x141>(v);
    return v + dpp_f<0x140>(v);
}
__device__ inline float row16_max(float v) {
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    v = fmaxf(v, dpp_f<0x141>(v));
    return fmaxf(v, dpp_f<0x140>(v));
}

// v(l) combined with v(l ^ 16) or v(l ^ 32) through one VALU swap
// (v_permlane16_swap / v_permlane32_swap: rows 2i and 2i+1, or the two
// halves of the wave, trade places); both lanes of a pair get the same bits.
__device__ inline float xor16_sum(float v) {
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}
__device__ inline float xor16_max(float v) {
    const auto p = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}
__device__ inline float xor32_sum(float v) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(p[0]) + __uint_as_float(p[1]);
}
__device__ inline float xor32_max(float v) {
    const auto p = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(p[0]), __uint_as_float(p[1]));
}

__device__ inline float block_sum256(float v, float* red) {
    v = xor32_sum(xor16_sum(row16_sum(v)));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

// The RMSNorm scale of a row from its sum of squares: 1 / sqrt(ss/n + eps),
// sqrt then reciprocal as the reference's rsqrt (aten.rs:11112-11133).
__device__ inline float rms_scale(float ss, int n, float eps) { return 1.0f / sqrtf(ss / (float)n + eps); }

// argmax's order on (value, index): NaN first (the lower index among NaNs),
// then the larger value, then the lower index. A strict total order, so the
// winner does not depend on how a reduction pairs the candidates.
__device__ inline bool arg_before(float v, int i, float w, int j) {
    const bool nv = v != v, nw = w != w;
    if (nv || nw) return nv && (!nw || i < j);
    return v > w || (v == w && i < j);
}

// end of a decode step (state = [position, KV length, token, argmax]):
// advance the position and pick the next input token, the prompt's while
// the position is inside it, else the argmax
__device__ inline void llama_commit(int32_t* state, int32_t* tokens, int pos, int next, int cap) {
    if (pos < cap) tokens[pos] = next;
    state[0] = pos;
    state[1] = pos + 1;
    state[2] = next;
}
__device__ inline void llama_advance(int32_t* state, int32_t* tokens, const int32_t* prompt, int prompt_len,
                                     int cap) {
    const int pos = state[0] + 1;
    llama_commit(state, tokens, pos, pos < prompt_len ? prompt[pos] : state[3], cap);
}

// Input transforms a decode linear can apply while it quantises its input.
// PRO_COMBINE builds the row from split attention partials (the decode
// step's o projection).
enum LinearPrologue { PRO_NONE = 0, PRO_RMSNORM = 1, PRO_SILU = 2, PRO_COMBINE = 3 };

// Keys per workgroup of the decode step's fused attention, and the most
// splits whose merge the o projection's prologue takes on; a longer cache
// runs the split-KV attention with its own combine.
constexpr int STEP_SPLIT = 32;
constexpr int STEP_MAX_SPLITS = 16;

// Prologue operands of the decode GEMV.
struct GemvPro {
    const float* w = nullptr;  // PRO_RMSNORM weight [K]
    float eps = 0.0f;
    // PRO_RMSNORM with the SiLU epilogue: the weight is [gate; up] (2n rows)
    // and y[i] = silu(gate_i) * up_i, n outputs (linear_decode)
    int glu = 0;
    // PRO_COMBINE: partials [heads][nsplit][head_dim] and (m, l) [heads][nsplit]
    // in log2 units over splits of STEP_SPLIT keys; the KV length is
    // min(*len, cap)
    const float* part_o = nullptr;
    const float2* part_ml = nullptr;
    const int32_t* len = nullptr;
    int nsplit = 0, head_dim = 0, cap = 0;
    int head_shift = 0;  // log2(head_dim): head_dim is a power of two
    // argmax epilogue (linear_decode_argmax): every workgroup's best (value,
    // index) of y goes to arg_v/arg_i[workgroup] (GEMV_ARG_MAX_PARTS
    // entries); a one-workgroup launch then reduces them and advances the
    // decode state (state, tokens, prompt, prompt_len, cap) as llama_advance.
    float* arg_v = nullptr;
    int32_t* arg_i = nullptr;
    int32_t* state = nullptr;
    int32_t* tokens = nullptr;
    const int32_t* prompt = nullptr;
    int prompt_len = 0;
};

// Workgroups of an argmax-epilogue launch at most, each writing one partial
// (the GEMV is persistent over row tiles beyond this).
constexpr int GEMV_ARG_MAX_PARTS = 2048;

// One f32 row through a q4_0 linear (qlinear.hip), y[n] = Q8_0(pro(x)) . W^T
// (+ resid[n]): pro is a LinearPrologue (PRO_RMSNORM scales by po.w with
// po.eps; PRO_SILU reads x as [gate | up], 2k floats; PRO_COMBINE ignores x
// and merges po's attention partials). With PRO_RMSNORM and po.glu the
// weight is [gate; up], 2n rows, and y[i] = silu(gate_i) * up_i (no resid).
// Bit-identical to the separate ops in sequence. y may alias resid, not x.
// k <= LINEAR_DECODE_MAX_K.
constexpr int64_t LINEAR_DECODE_MAX_K = 24576;  // 768 blocks: one per (row, block) item of the workgroup
tn_status linear_decode(hipStream_t st, const float* x, int64_t k, int pro, const GemvPro& po, const uint8_t* qs,
                        const uint16_t* d, int64_t n, const float* resid, float* y);
// The decode step's last linear: y = Q4(rmsnorm(x, po.w)) as linear_decode
// with PRO_RMSNORM, with per-workgroup argmax partials of y, then one
// workgroup reducing them and advancing the state (po's argmax fields).
// TN_ENOTIMPL when the activation row does not fit the GEMV.
tn_status linear_decode_argmax(hipStream_t st, const float* x, int64_t k, const GemvPro& po, const uint8_t* qs,
                               const uint16_t* d, int64_t n, float* y);
// A prompt's projection, y = Q4_0 linear of m activation rows (f32, 16-byte
// aligned) through the q4 GEMM, bit-identical to the separate ops: xm picks
// where row r's k activations come from (XM_ROWS: x[r][0..k); XM_GLU:
// silu(gate) * up of x's [m][2k] rows, as tn_silu_mul; XM_HEADS: an
// attention output [k / hd][m][hd], as the copy to token rows), and a
// non-null resid is added to the product as tn_add does (resid may be y).
constexpr int XM_ROWS = 0, XM_GLU = 1, XM_HEADS = 2;
tn_status linear_prefill(hipStream_t st, const float* x, int64_t m, int64_t k, int xm, int hd, const uint8_t* qs,
                         const uint16_t* d, int64_t n, const float* resid, float* y);

}  // namespace tn
