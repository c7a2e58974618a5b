// GGML q4_0 on gfx950: upload/repack, quantise, dequantise, and the
// quantised linear (decode GEMV and prefill MFMA GEMM).
//
// Arithmetic contract (candle-core/src/quantized/k_quants.rs, the reference's
// vendored candle): every output is
//     sumf = 0; for b in blocks: sumf += ((float)S_b * d_w[b]) * d_x[b]
// where S_b is the exact integer dot of the weight's Q4_0 codes (nib - 8) and
// the activation's Q8_0 codes (vec_dot_unopt, k_quants.rs:312-329), and the
// activation row is quantised by BlockQ8_0::from_float (k_quants.rs:676-705).
// The integer dot is exact in any order, and every kernel below performs the
// float steps in exactly that order with separate roundings (the library is
// built with -ffp-contract=off), so results are bit-identical to the
// reference's x86_64 scalar path for every row count.
#include "tn_common.h"

namespace tn {
namespace {

constexpr int QK = 32;

// ---- Rust cast semantics ---------------------------------------------------

__device__ inline int sat_i8(float v) {  // `f as i8`
    if (v != v) return 0;
    if (v >= 127.0f) return 127;
    if (v <= -128.0f) return -128;
    return (int)v;
}

__device__ inline int sat_u8(float v) {  // `f as u8`
    if (v != v) return 0;
    if (v >= 255.0f) return 255;
    if (v <= 0.0f) return 0;
    return (int)v;
}

template <typename XT>
__device__ inline float load_x(const XT* p);
template <>
__device__ inline float load_x<float>(const float* p) { return *p; }
template <>
__device__ inline float load_x<uint16_t>(const uint16_t* p) { return bf16_to_f32(*p); }

// Q8_0 of one 32-element block held one element per lane of a 32-lane group
// (BlockQ8_0::from_float, k_quants.rs:676-705): amax over the block, d =
// amax/127 (IEEE division), id = 1/d or 0, q = (round-half-away(x*id)) as i8.
// Returns q; *dx gets f32(f16(d)), the scale the dot product uses.
__device__ inline int q8_0_lane(float v, float* dx) {
    float a = fabsf(v);
#pragma unroll
    for (int off = 16; off >= 1; off >>= 1) a = fmaxf(a, __shfl_xor(a, off, 32));
    float d = a / 127.0f;
    float id = (d != 0.0f) ? 1.0f / d : 0.0f;
    *dx = f16_to_f32(f16_from_f32(d));
    return sat_i8(roundf(v * id));
}

// ---- layout conversion --------------------------------------------------------

__global__ void k_from_blob(const uint8_t* __restrict__ blob, int64_t nblocks, uint8_t* __restrict__ qs,
                            uint16_t* __restrict__ d) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks) return;
    const uint8_t* s = blob + i * 18;
    d[i] = (uint16_t)(s[0] | (s[1] << 8));
    uint32_t w[4];
#pragma unroll
    for (int j = 0; j < 4; j++)
        w[j] = (uint32_t)s[2 + 4 * j] | ((uint32_t)s[3 + 4 * j] << 8) | ((uint32_t)s[4 + 4 * j] << 16) |
               ((uint32_t)s[5 + 4 * j] << 24);
    *reinterpret_cast<uint4*>(qs + i * 16) = make_uint4(w[0], w[1], w[2], w[3]);
}

__global__ void k_to_blob(const uint8_t* __restrict__ qs, const uint16_t* __restrict__ d, int64_t nblocks,
                          uint8_t* __restrict__ blob) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks) return;
    uint8_t* o = blob + i * 18;
    uint16_t h = d[i];
    o[0] = (uint8_t)(h & 0xff);
    o[1] = (uint8_t)(h >> 8);
    uint4 w = *reinterpret_cast<const uint4*>(qs + i * 16);
    uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int j = 0; j < 16; j++) o[2 + j] = (uint8_t)(ws[j >> 2] >> (8 * (j & 3)));
}

// BlockQ4_0::from_float (k_quants.rs:241-277), one thread per block.
__global__ void k_quantize_w(const float* __restrict__ w, int64_t nblocks, uint8_t* __restrict__ qs,
                             uint16_t* __restrict__ d) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks) return;
    const float* xs = w + i * QK;
    float v[QK];
#pragma unroll
    for (int j = 0; j < QK; j += 4) {
        float4 t = *reinterpret_cast<const float4*>(xs + j);
        v[j] = t.x; v[j + 1] = t.y; v[j + 2] = t.z; v[j + 3] = t.w;
    }
    float amax = 0.0f, mx = 0.0f;
#pragma unroll
    for (int j = 0; j < QK; j++) {
        float a = fabsf(v[j]);
        if (amax < a) { amax = a; mx = v[j]; }  // first of the largest |x|, sign kept
    }
    float dd = mx / -8.0f;
    float id = (dd != 0.0f) ? 1.0f / dd : 0.0f;
    d[i] = f16_from_f32(dd);
    uint32_t out[4] = {0, 0, 0, 0};
#pragma unroll
    for (int j = 0; j < QK / 2; j++) {
        int q0 = sat_u8(v[j] * id + 8.5f);
        int q1 = sat_u8(v[j + QK / 2] * id + 8.5f);
        q0 = q0 < 15 ? q0 : 15;
        q1 = q1 < 15 ? q1 : 15;
        out[j >> 2] |= (uint32_t)(q0 | (q1 << 4)) << (8 * (j & 3));
    }
    *reinterpret_cast<uint4*>(qs + i * 16) = make_uint4(out[0], out[1], out[2], out[3]);
}

// BlockQ4_0::to_float (k_quants.rs:219-239): (nib - 8) as f32 * f32(d), exact.
__global__ void k_dequantize(const uint8_t* __restrict__ qs, const uint16_t* __restrict__ d, int64_t nblocks,
                             float* __restrict__ out) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks) return;
    float s = f16_to_f32(d[i]);
    uint4 w = *reinterpret_cast<const uint4*>(qs + i * 16);
    uint32_t ws[4] = {w.x, w.y, w.z, w.w};
    float lo[16], hi[16];
#pragma unroll
    for (int j = 0; j < 16; j++) {
        uint32_t byte = (ws[j >> 2] >> (8 * (j & 3))) & 0xffu;
        lo[j] = (float)((int)(byte & 0xf) - 8) * s;
        hi[j] = (float)((int)(byte >> 4) - 8) * s;
    }
    float4* o = reinterpret_cast<float4*>(out + i * QK);
#pragma unroll
    for (int j = 0; j < 4; j++) {
        o[j] = make_float4(lo[4 * j], lo[4 * j + 1], lo[4 * j + 2], lo[4 * j + 3]);
        o[4 + j] = make_float4(hi[4 * j], hi[4 * j + 1], hi[4 * j + 2], hi[4 * j + 3]);
    }
}

// ---- decode GEMV (m <= GEMV_MAX_M) ---------------------------------------------
//
// One workgroup owns `rows` consecutive weight rows. Phase 1 quantises the MR
// activation rows into LDS (every workgroup repeats this: x is a few KB and
// L2-resident). Phase 2 streams the weight: the (row, block) items of the
// workgroup are a contiguous range of the qs plane, so consecutive lanes issue
// consecutive 16-byte loads; each item's exact integer dot is 8 v_dot4_i32_i8
// on the unsigned nibbles minus 8 * sum(x codes), and its scaled term goes to
// LDS. Phase 3 adds each output's terms in block order.

constexpr int GEMV_THREADS = 256;
constexpr int GEMV_ITEMS = 4;  // (row, block) items per thread
constexpr int GEMV_MAX_M = 4;

__device__ inline int dot_block(uint4 w, const int* __restrict__ xw) {
    // xw: the 32 int8 codes of the block as 8 dwords, natural element order.
    // w dword j holds bytes 4j..4j+3: low nibbles = elements 4j..4j+3, high
    // nibbles = elements 16+4j..16+4j+3.
    int s = 0;
    s = __builtin_amdgcn_sdot4((int)(w.x & 0x0f0f0f0fu), xw[0], s, false);
    s = __builtin_amdgcn_sdot4((int)((w.x >> 4) & 0x0f0f0f0fu), xw[4], s, false);
    s = __builtin_amdgcn_sdot4((int)(w.y & 0x0f0f0f0fu), xw[1], s, false);
    s = __builtin_amdgcn_sdot4((int)((w.y >> 4) & 0x0f0f0f0fu), xw[5], s, false);
    s = __builtin_amdgcn_sdot4((int)(w.z & 0x0f0f0f0fu), xw[2], s, false);
    s = __builtin_amdgcn_sdot4((int)((w.z >> 4) & 0x0f0f0f0fu), xw[6], s, false);
    s = __builtin_amdgcn_sdot4((int)(w.w & 0x0f0f0f0fu), xw[3], s, false);
    s = __builtin_amdgcn_sdot4((int)((w.w >> 4) & 0x0f0f0f0fu), xw[7], s, false);
    return s;
}

template <int MR, typename XT>
__global__ __launch_bounds__(GEMV_THREADS) void k_gemv(const XT* __restrict__ x, int K, int nb,
                                                     const uint8_t* __restrict__ qs,
                                                     const uint16_t* __restrict__ dw, int N, int rows,
                                                     const float* __restrict__ bias, void* __restrict__ y,
                                                     int y_bf16) {
    extern __shared__ __align__(16) char smem[];
    int* xq = reinterpret_cast<int*>(smem);               // [MR][K/4] packed int8 codes
    float* dxs = reinterpret_cast<float*>(xq + MR * (K / 4));  // [MR][nb]
    int* sxs = reinterpret_cast<int*>(dxs + MR * nb);     // [MR][nb]
    float* terms = reinterpret_cast<float*>(sxs + MR * nb);  // [rows][MR][nb]
    const int tid = threadIdx.x;

    // phase 1: Q8_0 of the MR activation rows, one 32-lane group per block
    {
        const int grp = tid >> 5, lane = tid & 31;
        int8_t* xb = reinterpret_cast<int8_t*>(xq);
        for (int blk = grp; blk < MR * nb; blk += GEMV_THREADS / 32) {
            const int mr = blk / nb, b = blk - mr * nb;
            float v = load_x<XT>(x + (int64_t)mr * K + b * QK + lane);
            float dx;
            int q = q8_0_lane(v, &dx);
            xb[mr * K + b * QK + lane] = (int8_t)q;
            int s = q;
#pragma unroll
            for (int off = 16; off >= 1; off >>= 1) s += __shfl_xor(s, off, 32);
            if (lane == 0) {
                dxs[mr * nb + b] = dx;
                sxs[mr * nb + b] = s;
            }
        }
    }
    __syncthreads();

    // phase 2: stream the weight
    const int64_t row0 = (int64_t)blockIdx.x * rows;
    const int nrows = (int)((N - row0) < rows ? (N - row0) : rows);
    const int total = nrows * nb;
    const uint8_t* qbase = qs + row0 * nb * 16;
    const uint16_t* dbase = dw + row0 * nb;
    uint4 wv[GEMV_ITEMS];
    uint16_t dv[GEMV_ITEMS];
#pragma unroll
    for (int it = 0; it < GEMV_ITEMS; it++) {
        const int g = tid + it * GEMV_THREADS;
        if (g < total) {
            wv[it] = reinterpret_cast<const uint4*>(qbase)[g];
            dv[it] = dbase[g];
        }
    }
#pragma unroll
    for (int it = 0; it < GEMV_ITEMS; it++) {
        const int g = tid + it * GEMV_THREADS;
        if (g < total) {
            const int r = g / nb, b = g - r * nb;
            const float dwf = f16_to_f32(dv[it]);
#pragma unroll
            for (int mr = 0; mr < MR; mr++) {
                int s = dot_block(wv[it], xq + mr * (K / 4) + b * 8) - 8 * sxs[mr * nb + b];
                float t = (float)s * dwf;
                t = t * dxs[mr * nb + b];
                terms[(r * MR + mr) * nb + b] = t;
            }
        }
    }
    __syncthreads();

    // phase 3: each output's terms in block order
    for (int o = tid; o < nrows * MR; o += GEMV_THREADS) {
        const int r = o / MR, mr = o - r * MR;
        const float* tr = terms + (r * MR + mr) * nb;
        float acc = 0.0f;
        for (int b = 0; b < nb; b++) acc = acc + tr[b];
        const int64_t n = row0 + r;
        if (bias) acc = acc + bias[n];
        if (y_bf16)
            reinterpret_cast<uint16_t*>(y)[(int64_t)mr * N + n] = bf16_from_f32(acc);
        else
            reinterpret_cast<float*>(y)[(int64_t)mr * N + n] = acc;
    }
}

// ---- prefill GEMM on MFMA ---------------------------------------------------------
//
// Prepass: every activation row is quantised to Q8_0 once, into bf16 codes
// (|q| <= 127 is exact in bf16) laid out per block in the order the MFMA
// operand wants, plus the f32 block scales transposed [nb][M_pad].
//
// Main kernel: a 128x128 output tile per workgroup, four waves as 2x2, each
// wave 64x64 = 4x4 tiles of v_mfma_f32_16x16x32_bf16. The K loop walks blocks
// in order. One MFMA over one 32-element block, started from a zero
// accumulator, yields the block's integer dot exactly: products are at most
// 8*127 and the 32-term sum at most 32512 < 2^24. The weight nibbles are
// widened to bf16 codes (nib - 8) once per workgroup in LDS.
//
// K-slot order: MFMA lane group g (lanes 16g..16g+15) holds 8 of the 32 block
// elements, {4g..4g+3, 16+4g..16+4g+3}: the low and high nibbles of weight
// bytes 4g..4g+3. The activation codes are stored in the same order, so the
// two operands agree element for element.

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int GM_BM = 128, GM_BN = 128, GM_THREADS = 256;

__device__ inline int kslot_of_element(int e) {  // element (0..31) -> K slot
    return e < 16 ? 8 * (e >> 2) + (e & 3) : 8 * ((e - 16) >> 2) + 4 + (e & 3);
}

template <typename XT>
__global__ __launch_bounds__(256) void k_q8_rows(const XT* __restrict__ x, int M, int M_pad, int K, int nb,
                                               uint16_t* __restrict__ xc, float* __restrict__ dxT) {
    // one 32-lane group per (row, block); rows >= M become zero codes, zero scale
    const int64_t blk = (int64_t)blockIdx.x * (blockDim.x >> 5) + (threadIdx.x >> 5);
    const int lane = threadIdx.x & 31;
    if (blk >= (int64_t)M_pad * nb) return;
    const int row = (int)(blk / nb), b = (int)(blk - (int64_t)row * nb);
    float dx = 0.0f;
    int q = 0;
    if (row < M) {
        float v = load_x<XT>(x + (int64_t)row * K + b * QK + lane);
        q = q8_0_lane(v, &dx);
    }
    xc[blk * QK + kslot_of_element(lane)] = (uint16_t)(__builtin_bit_cast(uint32_t, (float)q) >> 16);
    if (lane == 0) dxT[(int64_t)b * M_pad + row] = dx;
}

__device__ inline uint32_t pack_bf16_codes(uint32_t n0, uint32_t n1) {
    // two nibbles -> bf16(n0 - 8) | bf16(n1 - 8) << 16 (small integers: exact,
    // the low 16 bits of the f32 are zero)
    uint32_t a = __builtin_bit_cast(uint32_t, (float)((int)n0 - 8));
    uint32_t b = __builtin_bit_cast(uint32_t, (float)((int)n1 - 8));
    return (a >> 16) | (b & 0xffff0000u);
}

__global__ __launch_bounds__(GM_THREADS) void k_gemm(const uint16_t* __restrict__ xc,
                                                    const float* __restrict__ dxT, int M, int M_pad, int nb,
                                                    const uint8_t* __restrict__ qs,
                                                    const uint16_t* __restrict__ dw, int N,
                                                    const float* __restrict__ bias, void* __restrict__ y,
                                                    int y_bf16) {
    // LDS: A codes [128][32] bf16 (64 B rows), B codes [128][32] bf16, dx[128], dw[128]
    __shared__ __align__(16) uint16_t sA[GM_BM * QK];
    __shared__ __align__(16) uint16_t sB[GM_BN * QK];
    __shared__ float sdx[GM_BM];
    __shared__ float sdw[GM_BN];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;  // wave's 64x64 sub-tile
    const int m0 = blockIdx.y * GM_BM, n0 = blockIdx.x * GM_BN;
    const int lrow = lane & 15, lgrp = lane >> 4;

    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};

    for (int b = 0; b < nb; b++) {
        // stage A: 128 rows x 64 B = 512 chunks of 16 B, two per thread
#pragma unroll
        for (int c = 0; c < 2; c++) {
            const int chunk = tid + c * GM_THREADS;
            const int r = chunk >> 2, part = chunk & 3;
            const uint4 v = *reinterpret_cast<const uint4*>(xc + ((int64_t)(m0 + r) * nb + b) * QK + part * 8);
            *reinterpret_cast<uint4*>(sA + r * QK + part * 8) = v;
        }
        // stage B: threads 0..127 widen one column's block; 128..255 load scales
        if (tid < GM_BN) {
            const int n = n0 + tid;
            uint4 w = make_uint4(0x88888888u, 0x88888888u, 0x88888888u, 0x88888888u);
            if (n < N) w = *reinterpret_cast<const uint4*>(qs + ((int64_t)n * nb + b) * 16);
            const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
            uint32_t out[16];
#pragma unroll
            for (int g = 0; g < 4; g++) {
                const uint32_t v = ws[g];
                // K slots 8g..8g+3 <- low nibbles of bytes 0..3, 8g+4..8g+7 <- high nibbles
                out[4 * g + 0] = pack_bf16_codes(v & 0xf, (v >> 8) & 0xf);
                out[4 * g + 1] = pack_bf16_codes((v >> 16) & 0xf, (v >> 24) & 0xf);
                out[4 * g + 2] = pack_bf16_codes((v >> 4) & 0xf, (v >> 12) & 0xf);
                out[4 * g + 3] = pack_bf16_codes((v >> 20) & 0xf, (v >> 28) & 0xf);
            }
            uint4* dst = reinterpret_cast<uint4*>(sB + tid * QK);
#pragma unroll
            for (int q = 0; q < 4; q++) dst[q] = make_uint4(out[4 * q], out[4 * q + 1], out[4 * q + 2], out[4 * q + 3]);
        } else {
            const int t = tid - GM_BN;  // 0..127
            const int n = n0 + t;
            sdw[t] = (n < N) ? f16_to_f32(dw[(int64_t)n * nb + b]) : 0.0f;
            sdx[t] = dxT[(int64_t)b * M_pad + m0 + t];
        }
        __syncthreads();

        bf16x8 afr[4], bfr[4];
#pragma unroll
        for (int i = 0; i < 4; i++)
            afr[i] = *reinterpret_cast<const bf16x8*>(sA + (wm * 64 + i * 16 + lrow) * QK + lgrp * 8);
#pragma unroll
        for (int j = 0; j < 4; j++)
            bfr[j] = *reinterpret_cast<const bf16x8*>(sB + (wn * 64 + j * 16 + lrow) * QK + lgrp * 8);
        float dwv[4];
        f32x4 dxv[4];
#pragma unroll
        for (int j = 0; j < 4; j++) dwv[j] = sdw[wn * 64 + j * 16 + lrow];
#pragma unroll
        for (int i = 0; i < 4; i++) dxv[i] = *reinterpret_cast<const f32x4*>(sdx + wm * 64 + i * 16 + lgrp * 4);

#pragma unroll
        for (int i = 0; i < 4; i++) {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const f32x4 zero = {0.f, 0.f, 0.f, 0.f};
                // C[row][col]: col = lane & 15 (weight column), row = 4*(lane>>4) + r
                // A = activation rows, B = weight columns
                f32x4 s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(afr[i], bfr[j], zero, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    float t = s[r] * dwv[j];
                    t = t * dxv[i][r];
                    acc[i][j][r] = acc[i][j][r] + t;
                }
            }
        }
        __syncthreads();
    }

#pragma unroll
    for (int i = 0; i < 4; i++) {
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int n = n0 + wn * 64 + j * 16 + lrow;
            if (n >= N) continue;
            const float bv = bias ? bias[n] : 0.0f;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = m0 + wm * 64 + i * 16 + lgrp * 4 + r;
                if (m >= M) continue;
                float v = acc[i][j][r];
                if (bias) v = v + bv;
                if (y_bf16)
                    reinterpret_cast<uint16_t*>(y)[(int64_t)m * N + n] = bf16_from_f32(v);
                else
                    reinterpret_cast<float*>(y)[(int64_t)m * N + n] = v;
            }
        }
    }
}

tn_status check_weight(const char* op, int64_t n, int64_t k) {
    if (n < 0 || k <= 0 || k % QK != 0) {
        char buf[384];
        std::snprintf(buf, sizeof buf,
                      "%s: q4_0 stores 32 elements per block, so it must have their last dim divisible by "
                      "block size -- got %lld, which is not a multiple of 32 (shape [%lld, %lld])",
                      op, (long long)k, (long long)n, (long long)k);
        return fail(TN_ENOTIMPL, buf);
    }
    if (n * (k / QK) > ((int64_t)1 << 40)) return fail(TN_EVALUE, std::string(op) + ": weight too large");
    return TN_OK;
}

template <int MR, typename XT>
tn_status launch_gemv(hipStream_t st, const XT* x, int K, const uint8_t* qs, const uint16_t* dw, int N,
                      const float* bias, void* y, int y_bf16) {
    const int nb = K / QK;
    int rows = (GEMV_THREADS * GEMV_ITEMS) / nb;
    if (rows < 1) rows = 1;
    if (rows > N) rows = N;
    size_t lds = (size_t)MR * K + (size_t)MR * nb * 8 + (size_t)rows * MR * nb * 4;
    while (rows > 1 && lds > 64 * 1024) {
        rows >>= 1;
        lds = (size_t)MR * K + (size_t)MR * nb * 8 + (size_t)rows * MR * nb * 4;
    }
    if (lds > 64 * 1024) return TN_ENOTIMPL;  // caller chunks rows / refuses
    // (row, block) items must fit GEMV_ITEMS per thread
    if ((int64_t)rows * nb > GEMV_THREADS * GEMV_ITEMS) return TN_ENOTIMPL;
    const unsigned grid = (unsigned)cdiv(N, rows);
    hipLaunchKernelGGL((k_gemv<MR, XT>), dim3(grid), dim3(GEMV_THREADS), lds, st, x, K, nb, qs, dw, N, rows,
                       bias, y, y_bf16);
    TN_LAUNCHED();
    return TN_OK;
}

template <typename XT>
tn_status linear_impl(hipStream_t st, const XT* x, int64_t m, int64_t k, const uint8_t* qs, const uint16_t* d,
                      int64_t n, const float* bias, void* y, int y_bf16) {
    if (m == 0 || n == 0) return TN_OK;
    const int nb = (int)(k / QK);
    const size_t ysz = y_bf16 ? 2 : 4;
    if (m <= GEMV_MAX_M && nb <= GEMV_THREADS * GEMV_ITEMS) {
        // decode: GEMV in chunks of up to 4 rows of x (a row's result does not
        // depend on the chunking: every output is the same recurrence)
        int64_t r = 0;
        tn_status s = TN_OK;
        while (r < m && s == TN_OK) {
            const int64_t c = (m - r) >= 4 ? 4 : (m - r);
            const XT* xr = x + r * k;
            void* yr = static_cast<char*>(y) + r * n * ysz;
            switch (c) {
                case 4: s = launch_gemv<4, XT>(st, xr, (int)k, qs, d, (int)n, bias, yr, y_bf16); break;
                case 3: s = launch_gemv<3, XT>(st, xr, (int)k, qs, d, (int)n, bias, yr, y_bf16); break;
                case 2: s = launch_gemv<2, XT>(st, xr, (int)k, qs, d, (int)n, bias, yr, y_bf16); break;
                default: s = launch_gemv<1, XT>(st, xr, (int)k, qs, d, (int)n, bias, yr, y_bf16); break;
            }
            r += c;
        }
        if (s == TN_OK) return TN_OK;
        if (s != TN_ENOTIMPL) return s;
        // too large for the LDS-resident GEMV: fall through to the GEMM kernels,
        // which compute the identical recurrence
    }
    const int64_t M_pad = cdiv(m, GM_BM) * GM_BM;
    if (M_pad > INT32_MAX || n > INT32_MAX) return fail(TN_EVALUE, "torch._C._quantized_linear: shape too large");
    const size_t xc_bytes = (size_t)M_pad * k * 2;
    const size_t dx_bytes = (size_t)M_pad * nb * 4;
    void* ws = nullptr;
    tn_status s = workspace(st, xc_bytes + dx_bytes, &ws);
    if (s != TN_OK) return s;
    uint16_t* xc = static_cast<uint16_t*>(ws);
    float* dxT = reinterpret_cast<float*>(static_cast<char*>(ws) + xc_bytes);
    {
        const int64_t blocks = M_pad * nb;
        const unsigned grid = (unsigned)cdiv(blocks, 8);
        hipLaunchKernelGGL((k_q8_rows<XT>), dim3(grid), dim3(256), 0, st, x, (int)m, (int)M_pad, (int)k, nb, xc,
                           dxT);
        TN_LAUNCHED();
    }
    dim3 grid((unsigned)cdiv(n, GM_BN), (unsigned)(M_pad / GM_BM));
    hipLaunchKernelGGL(k_gemm, grid, dim3(GM_THREADS), 0, st, xc, dxT, (int)m, (int)M_pad, nb, qs, d, (int)n, bias,
                       y, y_bf16);
    TN_LAUNCHED();
    return TN_OK;
}

}  // namespace
}  // namespace tn

using namespace tn;

extern "C" {

tn_status tn_q4_0_from_blob(void* stream, const uint8_t* blob, int64_t n, int64_t k, uint8_t* qs, uint16_t* d) {
    tn_status s = check_weight("torch._C._quantized_to", n, k);
    if (s != TN_OK) return s;
    const int64_t nblocks = n * (k / QK);
    if (!nblocks) return TN_OK;
    if (!blob || !qs || !d) return fail(TN_EVALUE, "tn_q4_0_from_blob: null pointer");
    hipLaunchKernelGGL(k_from_blob, dim3((unsigned)cdiv(nblocks, 256)), dim3(256), 0, (hipStream_t)stream, blob,
                       nblocks, qs, d);
    TN_LAUNCHED();
    return TN_OK;
}

tn_status tn_q4_0_to_blob(void* stream, const uint8_t* qs, const uint16_t* d, int64_t n, int64_t k, uint8_t* blob) {
    tn_status s = check_weight("torch._C._quantized_blob", n, k);
    if (s != TN_OK) return s;
    const int64_t nblocks = n * (k / QK);
    if (!nblocks) return TN_OK;
    if (!blob || !qs || !d) return fail(TN_EVALUE, "tn_q4_0_to_blob: null pointer");
    hipLaunchKernelGGL(k_to_blob, dim3((unsigned)cdiv(nblocks, 256)), dim3(256), 0, (hipStream_t)stream, qs, d,
                       nblocks, blob);
    TN_LAUNCHED();
    return TN_OK;
}

tn_status tn_q4_0_quantize(void* stream, const float* w, int64_t n, int64_t k, uint8_t* qs, uint16_t* d) {
    tn_status s = check_weight("torch._C._quantize", n, k);
    if (s != TN_OK) return s;
    const int64_t nblocks = n * (k / QK);
    if (!nblocks) return TN_OK;
    if (!w || !qs || !d) return fail(TN_EVALUE, "tn_q4_0_quantize: null pointer");
    hipLaunchKernelGGL(k_quantize_w, dim3((unsigned)cdiv(nblocks, 256)), dim3(256), 0, (hipStream_t)stream, w,
                       nblocks, qs, d);
    TN_LAUNCHED();
    return TN_OK;
}

tn_status tn_q4_0_dequantize(void* stream, const uint8_t* qs, const uint16_t* d, int64_t n, int64_t k, float* out) {
    tn_status s = check_weight("torch._C._dequantize", n, k);
    if (s != TN_OK) return s;
    const int64_t nblocks = n * (k / QK);
    if (!nblocks) return TN_OK;
    if (!out || !qs || !d) return fail(TN_EVALUE, "tn_q4_0_dequantize: null pointer");
    hipLaunchKernelGGL(k_dequantize, dim3((unsigned)cdiv(nblocks, 256)), dim3(256), 0, (hipStream_t)stream, qs, d,
                       nblocks, out);
    TN_LAUNCHED();
    return TN_OK;
}

tn_status tn_q4_0_linear(void* stream, const void* x, int x_dtype, int64_t m, int64_t k, const uint8_t* qs,
                         const uint16_t* d, int64_t n, const float* bias, void* y, int y_dtype) {
    const char* OP = "torch._C._quantized_linear";
    if (x_dtype != TN_F32 && x_dtype != TN_BF16)
        return fail(TN_ENOTIMPL, std::string(OP) +
                                     ": the activation must be float32 (or bfloat16, widened exactly in-kernel) "
                                     "on the hip device");
    if (y_dtype != TN_F32 && y_dtype != TN_BF16)
        return fail(TN_ENOTIMPL, std::string(OP) + ": the output must be float32 or bfloat16");
    if (k <= 0 || k % QK != 0 || m < 0 || n < 0) {
        char buf[256];
        std::snprintf(buf, sizeof buf, "%s: mat1 and mat2 shapes cannot be multiplied ([%lld, %lld] and %lldx%lld)",
                      OP, (long long)m, (long long)k, (long long)k, (long long)n);
        return fail(TN_EINVAL, buf);
    }
    if (m > 0 && n > 0 && (!x || !qs || !d || !y)) return fail(TN_EVALUE, std::string(OP) + ": null pointer");
    hipStream_t st = (hipStream_t)stream;
    const int yb = y_dtype == TN_BF16;
    if (x_dtype == TN_F32)
        return linear_impl<float>(st, static_cast<const float*>(x), m, k, qs, d, n, bias, y, yb);
    return linear_impl<uint16_t>(st, static_cast<const uint16_t*>(x), m, k, qs, d, n, bias, y, yb);
}

}  // extern "C"
