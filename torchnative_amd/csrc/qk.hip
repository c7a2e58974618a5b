// GGML q4_k weights on gfx950: upload/repack, the Q4_K writer, dequantise,
// and the quantised linear, bit-identical to the reference's x86_64 path.
//
// Arithmetic contract (candle-core/src/quantized/k_quants.rs, the reference's
// vendored candle). The activation row is quantised to Q8_K per 256 elements
// (BlockQ8K::from_float, k_quants.rs:2375-2413) and each output is
// BlockQ4K::vec_dot_unopt (k_quants.rs:1478-1558):
//     per super-block: aux32[l] = sum_j sc_j * sum_g q8[32j+8g+l] * nib[32j+8g+l]  (exact i32)
//                      sumi     = sum_j bsums[j] * m_{j/2}                         (exact i32)
//                      sums[l] += (d_w * d_x) * aux32[l]      (f32, l = 0..7)
//                      sumf    -= (dmin_w * d_x) * sumi       (f32)
//     result = sumf + (((sums[0] + sums[1]) + ...) + sums[7])
// The integer parts are exact in any order; the float steps below are done in
// exactly that order, one rounding each (-ffp-contract=off).
//
// Device layout. A super-block keeps its 144 bytes and its place (row-major,
// 144-byte stride, so every super-block is 16-byte aligned): f16 d, f16 dmin,
// the 12 packed 6-bit scale/min bytes, then the 128 nibble bytes in four
// 32-byte chunks. Within a chunk, byte 8g + l of the GGML block (g = 0..3,
// l = 0..7) is stored at 4l + g, so dword l holds the four elements of
// position l mod 8 -- exactly the operands of one aux32[l] term. The low
// nibbles of chunk c are sub-block 2c, the high nibbles sub-block 2c + 1.
// tn_q4_k_from_blob / _to_blob convert byte for byte.
#include "tn_common.h"

namespace tn {
namespace {

constexpr int QKK = 256;
constexpr int QK4K_BYTES = 144;

__device__ inline int sat_i8k(float v) {  // `v.clamp(-128, 127) as i8`, NaN -> 0 (selects, not branches)
    const int q = (int)fminf(fmaxf(v, -128.0f), 127.0f);
    return v != v ? 0 : q;
}

// llama.cpp's nearest_int (candle utils.rs:292-295): ties to even.
__device__ inline int nearest_int_even(float f) {
    const float v = f + 12582912.0f;
    return (int)(__float_as_uint(v) & 0x007fffffu) - 0x00400000;
}

__device__ inline void scale_min_k4(int j, const uint8_t* q, int* sc, int* m) {  // utils.rs:50-60
    if (j < 4) {
        *sc = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *sc = (q[j + 4] & 0x0f) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

// a 32-byte chunk as 8 dwords: natural byte order <-> position-major order
__device__ inline void chunk_transpose(const uint32_t* in, uint32_t* out, bool to_device) {
    uint8_t b[32], t[32];
#pragma unroll
    for (int i = 0; i < 32; i++) b[i] = (uint8_t)(in[i >> 2] >> (8 * (i & 3)));
#pragma unroll
    for (int g = 0; g < 4; g++)
#pragma unroll
        for (int l = 0; l < 8; l++) {
            if (to_device)
                t[4 * l + g] = b[8 * g + l];
            else
                t[8 * g + l] = b[4 * l + g];
        }
#pragma unroll
    for (int i = 0; i < 8; i++)
        out[i] = (uint32_t)t[4 * i] | ((uint32_t)t[4 * i + 1] << 8) | ((uint32_t)t[4 * i + 2] << 16) |
                 ((uint32_t)t[4 * i + 3] << 24);
}

// ---- layout conversion (one thread per super-block) ---------------------------

template <bool TO_DEVICE>
__global__ void k_qk_repack(const uint8_t* __restrict__ src, int64_t nsb, uint8_t* __restrict__ dst) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nsb) return;
    const uint4* s = reinterpret_cast<const uint4*>(src + i * QK4K_BYTES);
    uint4* o = reinterpret_cast<uint4*>(dst + i * QK4K_BYTES);
    o[0] = s[0];
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const uint4 a = s[1 + 2 * c], b = s[2 + 2 * c];
        const uint32_t in[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        uint32_t out[8];
        chunk_transpose(in, out, TO_DEVICE);
        o[1 + 2 * c] = make_uint4(out[0], out[1], out[2], out[3]);
        o[2 + 2 * c] = make_uint4(out[4], out[5], out[6], out[7]);
    }
}

// ---- dequantise: BlockQ4K::to_float (k_quants.rs:1722-1746) ----------------------
// Eight threads per super-block, one per 32-element sub-block.

__global__ void k_qk_dequantize(const uint8_t* __restrict__ w, int64_t nsb, float* __restrict__ out) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nsb * 8) return;
    const int64_t sb = t >> 3;
    const int j = (int)(t & 7), c = j >> 1;
    const uint8_t* blk = w + sb * QK4K_BYTES;
    const float d = f16_to_f32((uint16_t)(blk[0] | (blk[1] << 8)));
    const float dmin = f16_to_f32((uint16_t)(blk[2] | (blk[3] << 8)));
    int sc, m;
    scale_min_k4(j, blk + 4, &sc, &m);
    const float d1 = d * (float)sc, m1 = dmin * (float)m;
    const uint32_t* q = reinterpret_cast<const uint32_t*>(blk + 16 + 32 * c);
    float v[32];
#pragma unroll
    for (int l = 0; l < 8; l++) {
        const uint32_t dw = q[l];
#pragma unroll
        for (int g = 0; g < 4; g++) {
            const uint32_t byte = (dw >> (8 * g)) & 0xffu;
            const uint32_t nib = (j & 1) ? (byte >> 4) : (byte & 0x0fu);
            v[8 * g + l] = d1 * (float)nib - m1;
        }
    }
    float4* o = reinterpret_cast<float4*>(out + sb * QKK + 32 * j);
#pragma unroll
    for (int i = 0; i < 8; i++) o[i] = make_float4(v[4 * i], v[4 * i + 1], v[4 * i + 2], v[4 * i + 3]);
}

// ---- the Q4_K writer: BlockQ4K::from_float (k_quants.rs:1570-1654) -------------------
// llama.cpp's quantize_row_q4_K_ref. Eight threads per super-block, one per
// sub-block, each running make_qkx2_quants (candle utils.rs:308-397, with
// rmin -1, rdelta 0.1, 21 steps, squared error) on its 32 values in the
// reference's operation order; the super-block's max scale and max min are
// taken in sub-block order, as the reference's loop does.

__device__ float make_qkx2(const float* x, const float* w, uint8_t* L, float* the_min) {
    constexpr int n = 32, nmax = 15, nstep = 20;
    const float rmin = -1.0f, rdelta = 0.1f;
    float mn = x[0], mx = x[0];
    float sum_w = w[0];
    float sum_x = sum_w * x[0];
    for (int i = 1; i < n; i++) {
        if (x[i] < mn) mn = x[i];
        if (x[i] > mx) mx = x[i];
        sum_w = sum_w + w[i];
        sum_x = sum_x + w[i] * x[i];
    }
    if (mn > 0.0f) mn = 0.0f;
    if (mx == mn) {
        for (int i = 0; i < n; i++) L[i] = 0;
        *the_min = -mn;
        return 0.0f;
    }
    float iscale = (float)nmax / (mx - mn);
    float scale = 1.0f / iscale;
    float best = 0.0f;
    for (int i = 0; i < n; i++) {
        int li = nearest_int_even(iscale * (x[i] - mn));
        li = li < 0 ? 0 : (li > nmax ? nmax : li);
        L[i] = (uint8_t)li;
        float diff = scale * (float)li + mn - x[i];
        diff = diff * diff;
        best = best + w[i] * diff;
    }
    uint8_t laux[32];
    for (int is = 0; is <= nstep; is++) {
        iscale = (rmin + rdelta * (float)is + (float)nmax) / (mx - mn);
        float sum_l = 0.0f, sum_l2 = 0.0f, sum_xl = 0.0f;
        for (int i = 0; i < n; i++) {
            int li = nearest_int_even(iscale * (x[i] - mn));
            li = li < 0 ? 0 : (li > nmax ? nmax : li);
            laux[i] = (uint8_t)li;
            const float lf = (float)li;
            sum_l = sum_l + w[i] * lf;
            sum_l2 = sum_l2 + w[i] * lf * lf;
            sum_xl = sum_xl + w[i] * lf * x[i];
        }
        const float D = sum_w * sum_l2 - sum_l * sum_l;
        if (D > 0.0f) {
            float this_scale = (sum_w * sum_xl - sum_x * sum_l) / D;
            float this_min = (sum_l2 * sum_x - sum_l * sum_xl) / D;
            if (this_min > 0.0f) {
                this_min = 0.0f;
                this_scale = sum_xl / sum_l2;
            }
            float cur = 0.0f;
            for (int i = 0; i < n; i++) {
                float diff = this_scale * (float)laux[i] + this_min - x[i];
                diff = diff * diff;
                cur = cur + w[i] * diff;
            }
            if (cur < best) {
                for (int i = 0; i < n; i++) L[i] = laux[i];
                best = cur;
                scale = this_scale;
                mn = this_min;
            }
        }
    }
    *the_min = -mn;
    return scale;
}

__global__ __launch_bounds__(256) void k_qk_quantize(const float* __restrict__ xin, int64_t nsb,
                                                    uint8_t* __restrict__ out) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int j = (int)(t & 7);
    const int64_t sb = t >> 3;
    const bool live = sb < nsb;  // the 8 lanes of a super-block are live together
    float x[32], w[32];
    uint8_t L[32];
    float scale = 0.0f, mnv = 0.0f;
    if (live) {
        const float4* src = reinterpret_cast<const float4*>(xin + sb * QKK + 32 * j);
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const float4 v = src[i];
            x[4 * i] = v.x; x[4 * i + 1] = v.y; x[4 * i + 2] = v.z; x[4 * i + 3] = v.w;
        }
        float sum_x2 = 0.0f;
        for (int i = 0; i < 32; i++) sum_x2 = sum_x2 + x[i] * x[i];
        const float av_x = sqrtf(sum_x2 / 32.0f);
        for (int i = 0; i < 32; i++) w[i] = av_x + fabsf(x[i]);
        scale = make_qkx2(x, w, L, &mnv);
    }
    // max scale and max min over the super-block, in sub-block order, from +0
    const int lane = (int)(threadIdx.x & 63), base = lane & ~7;
    float max_scale = 0.0f, max_min = 0.0f;
#pragma unroll
    for (int s = 0; s < 8; s++) {
        const float sj = __shfl(scale, base + s, 64), mj = __shfl(mnv, base + s, 64);
        if (sj > max_scale) max_scale = sj;
        if (mj > max_min) max_min = mj;
    }
    const float inv_scale = max_scale > 0.0f ? 63.0f / max_scale : 0.0f;
    const float inv_min = max_min > 0.0f ? 63.0f / max_min : 0.0f;
    // `(nearest_int(..) as u8).min(63)`: the cast wraps, then the min
    int ls = nearest_int_even(inv_scale * scale) & 0xff;
    int lm = nearest_int_even(inv_min * mnv) & 0xff;
    ls = ls < 63 ? ls : 63;
    lm = lm < 63 ? lm : 63;
    const uint16_t dh = f16_from_f32(max_scale / 63.0f);
    const uint16_t mh = f16_from_f32(max_min / 63.0f);
    // the final levels; a sub-block whose d is zero keeps the search's levels
    const float d = f16_to_f32(dh) * (float)ls;
    if (live && d != 0.0f) {
        const float dm = f16_to_f32(mh) * (float)lm;
        for (int i = 0; i < 32; i++) {
            int lv = nearest_int_even((x[i] + dm) / d);
            L[i] = (uint8_t)(lv < 0 ? 0 : (lv > 15 ? 15 : lv));
        }
    }
    // the packed 6-bit scales (k_quants.rs:1625-1635) from all eight lanes
    int lsv[8], lmv[8];
#pragma unroll
    for (int s = 0; s < 8; s++) {
        lsv[s] = __shfl(ls, base + s, 64);
        lmv[s] = __shfl(lm, base + s, 64);
    }
    // sub-block 2c's levels are chunk c's low nibbles, 2c + 1's the high ones
    uint32_t mine[8], other[8];
#pragma unroll
    for (int q = 0; q < 8; q++) {
        // position-major: dword l holds elements l, 8 + l, 16 + l, 24 + l
        mine[q] = (uint32_t)L[q] | ((uint32_t)L[8 + q] << 8) | ((uint32_t)L[16 + q] << 16) | ((uint32_t)L[24 + q] << 24);
    }
#pragma unroll
    for (int q = 0; q < 8; q++) other[q] = __shfl((int)mine[q], lane ^ 1, 64);
    if (!live) return;
    uint8_t* blk = out + sb * QK4K_BYTES;
    if (j == 0) {
        uint8_t sc[12];
#pragma unroll
        for (int s = 0; s < 12; s++) sc[s] = 0;
#pragma unroll
        for (int s = 0; s < 8; s++) {
            if (s < 4) {
                sc[s] = (uint8_t)lsv[s];
                sc[s + 4] = (uint8_t)lmv[s];
            } else {
                sc[s + 4] = (uint8_t)((lsv[s] & 0x0f) | ((lmv[s] & 0x0f) << 4));
                sc[s - 4] |= (uint8_t)((lsv[s] >> 4) << 6);
                sc[s] |= (uint8_t)((lmv[s] >> 4) << 6);
            }
        }
        uint32_t h[4];
        h[0] = (uint32_t)dh | ((uint32_t)mh << 16);
        h[1] = (uint32_t)sc[0] | ((uint32_t)sc[1] << 8) | ((uint32_t)sc[2] << 16) | ((uint32_t)sc[3] << 24);
        h[2] = (uint32_t)sc[4] | ((uint32_t)sc[5] << 8) | ((uint32_t)sc[6] << 16) | ((uint32_t)sc[7] << 24);
        h[3] = (uint32_t)sc[8] | ((uint32_t)sc[9] << 8) | ((uint32_t)sc[10] << 16) | ((uint32_t)sc[11] << 24);
        *reinterpret_cast<uint4*>(blk) = make_uint4(h[0], h[1], h[2], h[3]);
    }
    if ((j & 1) == 0) {
        uint32_t q[8];
#pragma unroll
        for (int s = 0; s < 8; s++) q[s] = mine[s] | (other[s] << 4);
        uint4* o = reinterpret_cast<uint4*>(blk + 16 + 32 * (j >> 1));
        o[0] = make_uint4(q[0], q[1], q[2], q[3]);
        o[1] = make_uint4(q[4], q[5], q[6], q[7]);
    }
}

// ---- the linear ---------------------------------------------------------------------
//
// k_gemv_qk<MR>: MR <= 4 activation rows against the whole weight, persistent
// over row tiles like the q4_0/q8_0 GEMV.
//   Phase 1: Q8_K of the MR rows into LDS, one wave per 256-element
//     super-block (4 elements per lane): the first element of the largest |x|
//     is found by a (value, index) reduction, codes are stored in the
//     position-major order of the weight chunks, with d and the 16 code sums.
//   Phase 2: one (row, super-block) item per thread: its 144 bytes in nine
//     16-byte loads, aux32[l] as sc * v_dot4 terms, sumi, then the nine f32
//     terms (d_w*d_x)*aux32[l] and (dmin_w*d_x)*sumi into LDS.
//   Phase 3: 16 lanes per output; lane l < 8 adds term l over the
//     super-blocks in order, lane 8 subtracts the sumi terms, and lane 0
//     forms sumf + (((s0 + s1) + ...) + s7).

constexpr int QG_THREADS = 256;
constexpr int QG_TERMS = 9;

template <typename XT>
__device__ inline float4 load4(const XT* p);
template <>
__device__ inline float4 load4<float>(const float* p) { return *reinterpret_cast<const float4*>(p); }
template <>
__device__ inline float4 load4<uint16_t>(const uint16_t* p) {
    const uint2 h = *reinterpret_cast<const uint2*>(p);
    return make_float4(bf16_to_f32((uint16_t)(h.x & 0xffffu)), bf16_to_f32((uint16_t)(h.x >> 16)),
                       bf16_to_f32((uint16_t)(h.y & 0xffffu)), bf16_to_f32((uint16_t)(h.y >> 16)));
}

template <int MR, typename XT>
__global__ __launch_bounds__(QG_THREADS) void k_gemv_qk(const XT* __restrict__ x, int K, int nsb,
                                                       const uint8_t* __restrict__ w, int N, int rows,
                                                       const float* __restrict__ bias, void* y, int y_bf16) {
    extern __shared__ __align__(16) char smem[];
    int8_t* xq = reinterpret_cast<int8_t*>(smem);                     // [MR][nsb][256] position-major
    float* xd = reinterpret_cast<float*>(smem + (size_t)MR * K);      // [MR][nsb], padded to 16 bytes
    int* xbs = reinterpret_cast<int*>(xd + ((MR * nsb + 3) & ~3));    // [MR][nsb][16]
    float* terms = reinterpret_cast<float*>(xbs + MR * nsb * 16);      // [2][rows*MR][nsb][9]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int ntiles = (N + rows - 1) / rows;

    // phase 1: Q8_K of the activation rows (BlockQ8K::from_float)
    for (int blk = wave; blk < MR * nsb; blk += QG_THREADS / 64) {
        const int mr = blk / nsb, sb = blk - mr * nsb;
        const float4 v4 = load4<XT>(x + (int64_t)mr * K + sb * QKK + 4 * lane);
        const float e[4] = {v4.x, v4.y, v4.z, v4.w};
        // this lane's first largest |x| (strict <, NaN never taken), then the
        // wave's: larger value wins, equal values go to the lower index
        float am = 0.0f, mv = 0.0f;
        int idx = 0x7fffffff;
#pragma unroll
        for (int i = 0; i < 4; i++)
            if (am < fabsf(e[i])) { am = fabsf(e[i]); mv = e[i]; idx = 4 * lane + i; }
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1) {
            const float oa = __shfl_xor(am, off, 64), ov = __shfl_xor(mv, off, 64);
            const int oi = __shfl_xor(idx, off, 64);
            if (oa > am || (oa == am && oi < idx)) { am = oa; mv = ov; idx = oi; }
        }
        int q[4] = {0, 0, 0, 0};
        float d = 0.0f;
        if (am != 0.0f) {
            const float iscale = -127.0f / mv;
#pragma unroll
            for (int i = 0; i < 4; i++) q[i] = sat_i8k(roundf(iscale * e[i]));
            d = 1.0f / iscale;
        }
        // element e = 4*lane + i: sub-block j = lane / 8, within it r = 4*(lane % 8) + i,
        // g = r / 8, l = r % 8 -> position-major byte 32 j + 4 l + g
        int8_t* dst = xq + (int64_t)blk * QKK;
        const int j = lane >> 3, r0 = 4 * (lane & 7);
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int r = r0 + i;
            dst[32 * j + 4 * (r & 7) + (r >> 3)] = (int8_t)q[i];
        }
        // sums of 16 codes: lanes 4s .. 4s + 3 hold elements 16s .. 16s + 15
        int s = q[0] + q[1] + q[2] + q[3];
        s += __shfl_xor(s, 1, 64);
        s += __shfl_xor(s, 2, 64);
        if ((lane & 3) == 0) xbs[blk * 16 + (lane >> 2)] = (int)(int16_t)s;
        if (lane == 0) xd[blk] = d;
    }
    __syncthreads();

    // phases 2 and 3, persistent over row tiles with the next tile's bytes in flight
    // The super-block loads are unconditional buffer loads over the tile's
    // bytes (a thread past the tile, or a tile past the last, reads at an
    // offset past the descriptor: zero, no memory access), so the compiler
    // counts the loads in flight exactly and the waits for this tile's item
    // leave the next tile's in flight. Behind a branch, every wait on the
    // current item also waited for the whole prefetch.
    uint4 wv[9], wn[9];
    auto gload = [&](int tile, uint4* dst) {
        const bool live = tile < ntiles;
        const int64_t row0 = live ? (int64_t)tile * rows : 0;
        const int nrows = live ? (int)((N - row0) < rows ? (N - row0) : rows) : 0;
        const buf_rsrc rw = make_rsrc(w + row0 * nsb * QK4K_BYTES, (uint32_t)(nrows * nsb) * QK4K_BYTES);
        const uint32_t off = tid < nrows * nsb ? (uint32_t)tid * QK4K_BYTES : BUF_OOB;
#pragma unroll
        for (int i = 0; i < 9; i++) {
            const float4 f = buf_load_f4(rw, off + 16u * i);
            dst[i] = make_uint4(__float_as_uint(f.x), __float_as_uint(f.y), __float_as_uint(f.z), __float_as_uint(f.w));
        }
    };
    int tile = (int)blockIdx.x;
    gload(tile, wv);  // the grid never exceeds the tile count
    for (int buf = 0; tile < ntiles; tile += (int)gridDim.x, buf ^= 1) {
        gload(tile + (int)gridDim.x, wn);
        const int64_t row0 = (int64_t)tile * rows;
        const int nrows = (int)((N - row0) < rows ? (N - row0) : rows);
        float* tb = terms + (size_t)buf * rows * MR * nsb * QG_TERMS;
        if (tid < nrows * nsb) {
            const int r = tid / nsb, sb = tid - r * nsb;
            const uint32_t h0 = wv[0].x, s0 = wv[0].y, s1 = wv[0].z, s2 = wv[0].w;
            const uint8_t scb[12] = {(uint8_t)s0, (uint8_t)(s0 >> 8), (uint8_t)(s0 >> 16), (uint8_t)(s0 >> 24),
                                     (uint8_t)s1, (uint8_t)(s1 >> 8), (uint8_t)(s1 >> 16), (uint8_t)(s1 >> 24),
                                     (uint8_t)s2, (uint8_t)(s2 >> 8), (uint8_t)(s2 >> 16), (uint8_t)(s2 >> 24)};
            int sc[8], mn[8];
#pragma unroll
            for (int j = 0; j < 8; j++) scale_min_k4(j, scb, &sc[j], &mn[j]);
            const float dw = f16_bits_hw((uint16_t)(h0 & 0xffffu));
            const float dmw = f16_bits_hw((uint16_t)(h0 >> 16));
#pragma unroll
            for (int mr = 0; mr < MR; mr++) {
                const int blk = mr * nsb + sb;
                const int* xa = reinterpret_cast<const int*>(xq + (int64_t)blk * QKK);
                int aux[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    const uint4 a = wv[1 + 2 * c], b = wv[2 + 2 * c];
                    const uint32_t dws[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
                    int4 xl[4];
#pragma unroll
                    for (int u = 0; u < 4; u++) xl[u] = reinterpret_cast<const int4*>(xa + 16 * c)[u];
                    const int xs[16] = {xl[0].x, xl[0].y, xl[0].z, xl[0].w, xl[1].x, xl[1].y, xl[1].z, xl[1].w,
                                        xl[2].x, xl[2].y, xl[2].z, xl[2].w, xl[3].x, xl[3].y, xl[3].z, xl[3].w};
#pragma unroll
                    for (int l = 0; l < 8; l++) {
                        const int lo = __builtin_amdgcn_sdot4((int)(dws[l] & 0x0f0f0f0fu), xs[l], 0, false);
                        const int hi = __builtin_amdgcn_sdot4((int)((dws[l] >> 4) & 0x0f0f0f0fu), xs[8 + l], 0, false);
                        aux[l] += sc[2 * c] * lo + sc[2 * c + 1] * hi;
                    }
                }
                const int4* bs4 = reinterpret_cast<const int4*>(xbs + blk * 16);
                int sumi = 0;
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const int4 bs = bs4[u];
                    sumi += bs.x * mn[2 * u] + bs.y * mn[2 * u] + bs.z * mn[2 * u + 1] + bs.w * mn[2 * u + 1];
                }
                const float yd = xd[blk];
                const float d = dw * yd;
                const float dmin = dmw * yd;
                float* t = tb + ((size_t)(r * MR + mr) * nsb + sb) * QG_TERMS;
#pragma unroll
                for (int l = 0; l < 8; l++) t[l] = d * (float)aux[l];
                t[8] = dmin * (float)sumi;
            }
        }
        __syncthreads();
        // phase 3: 16 lanes per output
        for (int o = tid >> 4; o < nrows * MR; o += QG_THREADS / 16) {
            const int a = tid & 15;
            const int r = o / MR, mr = o - r * MR;
            float acc = 0.0f;
            if (a < QG_TERMS) {
                const float* tr = tb + (size_t)(r * MR + mr) * nsb * QG_TERMS + a;
                for (int sb = 0; sb < nsb; sb++) {
                    if (a < 8)
                        acc = acc + tr[sb * QG_TERMS];
                    else
                        acc = acc - tr[sb * QG_TERMS];
                }
            }
            float s[9];
#pragma unroll
            for (int u = 0; u < 9; u++) s[u] = __shfl(acc, (lane & ~15) + u, 64);
            if (a == 0) {
                float tot = 0.0f;
#pragma unroll
                for (int u = 0; u < 8; u++) tot = tot + s[u];
                float v = s[8] + tot;
                const int64_t n = row0 + r;
                if (bias) v = v + bias[n];
                if (y_bf16)
                    reinterpret_cast<uint16_t*>(y)[(int64_t)mr * N + n] = bf16_from_f32(v);
                else
                    reinterpret_cast<float*>(y)[(int64_t)mr * N + n] = v;
            }
        }
#pragma unroll
        for (int i = 0; i < 9; i++) wv[i] = wn[i];
    }
}

// ---- prefill GEMM on f16 MFMA (m > 4) --------------------------------------------
//
// The reference keeps nine f32 accumulators per output (sums[0..7], sumf), so
// a wave owns a 32x16 output tile (8 outputs per lane, 72 accumulators). A
// workgroup is four waves side by side: 32 rows x 64 weight columns, the
// activation rows shared through LDS.
//
// Exactness. For residue l the K dimension is the 32 elements 32j + 8g + l
// (j = 0..7, g = 0..3); with the weight operand sc_j * nib (an integer <= 945,
// exact in f16) and the activation operand the Q8_K code (exact in f16),
// one v_mfma_f32_16x16x32_f16 returns aux32[l] exactly (|aux32| < 2^22). The
// nibbles become f16 through the 0x6400 | nib pattern (1024 + nib) minus
// 1024, both exact. sumi is one v_mfma_f32_16x16x16_f16 of the 16 code sums
// (|sum| <= 2048, exact in f16) against m_{j/2}. The f32 steps are then the
// reference's, in its order.
//
// Operand order. MFMA lane group G (lanes 16G..16G+15) holds K slots
// 8G..8G+7 = sub-blocks j = 2G (slots 0-3) and 2G+1 (slots 4-7), positions
// g = 0, 2, 1, 3 in that order: the order in which two shifts and masks of a
// weight dword (chunk G, word l) yield nibble pairs. The prepass writes the
// activation codes in the same order.

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4v __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float f32x4q __attribute__((ext_vector_type(4)));

constexpr int QM_ROWS = 32, QM_COLS = 64, QM_THREADS = 256;
constexpr int QM_AS = 512 + 16;  // LDS row stride (bytes) of the activation codes: conflict-free b128 reads
constexpr int QM_XCD = 8;

__device__ inline int gslot(int g) { return ((g & 1) << 1) | (g >> 1); }  // g -> slot within a half: 0,2,1,3 -> 0,1,2,3

// Q8_K of every activation row (rows >= M: zero codes, sums and scale), one
// wave per (row, super-block), into the MFMA operand layout:
//   xa  f16 [M_pad][nsb][l][G][8]   codes, slot 4h + gslot(g) for sub-block 2G + h
//   xbs f16 [M_pad][nsb][16]         sums of 16 codes
//   xd  f32 [nsb][M_pad]             d = 1 / iscale
template <typename XT>
__global__ __launch_bounds__(256) void k_q8k_rows(const XT* __restrict__ x, int M, int M_pad, int K, int nsb,
                                                 uint16_t* __restrict__ xa, uint16_t* __restrict__ xbs,
                                                 float* __restrict__ xd) {
    const int64_t blk = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (blk >= (int64_t)M_pad * nsb) return;
    const int row = (int)(blk / nsb), sb = (int)(blk - (int64_t)row * nsb);
    float e[4] = {0.f, 0.f, 0.f, 0.f};
    if (row < M) {
        const float4 v4 = load4<XT>(x + (int64_t)row * K + sb * QKK + 4 * lane);
        e[0] = v4.x; e[1] = v4.y; e[2] = v4.z; e[3] = v4.w;
    }
    float am = 0.0f, mv = 0.0f;
    int idx = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < 4; i++)
        if (am < fabsf(e[i])) { am = fabsf(e[i]); mv = e[i]; idx = 4 * lane + i; }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float oa = __shfl_xor(am, off, 64), ov = __shfl_xor(mv, off, 64);
        const int oi = __shfl_xor(idx, off, 64);
        if (oa > am || (oa == am && oi < idx)) { am = oa; mv = ov; idx = oi; }
    }
    int q[4] = {0, 0, 0, 0};
    float d = 0.0f;
    if (am != 0.0f) {
        const float iscale = -127.0f / mv;
#pragma unroll
        for (int i = 0; i < 4; i++) q[i] = sat_i8k(roundf(iscale * e[i]));
        d = 1.0f / iscale;
    }
    uint16_t* dst = xa + blk * QKK;
    const int j = lane >> 3, G = j >> 1, h = j & 1;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const int r = 4 * (lane & 7) + i, g = r >> 3, l = r & 7;
        dst[(l * 4 + G) * 8 + 4 * h + gslot(g)] = __builtin_bit_cast(uint16_t, (_Float16)(float)q[i]);
    }
    int s = q[0] + q[1] + q[2] + q[3];
    s += __shfl_xor(s, 1, 64);
    s += __shfl_xor(s, 2, 64);
    if ((lane & 3) == 0) xbs[blk * 16 + (lane >> 2)] = __builtin_bit_cast(uint16_t, (_Float16)(float)s);
    if (lane == 0) xd[(int64_t)sb * M_pad + row] = d;
}

// byte k (0..11) of the three scale words, by selects (a lane-dependent
// index into an array would go through scratch memory)
__device__ inline uint32_t byte_of(uint32_t w0, uint32_t w1, uint32_t w2, int k) {
    const uint32_t wd = k < 4 ? w0 : (k < 8 ? w1 : w2);
    return (wd >> (8 * (k & 3))) & 0xffu;
}

__global__ __launch_bounds__(QM_THREADS, 2) void k_gemm_qk(const uint16_t* __restrict__ xa,
                                                         const uint16_t* __restrict__ xbs,
                                                         const float* __restrict__ xd, int M, int M_pad, int nsb,
                                                         const uint8_t* __restrict__ w, int N,
                                                         const float* __restrict__ bias, void* __restrict__ y,
                                                         int y_bf16) {
    __shared__ __align__(16) uint8_t sA[2][QM_ROWS * QM_AS];
    __shared__ __align__(16) uint16_t sBS[2][QM_ROWS * 16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int lrow = lane & 15, G = lane >> 4;

    const int mt = (int)gridDim.y;
    const int ntot = (int)(gridDim.x * gridDim.y);
    const int id = (int)(blockIdx.y * gridDim.x + blockIdx.x);
    int tile = id;
    if (ntot % QM_XCD == 0) tile = (id % QM_XCD) * (ntot / QM_XCD) + id / QM_XCD;
    const int m0 = (tile % mt) * QM_ROWS, n0 = (tile / mt) * QM_COLS;
    const int col = n0 + wave * 16 + lrow;  // this lane's weight column

    float sums[8][2][4], sumf[2][4];
#pragma unroll
    for (int l = 0; l < 8; l++)
#pragma unroll
        for (int rt = 0; rt < 2; rt++)
#pragma unroll
            for (int r = 0; r < 4; r++) sums[l][rt][r] = 0.0f;
#pragma unroll
    for (int rt = 0; rt < 2; rt++)
#pragma unroll
        for (int r = 0; r < 4; r++) sumf[rt][r] = 0.0f;

    // staging: the 32 activation rows' codes (1024 x 16 B: 4 per thread) and sums (64 x 16 B)
    // thread tid stages rows tid/32 + 8i (i = 0..3), 16-byte part tid % 32
    const int arow = tid >> 5, apart = tid & 31;
    auto ga = [&](int sb, int i) {
        return *reinterpret_cast<const uint4*>(xa + ((int64_t)(m0 + arow + 8 * i) * nsb + sb) * QKK + apart * 8);
    };
    auto sa = [&](int buf, int i, const uint4& v) {
        *reinterpret_cast<uint4*>(&sA[buf][(arow + 8 * i) * QM_AS + apart * 16]) = v;
    };
    auto gbs = [&](int sb) {
        return *reinterpret_cast<const uint4*>(xbs + ((int64_t)(m0 + (tid >> 1)) * nsb + sb) * 16 + (tid & 1) * 8);
    };
    auto sbs = [&](int buf, const uint4& v) {
        *reinterpret_cast<uint4*>(&sBS[buf][(tid >> 1) * 16 + (tid & 1) * 8]) = v;
    };
    // this lane's weight bytes for a super-block: the 16-byte head and chunk G
    auto load_b = [&](int sb, uint4& hd, uint4& c0, uint4& c1, float4& dx0, float4& dx1) {
        hd = c0 = c1 = make_uint4(0u, 0u, 0u, 0u);
        if (col < N) {
            const uint4* blk = reinterpret_cast<const uint4*>(w + ((int64_t)col * nsb + sb) * QK4K_BYTES);
            hd = blk[0];
            c0 = blk[1 + 2 * G];
            c1 = blk[2 + 2 * G];
        }
        dx0 = *reinterpret_cast<const float4*>(xd + (int64_t)sb * M_pad + m0 + 4 * G);
        dx1 = *reinterpret_cast<const float4*>(xd + (int64_t)sb * M_pad + m0 + 16 + 4 * G);
    };

    uint4 ra0, ra1, ra2, ra3, rb = make_uint4(0u, 0u, 0u, 0u);
    uint4 hd, c0, c1, nhd, nc0, nc1;
    float4 dx0, dx1, ndx0, ndx1;
    ra0 = ga(0, 0); ra1 = ga(0, 1); ra2 = ga(0, 2); ra3 = ga(0, 3);
    if (tid < 64) rb = gbs(0);
    load_b(0, hd, c0, c1, dx0, dx1);
    sa(0, 0, ra0); sa(0, 1, ra1); sa(0, 2, ra2); sa(0, 3, ra3);
    if (tid < 64) sbs(0, rb);
    __syncthreads();
    const half2v k1024 = {(_Float16)1024.0f, (_Float16)1024.0f};
    for (int sb = 0; sb < nsb; sb++) {
        const int buf = sb & 1;
        if (sb + 1 < nsb) {
            ra0 = ga(sb + 1, 0); ra1 = ga(sb + 1, 1); ra2 = ga(sb + 1, 2); ra3 = ga(sb + 1, 3);
            if (tid < 64) rb = gbs(sb + 1);
            load_b(sb + 1, nhd, nc0, nc1, ndx0, ndx1);
        }
        // the column's scales and mins for sub-blocks 2G, 2G + 1 (get_scale_min_k4)
        int scv[2], mnv[2];
#pragma unroll
        for (int hh = 0; hh < 2; hh++) {
            const int jj = 2 * G + hh;
            if (jj < 4) {
                scv[hh] = (int)(byte_of(hd.y, hd.z, hd.w, jj) & 63);
                mnv[hh] = (int)(byte_of(hd.y, hd.z, hd.w, jj + 4) & 63);
            } else {
                scv[hh] = (int)((byte_of(hd.y, hd.z, hd.w, jj + 4) & 0x0f) | ((byte_of(hd.y, hd.z, hd.w, jj - 4) >> 6) << 4));
                mnv[hh] = (int)((byte_of(hd.y, hd.z, hd.w, jj + 4) >> 4) | ((byte_of(hd.y, hd.z, hd.w, jj) >> 6) << 4));
            }
        }
        const half2v sc0 = {(_Float16)(float)scv[0], (_Float16)(float)scv[0]};
        const half2v sc1 = {(_Float16)(float)scv[1], (_Float16)(float)scv[1]};
        const float dwf = f16_bits_hw((uint16_t)(hd.x & 0xffffu));
        const float dmwf = f16_bits_hw((uint16_t)(hd.x >> 16));
        const float dxr[2][4] = {{dx0.x, dx0.y, dx0.z, dx0.w}, {dx1.x, dx1.y, dx1.z, dx1.w}};
        float dd[2][4];
#pragma unroll
        for (int rt = 0; rt < 2; rt++)
#pragma unroll
            for (int r = 0; r < 4; r++) dd[rt][r] = dwf * dxr[rt][r];
        const uint32_t cw[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
        const f32x4q zero = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int l = 0; l < 8; l++) {
            const uint32_t dw = cw[l];
            const half2v lo02 = (__builtin_bit_cast(half2v, (dw & 0x000f000fu) | 0x64006400u) - k1024) * sc0;
            const half2v lo13 = (__builtin_bit_cast(half2v, ((dw >> 8) & 0x000f000fu) | 0x64006400u) - k1024) * sc0;
            const half2v hi02 = (__builtin_bit_cast(half2v, ((dw >> 4) & 0x000f000fu) | 0x64006400u) - k1024) * sc1;
            const half2v hi13 = (__builtin_bit_cast(half2v, ((dw >> 12) & 0x000f000fu) | 0x64006400u) - k1024) * sc1;
            const half8 bop = {lo02[0], lo02[1], lo13[0], lo13[1], hi02[0], hi02[1], hi13[0], hi13[1]};
#pragma unroll
            for (int rt = 0; rt < 2; rt++) {
                const half8 aop =
                    *reinterpret_cast<const half8*>(&sA[buf][(rt * 16 + lrow) * QM_AS + (l * 4 + G) * 16]);
                const f32x4q aux = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop, bop, zero, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; r++) sums[l][rt][r] = sums[l][rt][r] + dd[rt][r] * aux[r];
            }
        }
        {
            const half4v mop = {(_Float16)(float)mnv[0], (_Float16)(float)mnv[0], (_Float16)(float)mnv[1],
                                (_Float16)(float)mnv[1]};
#pragma unroll
            for (int rt = 0; rt < 2; rt++) {
                const half4v bsop = *reinterpret_cast<const half4v*>(&sBS[buf][(rt * 16 + lrow) * 16 + 4 * G]);
                const f32x4q sumi = __builtin_amdgcn_mfma_f32_16x16x16f16(bsop, mop, zero, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const float dm = dmwf * dxr[rt][r];
                    sumf[rt][r] = sumf[rt][r] - dm * sumi[r];
                }
            }
        }
        if (sb + 1 < nsb) {
            sa(buf ^ 1, 0, ra0); sa(buf ^ 1, 1, ra1); sa(buf ^ 1, 2, ra2); sa(buf ^ 1, 3, ra3);
            if (tid < 64) sbs(buf ^ 1, rb);
            hd = nhd; c0 = nc0; c1 = nc1; dx0 = ndx0; dx1 = ndx1;
        }
        __syncthreads();
    }
    if (col >= N) return;
    const float bv = bias ? bias[col] : 0.0f;
#pragma unroll
    for (int rt = 0; rt < 2; rt++) {
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int m = m0 + rt * 16 + 4 * G + r;
            if (m >= M) continue;
            float tot = 0.0f;
#pragma unroll
            for (int l = 0; l < 8; l++) tot = tot + sums[l][rt][r];
            float v = sumf[rt][r] + tot;
            if (bias) v = v + bv;
            if (y_bf16)
                reinterpret_cast<uint16_t*>(y)[(int64_t)m * N + col] = bf16_from_f32(v);
            else
                reinterpret_cast<float*>(y)[(int64_t)m * N + col] = v;
        }
    }
}

tn_status check_qk(const char* op, int64_t n, int64_t k) {
    if (n < 0 || k <= 0 || k % QKK != 0) {
        char buf[384];
        std::snprintf(buf, sizeof buf,
                      "%s: q4_k stores 256 elements per block, so it must have their last dim divisible by "
                      "block size -- got %lld, which is not a multiple of 256 (shape [%lld, %lld])",
                      op, (long long)k, (long long)n, (long long)k);
        return fail(TN_ENOTIMPL, buf);
    }
    if (n * (k / QKK) > ((int64_t)1 << 36)) return fail(TN_EVALUE, std::string(op) + ": weight too large");
    return TN_OK;
}

size_t qk_lds(int mr, int k, int rows) {
    const int nsb = k / QKK;
    return (size_t)mr * k + (size_t)((mr * nsb + 3) & ~3) * 4 + (size_t)mr * nsb * 64 +
           2 * (size_t)rows * mr * nsb * QG_TERMS * 4;
}

template <int MR, typename XT>
tn_status launch_gemv_qk(hipStream_t st, const XT* x, int K, const uint8_t* w, int N, const float* bias, void* y,
                         int y_bf16) {
    const int nsb = K / QKK;
    int rows = QG_THREADS / nsb;
    const int spread = (int)cdiv(N, 256);
    if (rows > spread) rows = spread;
    if (rows > N) rows = N;
    if (rows < 1) return TN_ENOTIMPL;
    const size_t lds = qk_lds(MR, K, rows);
    if (lds > 64 * 1024) return TN_ENOTIMPL;
    int resident = 0;
    tn_status s = resident_workgroups(reinterpret_cast<const void*>(&k_gemv_qk<MR, XT>), QG_THREADS, lds, &resident);
    if (s != TN_OK) return s;
    const int64_t ntiles = cdiv(N, rows);
    const unsigned grid = (unsigned)(ntiles < resident ? ntiles : resident);
    hipLaunchKernelGGL((k_gemv_qk<MR, XT>), dim3(grid), dim3(QG_THREADS), lds, st, x, K, nsb, w, N, rows, bias, y,
                       y_bf16);
    TN_LAUNCHED();
    return TN_OK;
}

template <typename XT>
tn_status linear_qk(hipStream_t st, const XT* x, int64_t m, int64_t k, const uint8_t* w, int64_t n,
                    const float* bias, void* y, int y_bf16) {
    if (m == 0 || n == 0) return TN_OK;
    if (n > INT32_MAX || k > INT32_MAX) return fail(TN_EVALUE, "torch._C._quantized_linear: shape too large");
    const size_t ysz = y_bf16 ? 2 : 4;
    // prefill: Q8_K prepass, then the MFMA GEMM (any row count, and rows of
    // any length; bit-identical to the GEMV, since every output is the same
    // recurrence)
    auto gemm = [&](const XT* x, int64_t m, void* y) -> tn_status {
        const int nsb = (int)(k / QKK);
        const int64_t M_pad = cdiv(m, QM_ROWS) * QM_ROWS;
        if (M_pad > INT32_MAX) return fail(TN_EVALUE, "torch._C._quantized_linear: shape too large");
        const size_t xa_bytes = (size_t)M_pad * nsb * QKK * 2, bs_bytes = (size_t)M_pad * nsb * 32;
        void* ws = nullptr;
        tn_status s = workspace(st, xa_bytes + bs_bytes + (size_t)M_pad * nsb * 4, &ws);
        if (s != TN_OK) return s;
        uint16_t* xa = static_cast<uint16_t*>(ws);
        uint16_t* xbs = reinterpret_cast<uint16_t*>(static_cast<char*>(ws) + xa_bytes);
        float* xdv = reinterpret_cast<float*>(static_cast<char*>(ws) + xa_bytes + bs_bytes);
        hipLaunchKernelGGL((k_q8k_rows<XT>), dim3((unsigned)cdiv(M_pad * nsb, 4)), dim3(256), 0, st, x, (int)m,
                           (int)M_pad, (int)k, nsb, xa, xbs, xdv);
        TN_LAUNCHED();
        const dim3 grid((unsigned)cdiv(n, QM_COLS), (unsigned)(M_pad / QM_ROWS));
        hipLaunchKernelGGL(k_gemm_qk, grid, dim3(QM_THREADS), 0, st, xa, xbs, xdv, (int)m, (int)M_pad, nsb, w, (int)n,
                           bias, y, y_bf16);
        TN_LAUNCHED();
        return TN_OK;
    };
    if (m > 4) return gemm(x, m, y);
    // decode: rows of x in chunks of up to 4 (every output is the same recurrence, so
    // the chunking changes no bit); the widest chunk whose activations fit LDS
    int64_t r = 0;
    while (r < m) {
        const int64_t left = m - r;
        const XT* xr = x + r * k;
        void* yr = static_cast<char*>(y) + r * n * ysz;
        tn_status s = TN_ENOTIMPL;
        int64_t c = 0;
        if (left >= 4) {
            s = launch_gemv_qk<4, XT>(st, xr, (int)k, w, (int)n, bias, yr, y_bf16);
            c = 4;
        }
        if (s == TN_ENOTIMPL && left >= 2) {
            s = launch_gemv_qk<2, XT>(st, xr, (int)k, w, (int)n, bias, yr, y_bf16);
            c = 2;
        }
        if (s == TN_ENOTIMPL) {
            s = launch_gemv_qk<1, XT>(st, xr, (int)k, w, (int)n, bias, yr, y_bf16);
            c = 1;
        }
        if (s == TN_ENOTIMPL) return gemm(xr, left, yr);  // a row too long for the GEMV's LDS
        if (s != TN_OK) return s;
        r += c;
    }
    return TN_OK;
}

}  // namespace
}  // namespace tn

using namespace tn;

extern "C" {

tn_status tn_q4_k_from_blob(void* stream, const uint8_t* blob, int64_t n, int64_t k, uint8_t* w) {
    tn_status s = check_qk("torch._C._quantized_to", n, k);
    if (s != TN_OK) return s;
    const int64_t nsb = n * (k / QKK);
    if (!nsb) return TN_OK;
    if (!blob || !w) return fail(TN_EVALUE, "tn_q4_k_from_blob: null pointer");
    if ((reinterpret_cast<uintptr_t>(blob) | reinterpret_cast<uintptr_t>(w)) % 16)
        return fail(TN_EINVAL, "tn_q4_k_from_blob: blob and w must be 16-byte aligned");
    hipLaunchKernelGGL(k_qk_repack<true>, dim3((unsigned)cdiv(nsb, 256)), dim3(256), 0, (hipStream_t)stream, blob,
                       nsb, w);
    TN_LAUNCHED();
    return TN_OK;
}

tn_status tn_q4_k_to_blob(void* stream, const uint8_t* w, int64_t n, int64_t k, uint8_t* blob) {
    tn_status s = check_qk("torch._C._quantized_blob", n, k);
    if (s != TN_OK) return s;
    const int64_t nsb = n * (k / QKK);
    if (!nsb) return TN_OK;
    if (!blob || !w) return fail(TN_EVALUE, "tn_q4_k_to_blob: null pointer");
    if ((reinterpret_cast<uintptr_t>(blob) | reinterpret_cast<uintptr_t>(w)) % 16)
        return fail(TN_EINVAL, "tn_q4_k_to_blob: blob and w must be 16-byte aligned");
    hipLaunchKernelGGL(k_qk_repack<false>, dim3((unsigned)cdiv(nsb, 256)), dim3(256), 0, (hipStream_t)stream, w,
                       nsb, blob);
    TN_LAUNCHED();
    return TN_OK;
}

tn_status tn_q4_k_quantize(void* stream, const float* x, int64_t n, int64_t k, uint8_t* w) {
    tn_status s = check_qk("torch._C._quantize", n, k);
    if (s != TN_OK) return s;
    const int64_t nsb = n * (k / QKK);
    if (!nsb) return TN_OK;
    if (!x || !w) return fail(TN_EVALUE, "tn_q4_k_quantize: null pointer");
    if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w)) % 16)
        return fail(TN_EINVAL, "tn_q4_k_quantize: x and w must be 16-byte aligned");
    hipLaunchKernelGGL(k_qk_quantize, dim3((unsigned)cdiv(nsb * 8, 256)), dim3(256), 0, (hipStream_t)stream, x, nsb,
                       w);
    TN_LAUNCHED();
    return TN_OK;
}

tn_status tn_q4_k_dequantize(void* stream, const uint8_t* w, int64_t n, int64_t k, float* out) {
    tn_status s = check_qk("torch._C._dequantize", n, k);
    if (s != TN_OK) return s;
    const int64_t nsb = n * (k / QKK);
    if (!nsb) return TN_OK;
    if (!w || !out) return fail(TN_EVALUE, "tn_q4_k_dequantize: null pointer");
    if ((reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(out)) % 16)
        return fail(TN_EINVAL, "tn_q4_k_dequantize: w and out must be 16-byte aligned");
    hipLaunchKernelGGL(k_qk_dequantize, dim3((unsigned)cdiv(nsb * 8, 256)), dim3(256), 0, (hipStream_t)stream, w,
                       nsb, out);
    TN_LAUNCHED();
    return TN_OK;
}

tn_status tn_q4_k_linear(void* stream, const void* x, int x_dtype, int64_t m, int64_t k, const uint8_t* w,
                         int64_t n, const float* bias, void* y, int y_dtype) {
    const char* OP = "torch._C._quantized_linear";
    if (x_dtype != TN_F32 && x_dtype != TN_BF16)
        return fail(TN_ENOTIMPL, std::string(OP) +
                                     ": the activation must be float32 (or bfloat16, widened exactly in-kernel) "
                                     "on the hip device");
    if (y_dtype != TN_F32 && y_dtype != TN_BF16)
        return fail(TN_ENOTIMPL, std::string(OP) + ": the output must be float32 or bfloat16");
    if (k <= 0 || k % QKK != 0 || m < 0 || n < 0) {
        char buf[256];
        std::snprintf(buf, sizeof buf, "%s: mat1 and mat2 shapes cannot be multiplied ([%lld, %lld] and %lldx%lld)",
                      OP, (long long)m, (long long)k, (long long)k, (long long)n);
        return fail(TN_EINVAL, buf);
    }
    if (m > 0 && n > 0 && (!x || !w || !y)) return fail(TN_EVALUE, std::string(OP) + ": null pointer");
    if (m > 0 && n > 0 && (reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w)) % 16)
        return fail(TN_EINVAL, std::string(OP) + ": x and the q4_k weight must be 16-byte aligned");
    hipStream_t st = (hipStream_t)stream;
    const int yb = y_dtype == TN_BF16;
    if (x_dtype == TN_F32) return linear_qk<float>(st, static_cast<const float*>(x), m, k, w, n, bias, y, yb);
    return linear_qk<uint16_t>(st, static_cast<const uint16_t*>(x), m, k, w, n, bias, y, yb);
}

}  // extern "C"
