// GGML block-quantised weights on gfx950 (q4_0 and q8_0): upload/repack,
// quantise, dequantise, and the quantised linear (decode GEMV and prefill
// MFMA GEMM).
//
// Arithmetic contract (candle-core/src/quantized/k_quants.rs, the reference's
// vendored candle): every output is
//     sumf = 0; for b in blocks: sumf += ((float)S_b * d_w[b]) * d_x[b]
// where S_b is the exact integer dot of the weight's codes (q4_0: nib - 8,
// vec_dot_unopt k_quants.rs:312-329; q8_0: the int8 codes, k_quants.rs:738-757)
// and the activation's Q8_0 codes, and the activation row is quantised by
// BlockQ8_0::from_float (k_quants.rs:676-705) -- Q8_0 is the VecDotType of
// both weight formats. The integer dot is exact in any order, and every kernel
// below performs the float steps in exactly that order with separate
// roundings (the library is built with -ffp-contract=off), so results are
// bit-identical to the reference's x86_64 scalar path for every row count.
#include "tn_common.h"

namespace tn {
namespace {

constexpr int QK = 32;

// Weight formats. On the device a weight is two planes: the codes of every
// block back to back in row-major block order (q4_0: the 16 nibble bytes of
// the GGML block; q8_0: its 32 int8 codes) and the f16 block scales.
enum WeightFormat { FMT_Q4_0 = 0, FMT_Q8_0 = 1 };
template <int FMT>
struct Fmt;
template <>
struct Fmt<FMT_Q4_0> {
    static constexpr int CODE_BYTES = 16, BLOB_BYTES = 18;
    static constexpr int GEMV_ITEMS = 3;  // (row, block) items per GEMV thread: 3 streamed best on C1 (76% of HBM, 71% for 4)
    static constexpr const char* name = "q4_0";
};
template <>
struct Fmt<FMT_Q8_0> {
    static constexpr int CODE_BYTES = 32, BLOB_BYTES = 34;
    static constexpr int GEMV_ITEMS = 3;  // 32-byte items: 96 bytes in flight per thread (5.40 TB/s at the C1 shape; 5.12 for 2, 5.34 for 4)
    static constexpr const char* name = "q8_0";
};

// ---- Rust cast semantics ---------------------------------------------------

// Truncation toward zero after clamping to the type's range, NaN to 0. The
// clamp and the NaN test are selects: written as early returns they became
// three nested exec-mask branches per element.
__device__ inline int sat_i8(float v) {  // `f as i8`
    const int q = (int)fminf(fmaxf(v, -128.0f), 127.0f);
    return v != v ? 0 : q;
}

__device__ inline int sat_u8(float v) {  // `f as u8`
    const int q = (int)fminf(fmaxf(v, 0.0f), 255.0f);
    return v != v ? 0 : q;
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
    // f32::max from 0 (k_quants.rs:676-705): a NaN lane counts as 0, so a
    // block of NaNs has amax 0, id 0 and zero codes, as the reference's has
    float a = fmaxf(0.0f, fabsf(v));
#pragma unroll
    for (int off = 16; off >= 1; off >>= 1) a = fmaxf(a, __shfl_xor(a, off, 32));
    float d = a / 127.0f;
    float id = (d != 0.0f) ? 1.0f / d : 0.0f;
    *dx = f16_to_f32(f16_from_f32(d));
    return sat_i8(roundf(v * id));
}

// ---- layout conversion --------------------------------------------------------

// GGML blocks (f16 d, then the codes) <-> the two planes, one thread per block.
template <int FMT>
__global__ void k_from_blob(const uint8_t* __restrict__ blob, int64_t nblocks, uint8_t* __restrict__ qs,
                            uint16_t* __restrict__ d) {
    constexpr int CB = Fmt<FMT>::CODE_BYTES;
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks) return;
    const uint8_t* s = blob + i * Fmt<FMT>::BLOB_BYTES;
    d[i] = (uint16_t)(s[0] | (s[1] << 8));
#pragma unroll
    for (int c = 0; c < CB / 16; c++) {
        uint32_t w[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const uint8_t* b = s + 2 + 16 * c + 4 * j;
            w[j] = (uint32_t)b[0] | ((uint32_t)b[1] << 8) | ((uint32_t)b[2] << 16) | ((uint32_t)b[3] << 24);
        }
        reinterpret_cast<uint4*>(qs + i * CB)[c] = make_uint4(w[0], w[1], w[2], w[3]);
    }
}

template <int FMT>
__global__ void k_to_blob(const uint8_t* __restrict__ qs, const uint16_t* __restrict__ d, int64_t nblocks,
                          uint8_t* __restrict__ blob) {
    constexpr int CB = Fmt<FMT>::CODE_BYTES;
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks) return;
    uint8_t* o = blob + i * Fmt<FMT>::BLOB_BYTES;
    uint16_t h = d[i];
    o[0] = (uint8_t)(h & 0xff);
    o[1] = (uint8_t)(h >> 8);
#pragma unroll
    for (int c = 0; c < CB / 16; c++) {
        const uint4 w = reinterpret_cast<const uint4*>(qs + i * CB)[c];
        const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int j = 0; j < 16; j++) o[2 + 16 * c + j] = (uint8_t)(ws[j >> 2] >> (8 * (j & 3)));
    }
}

// BlockQ4_0::from_float (k_quants.rs:241-277) and BlockQ8_0::from_float
// (k_quants.rs:676-705), one thread per block.
template <int FMT>
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
    if constexpr (FMT == FMT_Q8_0) {
        float amax = 0.0f;
#pragma unroll
        for (int j = 0; j < QK; j++) amax = fmaxf(amax, fabsf(v[j]));
        const float dd = amax / 127.0f;
        const float id = (dd != 0.0f) ? 1.0f / dd : 0.0f;  // the f32 d, not the f16 one
        d[i] = f16_from_f32(dd);
        uint32_t out[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < QK; j++) out[j >> 2] |= ((uint32_t)sat_i8(roundf(v[j] * id)) & 0xffu) << (8 * (j & 3));
        uint4* o = reinterpret_cast<uint4*>(qs + i * QK);
        o[0] = make_uint4(out[0], out[1], out[2], out[3]);
        o[1] = make_uint4(out[4], out[5], out[6], out[7]);
    } else {
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
}

// BlockQ4_0::to_float (k_quants.rs:219-239): (nib - 8) as f32 * f32(d);
// BlockQ8_0::to_float (k_quants.rs:659-674): q as f32 * f32(d). Both exact.
template <int FMT>
__global__ void k_dequantize(const uint8_t* __restrict__ qs, const uint16_t* __restrict__ d, int64_t nblocks,
                             float* __restrict__ out) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nblocks) return;
    float s = f16_to_f32(d[i]);
    float e[QK];
    if constexpr (FMT == FMT_Q8_0) {
        const uint4* src = reinterpret_cast<const uint4*>(qs + i * QK);
#pragma unroll
        for (int c = 0; c < 2; c++) {
            const uint4 w = src[c];
            const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int j = 0; j < 16; j++) e[16 * c + j] = (float)(int8_t)(ws[j >> 2] >> (8 * (j & 3))) * s;
        }
    } else {
        uint4 w = *reinterpret_cast<const uint4*>(qs + i * 16);
        uint32_t ws[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
        for (int j = 0; j < 16; j++) {
            uint32_t byte = (ws[j >> 2] >> (8 * (j & 3))) & 0xffu;
            e[j] = (float)((int)(byte & 0xf) - 8) * s;
            e[j + 16] = (float)((int)(byte >> 4) - 8) * s;
        }
    }
    float4* o = reinterpret_cast<float4*>(out + i * QK);
#pragma unroll
    for (int j = 0; j < QK / 4; j++) o[j] = make_float4(e[4 * j], e[4 * j + 1], e[4 * j + 2], e[4 * j + 3]);
}

// ---- decode GEMV (m <= GEMV_MAX_M) ---------------------------------------------
//
// One workgroup owns `rows` consecutive weight rows. Phase 1 quantises the MR
// activation rows into LDS (every workgroup repeats this: x is a few KB and
// L2-resident). Phase 2 streams the weight: the (row, block) items of the
// workgroup are a contiguous range of the codes plane, so consecutive lanes
// issue consecutive 16-byte loads (two per q8_0 item); each item's exact
// integer dot is 8 v_dot4_i32_i8 (q4_0: on the unsigned nibbles, minus
// 8 * sum(x codes)), and its scaled term goes to LDS. Phase 3 adds each
// output's terms in block order.

constexpr int GEMV_THREADS = 256;
constexpr int GEMV_MAX_M = 4;

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

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

__device__ inline int dot_block_q8(const uint4& w0, const uint4& w1, const int* __restrict__ xw) {
    // both operands hold the 32 int8 codes in natural order, 4 per dword
    int s = 0;
    s = __builtin_amdgcn_sdot4((int)w0.x, xw[0], s, false);
    s = __builtin_amdgcn_sdot4((int)w0.y, xw[1], s, false);
    s = __builtin_amdgcn_sdot4((int)w0.z, xw[2], s, false);
    s = __builtin_amdgcn_sdot4((int)w0.w, xw[3], s, false);
    s = __builtin_amdgcn_sdot4((int)w1.x, xw[4], s, false);
    s = __builtin_amdgcn_sdot4((int)w1.y, xw[5], s, false);
    s = __builtin_amdgcn_sdot4((int)w1.z, xw[6], s, false);
    s = __builtin_amdgcn_sdot4((int)w1.w, xw[7], s, false);
    return s;
}

// Phase 1 gives each 32-element block to 8 lanes, a float4 each: lane l of
// the workgroup holds elements 4 (l % 8) .. 4 (l % 8) + 3 of block l / 8 + 32 p
// in pass p, so for one row thread t holds elements 1024p + 4t .. 1024p + 4t + 3.
// The block's amax and code sum are 8-lane DPP reductions (no LDS round
// trip). The RMSNorm prologue's sum of squares uses that partition -- thread
// t adds the squares of its elements in order, then block_sum256 -- which is
// k_rmsnorm's order, so the fused norm reproduces it bit for bit.
//
// Prologues (MR == 1, f32 x only):
//   PRO_RMSNORM  x -> w * (x * r), r = 1/sqrt(sum(x^2)/K + eps)
//   PRO_SILU     x holds [gate | up] (2K floats) -> gate/(1 + exp(-gate)) * up
//   PRO_COMBINE  the row is the attention output h * D + d, merged from the
//                split partials: sum_s O_s 2^(m_s - M) * (1 / sum_s l_s 2^(m_s - M))
// Epilogue: y = acc (+ bias, or + resid: never both); y may alias resid (each
// output's thread reads its residual before writing it), never x. x must be 16-byte aligned.
constexpr int GEMV_HOLD = 4;  // passes of 32 blocks held in registers (K <= 4096 per row at once)
constexpr int GEMV_ONE = 0, GEMV_STREAM = 1, GEMV_PASSES = 2;  // k_gemv's SHAPE

// The best (value, index) over a workgroup of GEMV_THREADS threads, in
// thread 0 (arg_before's order: any pairing gives the same winner).
__device__ inline void block_arg_best(float& v, int& i) {
    __shared__ float sv[GEMV_THREADS / 64];
    __shared__ int si[GEMV_THREADS / 64];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float ov = __shfl_xor(v, off);
        const int oi = __shfl_xor(i, off);
        if (arg_before(ov, oi, v, i)) {
            v = ov;
            i = oi;
        }
    }
    if (lane == 0) {
        sv[w] = v;
        si[w] = i;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
#pragma unroll
        for (int k = 1; k < GEMV_THREADS / 64; k++)
            if (arg_before(sv[k], si[k], v, i)) {
                v = sv[k];
                i = si[k];
            }
    }
}

// The argmax epilogue after a workgroup's last tile: its best (value, index)
// goes to arg_v/arg_i[workgroup] with plain stores. k_argmax_parts, the next
// launch, reduces them: a kernel boundary is all the ordering the partials
// need. (Reducing them inside this launch, the workgroup drawing the last
// ticket reading the others' partials back, kept the lm_head on the step's
// critical path for the stores' acknowledgement and the ticket's round trip:
// 17.8 us for the C5 lm_head, against 9.0 us without the argmax.)
__device__ inline void gemv_argmax_epilogue(float v, int i, const GemvPro& po) {
    block_arg_best(v, i);
    if (threadIdx.x == 0) {
        po.arg_v[blockIdx.x] = v;
        po.arg_i[blockIdx.x] = i;
    }
}

// One workgroup: the best of `parts` (<= GEMV_ARG_MAX_PARTS) (value, index)
// partials of an n-wide row (argmax's order, arg_before), into state[3], then
// the decode step's advance as k_argmax<true, ...> does. Every load is issued
// at the start: the partials all at once, and the position with the prompt
// token it may pick, so that nothing waits on memory after the reduction.
__global__ __launch_bounds__(GEMV_THREADS) void k_argmax_parts(const float* __restrict__ arg_v,
                                                             const int32_t* __restrict__ arg_i, int parts, int n,
                                                             int32_t* state, int32_t* tokens,
                                                             const int32_t* __restrict__ prompt, int prompt_len,
                                                             int cap) {
    constexpr int PER = GEMV_ARG_MAX_PARTS / GEMV_THREADS;
    static_assert(PER * GEMV_THREADS == GEMV_ARG_MAX_PARTS, "partials per thread");
    int pos = 0, ptok = 0;
    if (threadIdx.x == 0) {
        pos = state[0] + 1;
        if (pos < prompt_len) ptok = prompt[pos];
    }
    float pv[PER];
    int pi[PER];
#pragma unroll
    for (int j = 0; j < PER; j++) {
        const int g = threadIdx.x + j * GEMV_THREADS;
        pv[j] = -INFINITY;
        pi[j] = INT32_MAX;
        if (g < parts) {
            pv[j] = arg_v[g];
            pi[j] = arg_i[g];
        }
    }
    float v = pv[0];
    int i = pi[0];
#pragma unroll
    for (int j = 1; j < PER; j++)
        if (arg_before(pv[j], pi[j], v, i)) {
            v = pv[j];
            i = pi[j];
        }
    block_arg_best(v, i);
    if (threadIdx.x == 0) {
        const int am = i < n ? i : 0;
        state[3] = am;
        llama_commit(state, tokens, pos, pos < prompt_len ? ptok : am, cap);
    }
}

// Epilogue ARG (MR == 1, f32 y; linear_decode_argmax): each workgroup's best
// output of y to po.arg_v/arg_i[workgroup], for k_argmax_parts.
// Epilogue GLU (MR == 1, f32 y, no bias or residual): the weight is
// [gate; up], 2N rows, and y[n] = silu(gate_n) * up_n over the N outputs
// (tn_silu_mul of the two halves, its arithmetic): a tile holds gate rows
// row0 .. row0+rows-1 and the matching up rows, and the thread that sums
// output n's gate row sums its up row too.
// SHAPE (launch_gemv picks):
//   GEMV_ONE     the activation rows fit the registers (MR * nb <= 32 * HOLD
//                blocks) and every workgroup has one row tile: the rows are
//                loaded once, ahead of the weights, in straight-line code,
//                and every weight load is unconditional, so the compiler's
//                waits for the rows do not also wait for the weights (the
//                decode step's GEMVs, latency-bound)
//   GEMV_STREAM  rows held, several tiles per workgroup with the next tile's
//                loads in flight (a streamed weight, bandwidth-bound; these
//                loads stay conditional: the unconditional form takes ten
//                more VGPRs, which costs a wave per SIMD here)
//   GEMV_PASSES  rows too long to hold, loaded in passes (twice with the
//                RMSNorm prologue), several tiles per workgroup
// Separate instantiations rather than branches: in one kernel the compiler
// joins the paths, and the waits on one path then count the other's loads.
template <int FMT, int MR, typename XT, int PRO, bool ARG = false, bool GLU = false, int SHAPE = GEMV_ONE>
__global__ __launch_bounds__(GEMV_THREADS) void k_gemv(const XT* __restrict__ x, int K, int nb,
                                                     const uint8_t* __restrict__ qs,
                                                     const uint16_t* __restrict__ dw, int N, int rows,
                                                     const float* __restrict__ bias, const float* resid, void* y,
                                                     int y_bf16, const GemvPro po) {
    static_assert(PRO == PRO_NONE || (MR == 1 && sizeof(XT) == 4), "prologues take one f32 row");
    static_assert(!ARG || MR == 1, "the argmax epilogue takes one row");
    static_assert(!GLU || (MR == 1 && !ARG), "the SiLU epilogue takes one row");
    constexpr int HOLD = PRO == PRO_COMBINE ? 1 : GEMV_HOLD;
    constexpr int ITEMS = Fmt<FMT>::GEMV_ITEMS, NV = Fmt<FMT>::CODE_BYTES / 16;
    constexpr bool HELD = SHAPE != GEMV_PASSES, ONE = SHAPE == GEMV_ONE;
    extern __shared__ __align__(16) char smem[];
    __shared__ float red[4];
    int* xq = reinterpret_cast<int*>(smem);               // [MR][K/4] packed int8 codes
    float* dxs = reinterpret_cast<float*>(xq + MR * (K / 4));  // [MR][nb]
    int* sxs = reinterpret_cast<int*>(dxs + MR * nb);     // [MR][nb]
    // [2][rows (GLU: 2 rows)][MR][nbp]: term rows padded to 16 bytes for the float4 reads of phase 3
    const int nbp = (nb + 3) & ~3;
    float* terms = reinterpret_cast<float*>(smem + ((MR * K + 8 * MR * nb + 15) & ~15));
    const int tid = threadIdx.x;
    // PRO_COMBINE: the weight items start at the first wave that merges no
    // block of the row (wave 3 at K = 576), so that the merging waves issue
    // only their partial loads and wait on nothing else (a wave's loads
    // complete in order)
    int wt = tid;
    if constexpr (PRO == PRO_COMBINE) {
        const int busy = 8 * (nb < 32 ? nb : 32);  // threads with a block in phase 1 (MR == 1)
        wt = (tid + GEMV_THREADS - (((busy + 63) & ~63) & (GEMV_THREADS - 1))) & (GEMV_THREADS - 1);
    }

    const int ntiles = (N + rows - 1) / rows;
    const int tstride = (int)gridDim.x;
    // two register buffers: the tile being computed and the next one in flight
    // (a third, two tiles ahead, measured slower: fewer resident waves)
    uint4 wv[ITEMS][NV], wn[ITEMS][NV];
    uint16_t dv[ITEMS], dn[ITEMS];
    constexpr int RW = GLU ? 2 : 1;  // weight rows per output
    // GEMV_ONE: the weight loads are unconditional buffer loads, one
    // descriptor per plane over the tile's span; an item past the tile reads
    // at an offset past the descriptor, which returns zero without a memory
    // access. Otherwise they are plain loads of the items that exist.
    constexpr uint32_t OOB = 0x80000000u;  // past every descriptor here (spans < 2^31 bytes)
    constexpr int NT = 2;                  // cache policy: non-temporal, the weights are streamed once
    auto gload = [&](int tile, uint4 (*wr)[NV], uint16_t* dr) {
        const int64_t row0 = (int64_t)tile * rows;
        const int nrows = (int)((N - row0) < rows ? (N - row0) : rows);
        const int total = RW * nrows * nb;
        if constexpr (ONE) {
            // GLU: the tile's up rows sit N rows after its gate rows
            const uint32_t span = (uint32_t)((GLU ? N + nrows : nrows) * nb);
            const buf_rsrc rq = make_rsrc(qs + row0 * nb * (16 * NV), span * (16u * NV));
            const buf_rsrc rd = make_rsrc(dw + row0 * nb, span * 2u);
#pragma unroll
            for (int it = 0; it < ITEMS; it++) {
                const int g0 = wt + it * GEMV_THREADS;
                const int g = (GLU && g0 >= nrows * nb) ? g0 + (N - nrows) * nb : g0;
                const bool on = g0 < total;
                const uint32_t qo = on ? (uint32_t)g * (16u * NV) : OOB, dof = on ? (uint32_t)g * 2u : OOB;
#if __HIP_DEVICE_COMPILE__
#pragma unroll
                for (int v = 0; v < NV; v++)
                    wr[it][v] = __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(rq, qo, 16 * v, NT));
                dr[it] = __builtin_amdgcn_raw_buffer_load_b16(rd, dof, 0, 0);
#else
                (void)rq, (void)rd, (void)qo, (void)dof;
#endif
            }
        } else {
            const uint4* qbase = reinterpret_cast<const uint4*>(qs) + row0 * nb * NV;
            const uint16_t* dbase = dw + row0 * nb;
#pragma unroll
            for (int it = 0; it < ITEMS; it++) {
                int g = wt + it * GEMV_THREADS;
                if (g < total) {
                    // GLU: items past the tile's gate rows are its up rows, N rows on
                    if (GLU && g >= nrows * nb) g += (N - nrows) * nb;
                    // streamed once: a non-temporal load keeps it from evicting x and the terms
#pragma unroll
                    for (int v = 0; v < NV; v++) {
                        const u32x4 t =
                            __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(qbase + g * NV + v));
                        wr[it][v] = make_uint4(t[0], t[1], t[2], t[3]);
                    }
                    dr[it] = dbase[g];
                }
            }
        }
    };
    int tile = (int)blockIdx.x;
    float pre_add = 0.0f;
    // the first tile's weight loads (and this thread's residual or bias for
    // it), in flight during the activation work; unconditional as gload's
    // (the grid never exceeds the tile count, so the first tile exists)
    // the bias or residual of this thread's first output of tile t (output
    // o = tid), an unconditional buffer load: resid and bias are not
    // combined, and with neither the descriptor is empty
    [[maybe_unused]] auto load_add = [&](int t) -> float {
        const int64_t row0 = (int64_t)t * rows;
        const int nrows = (int)((N - row0) < rows ? (N - row0) : rows);
        const int r = tid / MR, mr = tid - r * MR;
        const float* src = bias ? bias : resid;
        const buf_rsrc rb = make_rsrc(src, src ? (uint32_t)((bias ? 1 : MR) * N) * 4u : 0u);
        const uint32_t off = tid < nrows * MR ? (uint32_t)((bias ? 0 : (int64_t)mr * N) + row0 + r) * 4u : OOB;
#if __HIP_DEVICE_COMPILE__
        return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rb, off, 0, 0));
#else
        (void)rb, (void)off;
        return 0.0f;
#endif
    };
    auto first_loads = [&]() {
        if constexpr (ONE) {
            gload(tile, wv, dv);
            pre_add = load_add(tile);
        } else if (tile < ntiles) {  // always true; the branch keeps this shape at 64 VGPRs (66 without)
            gload(tile, wv, dv);
            const int64_t row0 = (int64_t)tile * rows;
            const int nrows = (int)((N - row0) < rows ? (N - row0) : rows);
            if (tid < nrows * MR) {
                const int r = tid / MR, mr = tid - r * MR;
                if (bias) pre_add = bias[row0 + r];
                if (resid) pre_add = resid[(int64_t)mr * N + row0 + r];  // resid and bias are not combined
            }
        }
    };

    // phase 1: Q8_0 of the MR activation rows (after the prologue)
    {
        const int g8 = tid & 7, slot = tid >> 3;
        const int nblk = MR * nb, npass = (nblk + 31) / 32;
        // a row that fits the registers is loaded before the weights, whose
        // loads would otherwise stand in front of it in the memory pipeline
        // (the merge of the attention partials, PRO_COMBINE, after them: its
        // waves hold no weight items)
        (void)npass;
        float4 xv[HOLD], av[HOLD];  // the row, and the prologue's second operand
        int ns = 0;
        if constexpr (PRO == PRO_COMBINE) {
            int len = *po.len;
            len = len < 0 ? 0 : (len > po.cap ? po.cap : len);
            ns = (len + STEP_SPLIT - 1) / STEP_SPLIT;
            ns = ns < po.nsplit ? ns : po.nsplit;
        }
        // PRO_COMBINE: row block blk merged over the splits. Every split's
        // (m, l) and O piece is in flight at once, read before the length is
        // known (splits past it are not used). The loads are unconditional --
        // a split index past the launch's count reads the last split's row
        // again, a block past the row's reads its last block, and neither is
        // used -- so the compiler counts the loads in flight exactly.
        auto merge_block = [&](int blk) -> float4 {
            const int bc = blk < nblk ? blk : nblk - 1;
            const int o32 = bc * QK + 4 * g8;  // MR == 1: the element offset in the row
            const int h = o32 >> po.head_shift, d = o32 & ((1 << po.head_shift) - 1);
            // one descriptor per plane: a lane's (head, column) is its vector
            // offset and a split's row the scalar one
            const uint32_t rows = (uint32_t)(K >> po.head_shift) * (uint32_t)po.nsplit;
            const buf_rsrc rml = make_rsrc(po.part_ml, rows * 8u);
            const buf_rsrc ro = make_rsrc(po.part_o, rows * (uint32_t)po.head_dim * 4u);
            const uint32_t vml = (uint32_t)(h * po.nsplit) * 8u;
            const uint32_t vo = ((uint32_t)(h * po.nsplit) * (uint32_t)po.head_dim + (uint32_t)d) * 4u;
            u32x2 mlr[STEP_MAX_SPLITS] = {};
            u32x4 orr[STEP_MAX_SPLITS] = {};
#if __HIP_DEVICE_COMPILE__
#pragma unroll
            for (int sp = 0; sp < STEP_MAX_SPLITS; sp++) {
                const uint32_t spc = (uint32_t)(sp < po.nsplit ? sp : po.nsplit - 1);
                mlr[sp] = __builtin_amdgcn_raw_buffer_load_b64(rml, vml, spc * 8u, 0);
            }
#pragma unroll
            for (int sp = 0; sp < STEP_MAX_SPLITS; sp++) {
                const uint32_t spc = (uint32_t)(sp < po.nsplit ? sp : po.nsplit - 1);
                orr[sp] = __builtin_amdgcn_raw_buffer_load_b128(ro, vo, spc * (uint32_t)po.head_dim * 4u, 0);
            }
#else
            (void)rml, (void)ro, (void)vml, (void)vo;
#endif
            // every load issued before any result is used
            __builtin_amdgcn_sched_barrier(0);
            float2 ml[STEP_MAX_SPLITS];
            float4 o4[STEP_MAX_SPLITS];
#pragma unroll
            for (int sp = 0; sp < STEP_MAX_SPLITS; sp++) {
                ml[sp] = make_float2(__uint_as_float(mlr[sp][0]), __uint_as_float(mlr[sp][1]));
                o4[sp] = make_float4(__uint_as_float(orr[sp][0]), __uint_as_float(orr[sp][1]),
                                     __uint_as_float(orr[sp][2]), __uint_as_float(orr[sp][3]));
            }
            float mm = -INFINITY;
#pragma unroll
            for (int sp = 0; sp < STEP_MAX_SPLITS; sp++)
                if (sp < ns) mm = fmaxf(mm, ml[sp].x);
            const float mu = (mm == -INFINITY) ? 0.0f : mm;
            float tl = 0.0f;
            float4 acc = make_float4(0.f, 0.f, 0.f, 0.f);
            // One wave issues this whole merge, so its instruction count is
            // its time: the hardware exp2 (a factor below 2^-126 becomes 0,
            // where the library's would keep a subnormal), and one
            // reciprocal of the sum for the four columns.
#pragma unroll
            for (int sp = 0; sp < STEP_MAX_SPLITS; sp++) {
                if (sp < ns) {
                    const float f = __builtin_amdgcn_exp2f(ml[sp].x - mu);
                    tl = tl + ml[sp].y * f;
                    acc.x = acc.x + o4[sp].x * f;
                    acc.y = acc.y + o4[sp].y * f;
                    acc.z = acc.z + o4[sp].z * f;
                    acc.w = acc.w + o4[sp].w * f;
                }
            }
            const float inv = 1.0f / tl;
            return make_float4(acc.x * inv, acc.y * inv, acc.z * inv, acc.w * inv);
        };
        auto load_passes = [&](int p0) {
#pragma unroll
            for (int u = 0; u < HOLD; u++) {
                const int blk = (p0 + u) * 32 + slot;
                if constexpr (PRO == PRO_COMBINE) {
                    // waves with no block of the row skip it
                    if (__builtin_amdgcn_readfirstlane(blk) < nblk) xv[u] = merge_block(blk);
                } else if (blk < nblk) {
                    const int mr = blk / nb, b = blk - mr * nb;
                    const int64_t off = (int64_t)mr * K + b * QK + 4 * g8;
                    if constexpr (sizeof(XT) == 4) {
                        xv[u] = *reinterpret_cast<const float4*>(x + off);
                    } else {
                        const uint2 h = *reinterpret_cast<const uint2*>(x + off);
                        xv[u] = make_float4(bf16_to_f32((uint16_t)(h.x & 0xffffu)), bf16_to_f32((uint16_t)(h.x >> 16)),
                                            bf16_to_f32((uint16_t)(h.y & 0xffffu)), bf16_to_f32((uint16_t)(h.y >> 16)));
                    }
                    if constexpr (PRO == PRO_RMSNORM) av[u] = *reinterpret_cast<const float4*>(po.w + off);
                    if constexpr (PRO == PRO_SILU)
                        av[u] = *reinterpret_cast<const float4*>(reinterpret_cast<const float*>(x) + K + off);
                }
            }
        };
        if constexpr (PRO == PRO_COMBINE) {
            first_loads();
            if constexpr (HELD) load_passes(0);
        } else {
            if constexpr (HELD) load_passes(0);
            first_loads();
        }
        // thread t's squares in order (k_rmsnorm's), over the passes held in xv
        auto ss_pass = [&](int p0, float& ss) {
#pragma unroll
            for (int u = 0; u < HOLD; u++) {
                if ((p0 + u) * 32 + slot < nblk) {
                    ss = ss + xv[u].x * xv[u].x;
                    ss = ss + xv[u].y * xv[u].y;
                    ss = ss + xv[u].z * xv[u].z;
                    ss = ss + xv[u].w * xv[u].w;
                }
            }
        };
        int8_t* xb = reinterpret_cast<int8_t*>(xq);
        auto q8_pass = [&](int p0, float r) {
#pragma unroll
            for (int u = 0; u < HOLD; u++) {
                const int blk = (p0 + u) * 32 + slot;
                if (blk < nblk) {  // uniform over the block's 8 lanes
                    float e[4] = {xv[u].x, xv[u].y, xv[u].z, xv[u].w};
                    const float o[4] = {av[u].x, av[u].y, av[u].z, av[u].w};
                    float amax = 0.0f;
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        if constexpr (PRO == PRO_RMSNORM) e[i] = o[i] * (e[i] * r);
                        if constexpr (PRO == PRO_SILU) e[i] = (e[i] / (1.0f + expf(-e[i]))) * o[i];
                        amax = fmaxf(amax, fabsf(e[i]));
                    }
                    // BlockQ8_0::from_float (k_quants.rs:676-705)
                    amax = group8_max(amax);
                    const float d = amax / 127.0f;
                    const float id = (d != 0.0f) ? 1.0f / d : 0.0f;
                    uint32_t wd = 0;
                    int sq = 0;
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const int q = sat_i8(roundf(e[i] * id));
                        sq += q;
                        wd |= ((uint32_t)q & 0xffu) << (8 * i);
                    }
                    sq = group8_sum(sq);
                    reinterpret_cast<uint32_t*>(xb)[blk * 8 + g8] = wd;  // blocks of all rows are contiguous
                    if (g8 == 0) {
                        dxs[blk] = f16_round_hw(d);  // d is never NaN: amax ignores NaN
                        sxs[blk] = sq;
                    }
                }
            }
        };
        if constexpr (HELD) {
            // the held row in straight-line code: the waits for the row count
            // only the loads issued after it
            float r = 0.0f;
            if constexpr (PRO == PRO_RMSNORM) {
                float ss = 0.0f;
                ss_pass(0, ss);
                r = rms_scale(block_sum256(ss, red), K, po.eps);
            }
            q8_pass(0, r);
        } else {
            float r = 0.0f;
            if constexpr (PRO == PRO_RMSNORM) {
                float ss = 0.0f;
                for (int p0 = 0; p0 < npass; p0 += HOLD) {
                    load_passes(p0);
                    ss_pass(p0, ss);
                }
                r = rms_scale(block_sum256(ss, red), K, po.eps);
            }
            for (int p0 = 0; p0 < npass; p0 += HOLD) {
                load_passes(p0);
                q8_pass(p0, r);
            }
        }
    }
    __syncthreads();

    // phase 2/3, persistent over row tiles: the next tile's weight loads are in
    // flight while this tile's terms are computed and summed; the terms live
    // in two LDS buffers, so one barrier per tile suffices
    float best_v = -INFINITY;  // ARG: this thread's best output so far
    int best_i = INT32_MAX;    // loses every tie against a real output
    for (int buf = 0; tile < ntiles; tile += tstride, buf ^= 1) {
        // GEMV_ONE: this is the workgroup's only tile
        if constexpr (!ONE) {
            if (tile + tstride < ntiles) gload(tile + tstride, wn, dn);
        }
        const int64_t row0 = (int64_t)tile * rows;
        const int nrows = (int)((N - row0) < rows ? (N - row0) : rows);
        const int total = RW * nrows * nb;
        float* tb = terms + buf * RW * rows * MR * nbp;
#pragma unroll
        for (int it = 0; it < ITEMS; it++) {
            const int g = wt + it * GEMV_THREADS;
            if (g < total) {
                const int r = g / nb, b = g - r * nb;
                const float dwf = f16_bits_hw(dv[it]);
#pragma unroll
                for (int mr = 0; mr < MR; mr++) {
                    const int* xw = xq + mr * (K / 4) + b * 8;
                    int s;
                    if constexpr (FMT == FMT_Q8_0)
                        s = dot_block_q8(wv[it][0], wv[it][1], xw);
                    else
                        s = dot_block(wv[it][0], xw) - 8 * sxs[mr * nb + b];
                    float t = (float)s * dwf;
                    t = t * dxs[mr * nb + b];
                    tb[(r * MR + mr) * nbp + b] = t;
                }
            }
        }
        __syncthreads();
        // each output's terms in block order, read 16 at a time
        // one row's terms in block order
        auto ordered_sum = [&](const float* tr) {
            float acc = 0.0f;
            int b = 0;
            for (; b + 16 <= nb; b += 16) {
                float4 t4[4];
#pragma unroll
                for (int j = 0; j < 4; j++) t4[j] = reinterpret_cast<const float4*>(tr + b)[j];
#pragma unroll
                for (int j = 0; j < 4; j++) {
                    acc = acc + t4[j].x;
                    acc = acc + t4[j].y;
                    acc = acc + t4[j].z;
                    acc = acc + t4[j].w;
                }
            }
            for (; b + 4 <= nb; b += 4) {
                const float4 t4 = *reinterpret_cast<const float4*>(tr + b);
                acc = acc + t4.x;
                acc = acc + t4.y;
                acc = acc + t4.z;
                acc = acc + t4.w;
            }
            for (; b < nb; b++) acc = acc + tr[b];
            return acc;
        };
        auto out_row = [&](int o, float add) {
            const int r = o / MR, mr = o - r * MR;
            const int64_t n = row0 + r;
            float acc = ordered_sum(tb + (r * MR + mr) * nbp);
            if constexpr (GLU) {
                // silu(gate) * up, tn_silu_mul's arithmetic
                const float up = ordered_sum(tb + (nrows + r) * nbp);
                acc = (acc / (1.0f + expf(-acc))) * up;
            }
            if (bias || resid) acc = acc + add;
            if constexpr (ARG) {
                if (arg_before(acc, (int)n, best_v, best_i)) {
                    best_v = acc;
                    best_i = (int)n;
                }
            }
            if (y_bf16)
                reinterpret_cast<uint16_t*>(y)[(int64_t)mr * N + n] = bf16_from_f32(acc);
            else
                reinterpret_cast<float*>(y)[(int64_t)mr * N + n] = acc;
        };
        if constexpr (ONE) {
            // the thread's first output outside the loop: its add was loaded
            // unconditionally, before the weights, and its wait counts them out
            if (tid < nrows * MR) out_row(tid, pre_add);
            for (int o = tid + GEMV_THREADS; o < nrows * MR; o += GEMV_THREADS) {
                const int r = o / MR, mr = o - r * MR;
                const int64_t n = row0 + r;
                out_row(o, bias ? bias[n] : resid ? resid[(int64_t)mr * N + n] : 0.0f);
            }
        } else {
            for (int o = tid; o < nrows * MR; o += GEMV_THREADS) {
                const int r = o / MR, mr = o - r * MR;
                const int64_t n = row0 + r;
                float add = pre_add;
                if (tile != (int)blockIdx.x || o != tid)
                    add = bias ? bias[n] : resid ? resid[(int64_t)mr * N + n] : 0.0f;
                out_row(o, add);
            }
        }
        if constexpr (ONE) break;  // the launch gives every workgroup one tile
#pragma unroll
        for (int it = 0; it < ITEMS; it++) {
#pragma unroll
            for (int v = 0; v < NV; v++) wv[it][v] = wn[it][v];
            dv[it] = dn[it];
        }
    }
    if constexpr (ARG) gemv_argmax_epilogue(best_v, best_i, po);
}

// ---- prefill GEMM on MFMA ---------------------------------------------------------
//
// Prepass: every activation row is quantised to Q8_0 once, into bf16 codes
// (|q| <= 127 is exact in bf16) laid out per block in the order the MFMA
// operand wants, plus the f32 block scales transposed [nb][M_pad].
//
// Main kernel: a 128x128 output tile per workgroup, four waves as 2x2, each
// wave 64x64 = 4x4 tiles of v_mfma_f32_16x16x32_bf16. The K loop walks blocks
// in order, double-buffered in LDS: the next block's loads are issued into
// registers before the current block is computed.
//
// Exactness. The weight codes enter the MFMA as bf16(128 + nib), built by one
// byte permute per two nibbles (the bf16 bit pattern of 128 + n is 0x4300 | n),
// and the accumulator starts at -136 * sum_j(x codes) for the row, so the MFMA
// returns sum_j (nib_j - 8) * q_j = the block's integer dot S_b exactly: every
// product (<= 143*127), every partial sum and the start value stay below 2^24
// in magnitude, so no fp32 step rounds. S_b then gets the reference's two
// roundings, (S_b * d_w) * d_x, and one addition into the running sum, in
// block order.
//
// K-slot order: MFMA lane group g (lanes 16g..16g+15) holds 8 of the 32 block
// elements, {4g..4g+3, 16+4g..16+4g+3}: the low and high nibbles of weight
// bytes 4g..4g+3. The activation codes are stored in the same order, so the
// two operands agree element for element.
//
// Tile order is XCD-aware: consecutive workgroups go to different XCDs, so the
// workgroup index is remapped such that each XCD works on a contiguous range
// of weight columns and reads those columns into its own L2 once for all the
// row tiles.

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int GM_BM = 128, GM_BN = 128, GM_THREADS = 256;
constexpr int NUM_XCD = 8;

__device__ inline int kslot_of_element(int e) {  // element (0..31) -> K slot
    return e < 16 ? 8 * (e >> 2) + (e & 3) : 8 * ((e - 16) >> 2) + 4 + (e & 3);
}

template <typename XT>
__global__ __launch_bounds__(256) void k_q8_rows(const XT* __restrict__ x, int M, int M_pad, int K, int nb,
                                               uint16_t* __restrict__ xc, float* __restrict__ dxT,
                                               float* __restrict__ corrT) {
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
    int s = q;
#pragma unroll
    for (int off = 16; off >= 1; off >>= 1) s += __shfl_xor(s, off, 32);
    xc[blk * QK + kslot_of_element(lane)] = (uint16_t)(__builtin_bit_cast(uint32_t, (float)q) >> 16);
    if (lane == 0) {
        dxT[(int64_t)b * M_pad + row] = dx;
        corrT[(int64_t)b * M_pad + row] = (float)(-136 * s);
    }
}

// Eight consecutive activations as floats: 16 bytes of bf16 or 32 of f32
// (p 16-byte aligned).
template <typename XT>
__device__ inline void load_x8(const XT* p, float (&v)[8]);
template <>
__device__ inline void load_x8<float>(const float* p, float (&v)[8]) {
    const float4 a = reinterpret_cast<const float4*>(p)[0], b = reinterpret_cast<const float4*>(p)[1];
    v[0] = a.x, v[1] = a.y, v[2] = a.z, v[3] = a.w, v[4] = b.x, v[5] = b.y, v[6] = b.z, v[7] = b.w;
}
template <>
__device__ inline void load_x8<uint16_t>(const uint16_t* p, float (&v)[8]) {
    const uint4 a = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        v[2 * i] = __builtin_bit_cast(float, w[i] << 16);
        v[2 * i + 1] = __builtin_bit_cast(float, w[i] & 0xffff0000u);
    }
}

// The Q8_0 codes of one block held by four lanes, eight elements each: the
// block's amax (order-free), d = amax/127, id = 1/d and the rounding are
// q8_0_lane's, element for element, so the codes, the scale and the code sum
// are identical; the sum comes back through `s`.
__device__ inline void q8_0_quad(const float (&v)[8], int (&q)[8], float* dx, int* s) {
    float a = 0.0f;  // f32::max from 0: NaNs are skipped (k_quants.rs:676-705)
#pragma unroll
    for (int e = 0; e < 8; e++) a = fmaxf(a, fabsf(v[e]));
    a = fmaxf(a, __shfl_xor(a, 1, 4));
    a = fmaxf(a, __shfl_xor(a, 2, 4));
    const float d = a / 127.0f;
    const float id = (d != 0.0f) ? 1.0f / d : 0.0f;
    *dx = f16_to_f32(f16_from_f32(d));
    int sum = 0;
#pragma unroll
    for (int e = 0; e < 8; e++) {
        q[e] = sat_i8(roundf(v[e] * id));
        sum += q[e];
    }
    sum += __shfl_xor(sum, 1, 4);
    sum += __shfl_xor(sum, 2, 4);
    *s = sum;
}

// How the prepass finds a row's activations (XM_* in tn_common.h). XM_ROWS:
// row r is x[r][0..K). XM_GLU: x holds [M][2K] rows (gate | up) and the
// activation is silu(gate) * up, k_silu_mul's arithmetic (decode.hip).
// XM_HEADS: x is an attention output [K / hd][M][hd] (head-major) and row r
// is its heads' rows of token r side by side. The last two let a prompt's
// down and o projections read their producers' outputs without a copy in
// between.

// k_q8_rows for a 16-byte aligned x: four lanes per (row, block), one 16- or
// 32-byte load each. Lane part p holds elements 8p .. 8p+7, whose K slots are
// two runs of four (kslot_of_element), written as two 8-byte stores.
template <typename XT, int XM = XM_ROWS>
__global__ __launch_bounds__(256) void k_q8_rows_v(const XT* __restrict__ x, int M, int M_pad, int K, int nb,
                                                   uint16_t* __restrict__ xc, float* __restrict__ dxT,
                                                   float* __restrict__ corrT, int hd = 0) {
    const int64_t blk = (int64_t)blockIdx.x * (blockDim.x >> 2) + (threadIdx.x >> 2);
    const int part = threadIdx.x & 3;
    if (blk >= (int64_t)M_pad * nb) return;  // the four lanes of a block leave together
    const int row = (int)(blk / nb), b = (int)(blk - (int64_t)row * nb);
    float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (row < M) {
        if constexpr (XM == XM_GLU) {
            float g[8], u[8];
            load_x8<XT>(x + (int64_t)row * 2 * K + b * QK + 8 * part, g);
            load_x8<XT>(x + (int64_t)row * 2 * K + K + b * QK + 8 * part, u);
#pragma unroll
            for (int e = 0; e < 8; e++) v[e] = (g[e] / (1.0f + expf(-g[e]))) * u[e];
        } else if constexpr (XM == XM_HEADS) {
            const int e0 = b * QK, h = e0 / hd;
            load_x8<XT>(x + ((int64_t)h * M + row) * hd + (e0 - h * hd) + 8 * part, v);
        } else {
            load_x8<XT>(x + (int64_t)row * K + b * QK + 8 * part, v);
        }
    }
    int q[8], s;
    float dx;
    q8_0_quad(v, q, &dx, &s);
    if (row >= M) dx = 0.0f;
    auto code = [](int c) { return __builtin_bit_cast(uint32_t, (float)c) >> 16; };
    const int slot0 = kslot_of_element(8 * part), slot1 = kslot_of_element(8 * part + 4);
    *reinterpret_cast<uint2*>(xc + blk * QK + slot0) =
        make_uint2(code(q[0]) | (code(q[1]) << 16), code(q[2]) | (code(q[3]) << 16));
    *reinterpret_cast<uint2*>(xc + blk * QK + slot1) =
        make_uint2(code(q[4]) | (code(q[5]) << 16), code(q[6]) | (code(q[7]) << 16));
    if (part == 0) {
        dxT[(int64_t)b * M_pad + row] = dx;
        corrT[(int64_t)b * M_pad + row] = (float)(-136 * s);
    }
}

// bytes 0,1 (or 2,3) of x -> the bf16 pair (128 + byte0, 128 + byte1): the
// high byte of each half comes from the constant 0x43
__device__ inline uint32_t codes_pair01(uint32_t x) { return __builtin_amdgcn_perm(0x43434343u, x, 0x04010400u); }
__device__ inline uint32_t codes_pair23(uint32_t x) { return __builtin_amdgcn_perm(0x43434343u, x, 0x04030402u); }

constexpr int GM_AS = QK + 8;  // LDS row stride (bf16) of the code tiles: 80 B, conflict-free b128 reads
constexpr int GM_RS = 4;       // K blocks whose operands are in flight ahead of the one computed

// WR x WC waves over a GM_BM x BN tile, each wave TI x TJ MFMA tiles of
// 16x16: <2, 2, 4> is 128 x 128 (waves of 64 x 64), <4, 1, 7> is 128 x 112
// (waves of 32 x 112), chosen at launch so the tiles fill the device evenly.
// Products with few rows and columns (a prompt's projections) take narrow
// tiles, <4, 1, TJ> with 16 TJ columns, so that more workgroups share the
// work: each walks every K block in order whatever its tile, so the number
// of workgroups, not their width, sets such a call's time.
template <int WR, int WC, int TJ>
__global__ __launch_bounds__(GM_THREADS) void k_gemm(const uint16_t* __restrict__ xc,
                                                    const float* __restrict__ dxT,
                                                    const float* __restrict__ corrT, int M, int M_pad, int nb,
                                                    const uint8_t* __restrict__ qs,
                                                    const uint16_t* __restrict__ dw, int N,
                                                    const float* __restrict__ bias, void* y, int y_bf16,
                                                    const float* resid = nullptr) {
    static_assert(WR * WC == GM_THREADS / 64, "one wave per sub-tile");
    constexpr int TI = GM_BM / (16 * WR);  // MFMA row tiles per wave
    constexpr int BN = 16 * TJ * WC;       // columns per workgroup
    static_assert(2 * BN <= GM_THREADS && GM_BM + BN <= GM_THREADS, "staging threads");
    __shared__ __align__(16) uint16_t sA[2][GM_BM * GM_AS];
    __shared__ __align__(16) uint16_t sB[2][BN * GM_AS];
    __shared__ __align__(16) float sdx[2][GM_BM];
    __shared__ __align__(16) float scr[2][GM_BM];
    __shared__ __align__(16) float sdw[2][BN];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WC, wn = wave % WC;  // wave's (16 TI) x (16 TJ) sub-tile
    const int lrow = lane & 15, lgrp = lane >> 4;

    // XCD-aware tile order: workgroup id -> (row tile, column tile)
    const int mt = (int)gridDim.y;              // row tiles
    const int ntot = (int)(gridDim.x * gridDim.y);
    const int id = (int)(blockIdx.y * gridDim.x + blockIdx.x);
    int tile = id;
    if (ntot % NUM_XCD == 0) tile = (id % NUM_XCD) * (ntot / NUM_XCD) + id / NUM_XCD;
    const int m0 = (tile % mt) * GM_BM, n0 = (tile / mt) * BN;

    f32x4 acc[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; i++)
#pragma unroll
        for (int j = 0; j < TJ; j++) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};

    // Per-thread staging registers, GM_RS register sets: block b's operands are
    // requested GM_RS blocks before they are computed (about 1.7 us of
    // memory latency against about 0.4 us of work per block), then stored to
    // the LDS double buffer one block ahead. The set index is a compile-time
    // constant (the K loop is unrolled by GM_RS), so the sets stay in VGPRs.
    // one register set: two 16-byte chunks of activation codes, 8 bytes of
    // weight nibbles (threads < 2 BN), and (threads < GM_BM) the row's Q8_0
    // scale and accumulator start or (GM_BM <= threads < GM_BM + BN) the
    // column's f16 weight scale
    const int bcol = tid >> 1, bhalf = tid & 1;
    const int ar0 = tid >> 2, ar1 = (tid + GM_THREADS) >> 2, apart = tid & 3;  // the two A chunks
    // Every load is an unconditional buffer load: a descriptor per operand
    // over this tile's rows or columns, a per-thread offset computed once and
    // the block's offset in a scalar register, so a step costs no address
    // arithmetic. What lies past a descriptor's range (columns past N, the
    // threads that stage nothing of an operand, blocks past the last) reads
    // as zero and is not used; loads behind branches made the compiler's wait
    // counting fall back to waiting for every load in flight.
    const uint32_t OOB = 0x80000000u;  // an offset past every range here
    const int ncols = min(BN, N - n0);
    const buf_rsrc ra = make_rsrc(xc + (int64_t)m0 * nb * QK, (uint32_t)(GM_BM * nb * QK * 2));
    const buf_rsrc rw = make_rsrc(qs + (int64_t)n0 * nb * 16, (uint32_t)(ncols * nb * 16));
    const buf_rsrc rdx = make_rsrc(dxT + m0, (uint32_t)(((int64_t)nb * M_pad - m0) * 4));
    const buf_rsrc rcr = make_rsrc(corrT + m0, (uint32_t)(((int64_t)nb * M_pad - m0) * 4));
    const buf_rsrc rdw = make_rsrc(dw + (int64_t)n0 * nb, (uint32_t)(ncols * nb * 2));
    const uint32_t va0 = (uint32_t)((ar0 * nb * QK + apart * 8) * 2), va1 = (uint32_t)((ar1 * nb * QK + apart * 8) * 2);
    const uint32_t vw = bcol < BN ? (uint32_t)(bcol * nb * 16 + bhalf * 8) : OOB;
    const uint32_t vs = tid < GM_BM ? (uint32_t)(tid * 4) : OOB;
    const uint32_t vd = (tid >= GM_BM && tid < GM_BM + BN) ? (uint32_t)((tid - GM_BM) * nb * 2) : OOB;
    auto gload = [&](int b, uint4& a0, uint4& a1, uint2& w, float& dx, float& corr, uint32_t& dws)
                     __attribute__((always_inline)) {
        // Blocks past the last (the prefetches of the final steps, and the
        // first four when nb < 4) are clamped to the last block. The block
        // offset travels in the scalar offset, which the descriptor's range
        // check does not cover, so it must itself stay inside the operands.
        // The clamped data lands in an LDS buffer no later step reads.
        b = min(b, nb - 1);
#if __HIP_DEVICE_COMPILE__
        typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
        typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
        const u32x4_t x0 = __builtin_amdgcn_raw_buffer_load_b128(ra, va0, (uint32_t)(b * QK * 2), 0);
        const u32x4_t x1 = __builtin_amdgcn_raw_buffer_load_b128(ra, va1, (uint32_t)(b * QK * 2), 0);
        const u32x2_t ww = __builtin_amdgcn_raw_buffer_load_b64(rw, vw, (uint32_t)(b * 16), 0);
        a0 = make_uint4(x0[0], x0[1], x0[2], x0[3]);
        a1 = make_uint4(x1[0], x1[1], x1[2], x1[3]);
        w = make_uint2(ww[0], ww[1]);
        dx = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rdx, vs, (uint32_t)(b * M_pad * 4), 0));
        corr = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rcr, vs, (uint32_t)(b * M_pad * 4), 0));
        dws = __builtin_amdgcn_raw_buffer_load_b16(rdw, vd, (uint32_t)(b * 2), 0);
#else
        (void)b;
        a0 = a1 = make_uint4(0, 0, 0, 0);
        w = make_uint2(0, 0);
        dx = corr = 0.0f;
        dws = 0;
#endif
    };
    auto lstore = [&](int buf, const uint4& a0, const uint4& a1, const uint2& w, float dx, float corr,
                      uint32_t dws) __attribute__((always_inline)) {
        *reinterpret_cast<uint4*>(&sA[buf][ar0 * GM_AS + apart * 8]) = a0;
        *reinterpret_cast<uint4*>(&sA[buf][ar1 * GM_AS + apart * 8]) = a1;
        // weight dwords g = 2*bhalf, 2*bhalf+1 -> K slots 8g..8g+7 each
        const uint32_t w0 = w.x, w1 = w.y;
        const uint32_t lo0 = w0 & 0x0f0f0f0fu, hi0 = (w0 >> 4) & 0x0f0f0f0fu;
        const uint32_t lo1 = w1 & 0x0f0f0f0fu, hi1 = (w1 >> 4) & 0x0f0f0f0fu;
        if (bcol < BN) {
            uint4* dst = reinterpret_cast<uint4*>(&sB[buf][bcol * GM_AS + bhalf * 16]);
            dst[0] = make_uint4(codes_pair01(lo0), codes_pair23(lo0), codes_pair01(hi0), codes_pair23(hi0));
            dst[1] = make_uint4(codes_pair01(lo1), codes_pair23(lo1), codes_pair01(hi1), codes_pair23(hi1));
        }
        if (tid < GM_BM) {
            sdx[buf][tid] = dx;
            scr[buf][tid] = corr;
        } else if (tid < GM_BM + BN) {
            sdw[buf][tid - GM_BM] = f16_bits_hw((uint16_t)dws);
        }
    };
    // one K block from LDS buffer `buf`: the exact block dot on MFMA, then
    // the reference's two roundings and the ordered addition
    auto compute = [&](int buf) __attribute__((always_inline)) {
        constexpr int WROWS = 16 * TI, WCOLS = 16 * TJ;  // the wave's sub-tile
        bf16x8 afr[TI], bfr[TJ];
#pragma unroll
        for (int i = 0; i < TI; i++)
            afr[i] = *reinterpret_cast<const bf16x8*>(&sA[buf][(wm * WROWS + i * 16 + lrow) * GM_AS + lgrp * 8]);
#pragma unroll
        for (int j = 0; j < TJ; j++)
            bfr[j] = *reinterpret_cast<const bf16x8*>(&sB[buf][(wn * WCOLS + j * 16 + lrow) * GM_AS + lgrp * 8]);
        float dwv[TJ];
        f32x4 dxv[TI], crv[TI];
#pragma unroll
        for (int j = 0; j < TJ; j++) dwv[j] = sdw[buf][wn * WCOLS + j * 16 + lrow];
#pragma unroll
        for (int i = 0; i < TI; i++) {
            dxv[i] = *reinterpret_cast<const f32x4*>(&sdx[buf][wm * WROWS + i * 16 + lgrp * 4]);
            crv[i] = *reinterpret_cast<const f32x4*>(&scr[buf][wm * WROWS + i * 16 + lgrp * 4]);
        }
        // C[row][col]: col = lane & 15 (weight column), row = 4*(lane>>4) + r;
        // A = activation rows, B = weight columns; C starts at -136*sum(x codes).
        // Tile k + 1's product is issued before tile k's recurrence, in that
        // order (the scheduling barriers pin it), so each product runs on the
        // matrix core under the previous tile's VALU work.
        constexpr int NT = TI * TJ;
        f32x4 sv[2];
        sv[0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(afr[0], bfr[0], crv[0], 0, 0, 0);
#pragma unroll
        for (int k = 0; k < NT; k++) {
            const int i = k / TJ, j = k % TJ;
            if (k + 1 < NT) {
                const int i1 = (k + 1) / TJ, j1 = (k + 1) % TJ;
                __builtin_amdgcn_sched_barrier(0);
                sv[(k + 1) & 1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(afr[i1], bfr[j1], crv[i1], 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int r = 0; r < 4; r++) {
                float t = sv[k & 1][r] * dwv[j];
                t = t * dxv[i][r];
                acc[i][j][r] = acc[i][j][r] + t;
            }
        }
        // the block's additions are done here, before the step's barrier: left
        // to itself the compiler sinks them past the next steps' products and
        // holds several blocks' products in registers at once
#pragma unroll
        for (int i = 0; i < TI; i++)
#pragma unroll
            for (int j = 0; j < TJ; j++) asm volatile("" : "+v"(acc[i][j]));
    };
    // Four register sets, named: step b refills set b % 4 with block b + 4
    // (set b's data went to LDS at the end of step b - 1), computes block b,
    // and stores block b + 1 to the other LDS buffer.
    uint4 a0_0, a1_0, a0_1, a1_1, a0_2, a1_2, a0_3, a1_3;
    uint2 w_0, w_1, w_2, w_3;
    float dx_0, dx_1, dx_2, dx_3, cr_0, cr_1, cr_2, cr_3;
    uint32_t dw_0, dw_1, dw_2, dw_3;
    static_assert(GM_RS == 4, "the unrolled K loop below names four register sets");
#define TN_GM_SET(S) a0_##S, a1_##S, w_##S, dx_##S, cr_##S, dw_##S
    // (the last steps load and stage a block past the end, clamped by gload
    // to the last one, into the LDS buffer no later step reads)
#define TN_GM_STEP(S, NEXT, B)                          \
    {                                                   \
        gload((B) + GM_RS, TN_GM_SET(S));               \
        compute((B)&1);                                 \
        lstore(((B) + 1) & 1, TN_GM_SET(NEXT));         \
        __syncthreads();                                \
    }
    gload(0, TN_GM_SET(0));
    gload(1, TN_GM_SET(1));
    gload(2, TN_GM_SET(2));
    gload(3, TN_GM_SET(3));
    lstore(0, TN_GM_SET(0));
    __syncthreads();
    // whole rounds of four steps as straight-line code, then the rest
    int b = 0;
    for (; b + GM_RS <= nb; b += GM_RS) {
        TN_GM_STEP(0, 1, b)
        TN_GM_STEP(1, 2, b + 1)
        TN_GM_STEP(2, 3, b + 2)
        TN_GM_STEP(3, 0, b + 3)
    }
    if (b < nb) TN_GM_STEP(0, 1, b)
    if (b + 1 < nb) TN_GM_STEP(1, 2, b + 1)
    if (b + 2 < nb) TN_GM_STEP(2, 3, b + 2)
#undef TN_GM_STEP
#undef TN_GM_SET

#pragma unroll
    for (int i = 0; i < TI; i++) {
#pragma unroll
        for (int j = 0; j < TJ; j++) {
            const int n = n0 + wn * 16 * TJ + j * 16 + lrow;
            if (n >= N) continue;
            const float bv = bias ? bias[n] : 0.0f;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = m0 + wm * 16 * TI + i * 16 + lgrp * 4 + r;
                if (m >= M) continue;
                float v = acc[i][j][r];
                if (bias) v = v + bv;
                // resid + y, tn_add's operation, into y (f32); resid may be y
                if (resid) v = resid[(int64_t)m * N + n] + v;
                if (y_bf16)
                    reinterpret_cast<uint16_t*>(y)[(int64_t)m * N + n] = bf16_from_f32(v);
                else
                    reinterpret_cast<float*>(y)[(int64_t)m * N + n] = v;
            }
        }
    }
}


// ---- q8_0 prefill GEMM on integer MFMA -----------------------------------------
//
// With q8_0 weights both operands are int8 codes, so the block dot S_b is one
// v_mfma_i32_16x16x32_i8 per 16x16 output tile and K block: an exact i32
// result with no offset correction and no code conversion. The tile shape,
// the XCD-aware tile order, the LDS double buffer and the four register sets
// in flight are k_gemm's; the float steps are the same (S_b * d_w) * d_x and
// ordered addition.
//
// Prepass: the activation rows' Q8_0 codes as int8 in natural element order
// ([M_pad][nb][32]) and the f32 block scales transposed [nb][M_pad].
//
// LDS holds each 128 x 32-byte operand tile in MFMA fragment order: for row
// tile t (16 rows) and lane group g, the 16 rows' bytes 8g..8g+7 are 128
// consecutive bytes, so a fragment read is one conflict-free ds_read_b64 of
// 512 contiguous bytes per wave. Lane l of the MFMA holds row l % 16, block
// elements 8 (l / 16) .. 8 (l / 16) + 7 of both operands.

template <typename XT>
__global__ __launch_bounds__(256) void k_q8_rows_i8(const XT* __restrict__ x, int M, int M_pad, int K, int nb,
                                                   int8_t* __restrict__ xc, float* __restrict__ dxT) {
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
    xc[blk * QK + lane] = (int8_t)q;
    if (lane == 0) dxT[(int64_t)b * M_pad + row] = dx;
}

// k_q8_rows_i8 for a 16-byte aligned x: four lanes per (row, block), eight
// int8 codes each in natural order (one 8-byte store).
template <typename XT>
__global__ __launch_bounds__(256) void k_q8_rows_i8_v(const XT* __restrict__ x, int M, int M_pad, int K, int nb,
                                                      int8_t* __restrict__ xc, float* __restrict__ dxT) {
    const int64_t blk = (int64_t)blockIdx.x * (blockDim.x >> 2) + (threadIdx.x >> 2);
    const int part = threadIdx.x & 3;
    if (blk >= (int64_t)M_pad * nb) return;
    const int row = (int)(blk / nb), b = (int)(blk - (int64_t)row * nb);
    float v[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    if (row < M) load_x8<XT>(x + (int64_t)row * K + b * QK + 8 * part, v);
    int q[8], s;
    float dx;
    q8_0_quad(v, q, &dx, &s);
    if (row >= M) dx = 0.0f;
    uint32_t w[2] = {0u, 0u};
#pragma unroll
    for (int e = 0; e < 8; e++) w[e >> 2] |= ((uint32_t)q[e] & 0xffu) << (8 * (e & 3));
    *reinterpret_cast<uint2*>(xc + blk * QK + 8 * part) = make_uint2(w[0], w[1]);
    if (part == 0) dxT[(int64_t)b * M_pad + row] = dx;
}

typedef int i32x4 __attribute__((ext_vector_type(4)));

__device__ inline int frag_offset(int r, int g) {  // byte offset of row r, bytes 8g..8g+7, in a fragment-ordered tile
    return ((r >> 4) * 4 + g) * 128 + (r & 15) * 8;
}

__global__ __launch_bounds__(GM_THREADS) void k_gemm_q8(const int8_t* __restrict__ xc, const float* __restrict__ dxT,
                                                       int M, int M_pad, int nb, const uint8_t* __restrict__ qs,
                                                       const uint16_t* __restrict__ dw, int N,
                                                       const float* __restrict__ bias, void* __restrict__ y,
                                                       int y_bf16) {
    __shared__ __align__(16) uint8_t sA[2][GM_BM * QK];
    __shared__ __align__(16) uint8_t sB[2][GM_BN * QK];
    __shared__ __align__(16) float sdx[2][GM_BM];
    __shared__ __align__(16) float sdw[2][GM_BN];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;  // wave's 64x64 sub-tile
    const int lrow = lane & 15, lgrp = lane >> 4;

    const int mt = (int)gridDim.y;
    const int ntot = (int)(gridDim.x * gridDim.y);
    const int id = (int)(blockIdx.y * gridDim.x + blockIdx.x);
    int tile = id;
    if (ntot % NUM_XCD == 0) tile = (id % NUM_XCD) * (ntot / NUM_XCD) + id / NUM_XCD;
    const int m0 = (tile % mt) * GM_BM, n0 = (tile / mt) * GM_BN;

    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int j = 0; j < 4; j++) acc[i][j] = (f32x4){0.f, 0.f, 0.f, 0.f};

    // one register set: 16 bytes of activation codes (row tid / 2, half tid % 2),
    // 16 bytes of weight codes (column tid / 2), and (threads < GM_BM) the
    // row's Q8_0 scale or (threads >= GM_BM) the column's f16 weight scale
    const int prow = tid >> 1, phalf = tid & 1;
    const int so0 = frag_offset(prow, 2 * phalf), so1 = frag_offset(prow, 2 * phalf + 1);
    auto gload = [&](int b, uint4& a, uint4& w, float& dx, uint32_t& dws) {
        a = *reinterpret_cast<const uint4*>(xc + ((int64_t)(m0 + prow) * nb + b) * QK + phalf * 16);
        w = make_uint4(0u, 0u, 0u, 0u);
        if (n0 + prow < N) w = *reinterpret_cast<const uint4*>(qs + ((int64_t)(n0 + prow) * nb + b) * QK + phalf * 16);
        dx = 0.0f;
        dws = 0;
        if (tid < GM_BM) {
            dx = dxT[(int64_t)b * M_pad + m0 + tid];
        } else {
            const int n = n0 + tid - GM_BM;
            dws = (n < N) ? dw[(int64_t)n * nb + b] : 0u;
        }
    };
    auto lstore = [&](int buf, const uint4& a, const uint4& w, float dx, uint32_t dws) {
        *reinterpret_cast<uint2*>(&sA[buf][so0]) = make_uint2(a.x, a.y);
        *reinterpret_cast<uint2*>(&sA[buf][so1]) = make_uint2(a.z, a.w);
        *reinterpret_cast<uint2*>(&sB[buf][so0]) = make_uint2(w.x, w.y);
        *reinterpret_cast<uint2*>(&sB[buf][so1]) = make_uint2(w.z, w.w);
        if (tid < GM_BM)
            sdx[buf][tid] = dx;
        else
            sdw[buf][tid - GM_BM] = f16_bits_hw((uint16_t)dws);
    };
    auto compute = [&](int buf) {
        long afr[4], bfr[4];
#pragma unroll
        for (int i = 0; i < 4; i++) afr[i] = *reinterpret_cast<const long*>(&sA[buf][frag_offset(wm * 64 + i * 16 + lrow, lgrp)]);
#pragma unroll
        for (int j = 0; j < 4; j++) bfr[j] = *reinterpret_cast<const long*>(&sB[buf][frag_offset(wn * 64 + j * 16 + lrow, lgrp)]);
        float dwv[4];
        f32x4 dxv[4];
#pragma unroll
        for (int j = 0; j < 4; j++) dwv[j] = sdw[buf][wn * 64 + j * 16 + lrow];
#pragma unroll
        for (int i = 0; i < 4; i++) dxv[i] = *reinterpret_cast<const f32x4*>(&sdx[buf][wm * 64 + i * 16 + lgrp * 4]);
        const i32x4 zero = {0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < 4; i++) {
#pragma unroll
            for (int j = 0; j < 4; j++) {
                // C[row][col]: col = lane & 15 (weight column), row = 4*(lane>>4) + r
                const i32x4 sv = __builtin_amdgcn_mfma_i32_16x16x32_i8(afr[i], bfr[j], zero, 0, 0, 0);
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    float t = (float)sv[r] * dwv[j];
                    t = t * dxv[i][r];
                    acc[i][j][r] = acc[i][j][r] + t;
                }
            }
        }
    };
    uint4 a_0, a_1, a_2, a_3, w_0, w_1, w_2, w_3;
    float dx_0, dx_1, dx_2, dx_3;
    uint32_t dw_0, dw_1, dw_2, dw_3;
    static_assert(GM_RS == 4, "the unrolled K loop below names four register sets");
#define TN_GQ_SET(S) a_##S, w_##S, dx_##S, dw_##S
#define TN_GQ_STEP(S, NEXT, B)                                    \
    {                                                             \
        if ((B) + GM_RS < nb) gload((B) + GM_RS, TN_GQ_SET(S));   \
        compute((B)&1);                                           \
        if ((B) + 1 < nb) lstore(((B) + 1) & 1, TN_GQ_SET(NEXT)); \
        __syncthreads();                                          \
    }
    gload(0, TN_GQ_SET(0));
    if (1 < nb) gload(1, TN_GQ_SET(1));
    if (2 < nb) gload(2, TN_GQ_SET(2));
    if (3 < nb) gload(3, TN_GQ_SET(3));
    lstore(0, TN_GQ_SET(0));
    __syncthreads();
    for (int b = 0; b < nb; b += GM_RS) {
        TN_GQ_STEP(0, 1, b)
        if (b + 1 < nb) TN_GQ_STEP(1, 2, b + 1)
        if (b + 2 < nb) TN_GQ_STEP(2, 3, b + 2)
        if (b + 3 < nb) TN_GQ_STEP(3, 0, b + 3)
    }
#undef TN_GQ_STEP
#undef TN_GQ_SET

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

tn_status check_weight(const char* op, const char* fmt, int64_t n, int64_t k) {
    if (n < 0 || k <= 0 || k % QK != 0) {
        char buf[384];
        std::snprintf(buf, sizeof buf,
                      "%s: %s stores 32 elements per block, so it must have their last dim divisible by "
                      "block size -- got %lld, which is not a multiple of 32 (shape [%lld, %lld])",
                      op, fmt, (long long)k, (long long)n, (long long)k);
        return fail(TN_ENOTIMPL, buf);
    }
    if (n * (k / QK) > ((int64_t)1 << 40)) return fail(TN_EVALUE, std::string(op) + ": weight too large");
    return TN_OK;
}

template <int FMT, int MR, typename XT, int PRO = PRO_NONE, bool ARG = false, bool GLU = false>
tn_status launch_gemv(hipStream_t st, const XT* x, int K, const uint8_t* qs, const uint16_t* dw, int N,
                      const float* bias, void* y, int y_bf16, const float* resid = nullptr,
                      const GemvPro& po = GemvPro(), unsigned* grid_out = nullptr) {
    const int nb = K / QK;
    constexpr int ITEMS = Fmt<FMT>::GEMV_ITEMS;
    // rows per tile: as many as ITEMS items per thread allow, but no more
    // than it takes to give every CU a tile of a small matrix
    constexpr int RW = GLU ? 2 : 1;  // weight rows per output (GLU: gate and up)
    int rows = (GEMV_THREADS * ITEMS) / (RW * nb);
    const int spread = (int)cdiv(N, 256);
    if (rows > spread) rows = spread;
    if (rows < 1) rows = 1;
    if (rows > N) rows = N;
    // two term buffers (double-buffered across tiles)
    if (bias && resid) return fail(TN_EINVAL, "quantised GEMV: bias and residual together are not supported");
    const int nbp = (nb + 3) & ~3;
    auto lds_of = [&](int r) {
        return (((size_t)MR * K + (size_t)MR * nb * 8 + 15) & ~(size_t)15) + 2 * (size_t)RW * r * MR * nbp * 4;
    };
    size_t lds = lds_of(rows);
    while (rows > 1 && lds > 64 * 1024) {
        rows >>= 1;
        lds = lds_of(rows);
    }
    if (lds > 64 * 1024) return TN_ENOTIMPL;  // caller falls through to the GEMM path
    // (row, block) items must fit ITEMS per thread
    if ((int64_t)RW * rows * nb > GEMV_THREADS * ITEMS) return TN_ENOTIMPL;
    if (GLU && (bias || resid)) return fail(TN_EINVAL, "quantised GEMV: the SiLU epilogue takes no bias or residual");
    const int64_t ntiles = cdiv(N, rows);
    // persistent: exactly as many workgroups as the device holds at once (a
    // workgroup that had to wait for a slot would start its whole share of
    // tiles late). SHAPE: the activation rows held in registers (k_gemv's
    // HOLD passes of 32 blocks), and GEMV_ONE when the resident workgroups
    // cover the tiles and its buffer descriptors (a tile's weight span, GLU:
    // N + rows rows; the bias or residual rows) stay below 2^31 bytes
    const bool held = MR * nb <= 32 * (PRO == PRO_COMBINE ? 1 : GEMV_HOLD);
    const bool spans = (int64_t)(GLU ? N + rows : rows) * nb * Fmt<FMT>::CODE_BYTES < (int64_t(1) << 31) &&
                       (int64_t)MR * N * 4 < (int64_t(1) << 31);
    auto kern_of = [](int shape) -> const void* {
        return shape == GEMV_ONE      ? reinterpret_cast<const void*>(&k_gemv<FMT, MR, XT, PRO, ARG, GLU, GEMV_ONE>)
               : shape == GEMV_STREAM ? reinterpret_cast<const void*>(&k_gemv<FMT, MR, XT, PRO, ARG, GLU, GEMV_STREAM>)
                                      : reinterpret_cast<const void*>(&k_gemv<FMT, MR, XT, PRO, ARG, GLU, GEMV_PASSES>);
    };
    const int64_t cap = ARG ? GEMV_ARG_MAX_PARTS : INT32_MAX;
    int shape = held ? GEMV_ONE : GEMV_PASSES, resident = 0;
    tn_status s = resident_workgroups(kern_of(shape), GEMV_THREADS, lds, &resident);
    if (s != TN_OK) return s;
    if (shape == GEMV_ONE && (ntiles > resident || ntiles > cap || !spans)) {
        shape = GEMV_STREAM;
        s = resident_workgroups(kern_of(shape), GEMV_THREADS, lds, &resident);
        if (s != TN_OK) return s;
    }
    unsigned grid = (unsigned)(ntiles < resident ? ntiles : resident);
    if (grid > (unsigned)cap) grid = (unsigned)cap;
#define TN_GEMV(SH)                                                                                                   \
    hipLaunchKernelGGL((k_gemv<FMT, MR, XT, PRO, ARG, GLU, SH>), dim3(grid), dim3(GEMV_THREADS), lds, st, x, K, nb, qs, \
                       dw, N, rows, bias, resid, y, y_bf16, po)
    if (shape == GEMV_ONE) TN_GEMV(GEMV_ONE);
    else if (shape == GEMV_STREAM) TN_GEMV(GEMV_STREAM);
    else TN_GEMV(GEMV_PASSES);
#undef TN_GEMV
    TN_LAUNCHED();
    if (grid_out) *grid_out = grid;
    return TN_OK;
}

// The q4 GEMM over the prepass's codes: 112-column tiles when they fill the
// device in whole rounds of two workgroups per CU and 128-column ones would
// not; when 128-column tiles would give fewer than 128 workgroups, 32-column
// ones if they give a workgroup per CU, else 16-column ones (64 columns
// would give fewer than 256 workgroups whenever 128 give fewer than 128).
void gemm_q4_launch(hipStream_t st, const uint16_t* xc, const float* dxT, const float* corrT, int64_t m,
                    int64_t M_pad, int nb, const uint8_t* qs, const uint16_t* d, int64_t n, const float* bias, void* y,
                    int y_bf16, const float* resid) {
    const int64_t mt = M_pad / GM_BM;
    const bool t112 = n % 112 == 0 && (mt * (n / 112)) % 512 == 0 && (mt * cdiv(n, GM_BN)) % 512 != 0;
    int bn = GM_BN;
    if (mt * cdiv(n, GM_BN) < 128) bn = mt * cdiv(n, 32) >= 256 ? 32 : 16;
#define TN_GEMM(WR, WC, TJ, BNN)                                                                                   \
    hipLaunchKernelGGL((k_gemm<WR, WC, TJ>), dim3((unsigned)cdiv(n, BNN), (unsigned)mt), dim3(GM_THREADS), 0, st, \
                       xc, dxT, corrT, (int)m, (int)M_pad, nb, qs, d, (int)n, bias, y, y_bf16, resid)
    if (t112) TN_GEMM(4, 1, 7, 112);
    else if (bn == 16) TN_GEMM(4, 1, 1, 16);
    else if (bn == 32) TN_GEMM(4, 1, 2, 32);
    else TN_GEMM(2, 2, 4, GM_BN);
#undef TN_GEMM
}

template <int FMT, typename XT>
tn_status linear_impl(hipStream_t st, const XT* x, int64_t m, int64_t k, const uint8_t* qs, const uint16_t* d,
                      int64_t n, const float* bias, void* y, int y_bf16) {
    if (m == 0 || n == 0) return TN_OK;
    const int nb = (int)(k / QK);
    const size_t ysz = y_bf16 ? 2 : 4;
    // the GEMV reads x in 16-byte pieces; an unaligned x takes the GEMM path
    if (m <= GEMV_MAX_M && nb <= GEMV_THREADS * Fmt<FMT>::GEMV_ITEMS && reinterpret_cast<uintptr_t>(x) % 16 == 0) {
        // decode: GEMV in chunks of up to 4 rows of x (a row's result does not
        // depend on the chunking: every output is the same recurrence)
        int64_t r = 0;
        tn_status s = TN_OK;
        while (r < m && s == TN_OK) {
            const int64_t c = (m - r) >= 4 ? 4 : (m - r);
            const XT* xr = x + r * k;
            void* yr = static_cast<char*>(y) + r * n * ysz;
            switch (c) {
                case 4: s = launch_gemv<FMT, 4, XT>(st, xr, (int)k, qs, d, (int)n, bias, yr, y_bf16); break;
                case 3: s = launch_gemv<FMT, 3, XT>(st, xr, (int)k, qs, d, (int)n, bias, yr, y_bf16); break;
                case 2: s = launch_gemv<FMT, 2, XT>(st, xr, (int)k, qs, d, (int)n, bias, yr, y_bf16); break;
                default: s = launch_gemv<FMT, 1, XT>(st, xr, (int)k, qs, d, (int)n, bias, yr, y_bf16); break;
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
    const int64_t blocks = M_pad * nb;
    const unsigned pgrid = (unsigned)cdiv(blocks, 8);   // 32 lanes per block
    const unsigned vgrid = (unsigned)cdiv(blocks, 64);  // 4 lanes per block
    const bool aligned = reinterpret_cast<uintptr_t>(x) % 16 == 0;
    const dim3 grid((unsigned)cdiv(n, GM_BN), (unsigned)(M_pad / GM_BM));
    const size_t dx_bytes = (size_t)M_pad * nb * 4;
    void* ws = nullptr;
    if constexpr (FMT == FMT_Q8_0) {
        const size_t xc_bytes = (size_t)M_pad * k;
        tn_status s = workspace(st, xc_bytes + dx_bytes, &ws);
        if (s != TN_OK) return s;
        int8_t* xc = static_cast<int8_t*>(ws);
        float* dxT = reinterpret_cast<float*>(static_cast<char*>(ws) + xc_bytes);
        if (aligned)
            hipLaunchKernelGGL((k_q8_rows_i8_v<XT>), dim3(vgrid), dim3(256), 0, st, x, (int)m, (int)M_pad, (int)k, nb,
                               xc, dxT);
        else
            hipLaunchKernelGGL((k_q8_rows_i8<XT>), dim3(pgrid), dim3(256), 0, st, x, (int)m, (int)M_pad, (int)k, nb,
                               xc, dxT);
        TN_LAUNCHED();
        hipLaunchKernelGGL(k_gemm_q8, grid, dim3(GM_THREADS), 0, st, xc, dxT, (int)m, (int)M_pad, nb, qs, d, (int)n,
                           bias, y, y_bf16);
        TN_LAUNCHED();
    } else {
        const size_t xc_bytes = (size_t)M_pad * k * 2;
        tn_status s = workspace(st, xc_bytes + 2 * dx_bytes, &ws);
        if (s != TN_OK) return s;
        uint16_t* xc = static_cast<uint16_t*>(ws);
        float* dxT = reinterpret_cast<float*>(static_cast<char*>(ws) + xc_bytes);
        float* corrT = reinterpret_cast<float*>(static_cast<char*>(ws) + xc_bytes + dx_bytes);
        if (aligned)
            hipLaunchKernelGGL((k_q8_rows_v<XT>), dim3(vgrid), dim3(256), 0, st, x, (int)m, (int)M_pad, (int)k, nb, xc,
                               dxT, corrT);
        else
            hipLaunchKernelGGL((k_q8_rows<XT>), dim3(pgrid), dim3(256), 0, st, x, (int)m, (int)M_pad, (int)k, nb, xc,
                               dxT, corrT);
        TN_LAUNCHED();
        gemm_q4_launch(st, xc, dxT, corrT, m, M_pad, nb, qs, d, n, bias, y, y_bf16, nullptr);
        TN_LAUNCHED();
    }
    return TN_OK;
}

// The codec entry points of one format.
template <int FMT>
tn_status codec_launch(const char* op, void* stream, int64_t n, int64_t k, int kind, const void* in0,
                       const void* in1, void* out0, void* out1) {
    tn_status s = check_weight(op, Fmt<FMT>::name, n, k);
    if (s != TN_OK) return s;
    const int64_t nblocks = n * (k / QK);
    if (!nblocks) return TN_OK;
    if (!in0 || !out0 || (kind >= 2 ? !in1 : !out1)) return fail(TN_EVALUE, std::string(op) + ": null pointer");
    const dim3 grid((unsigned)cdiv(nblocks, 256));
    hipStream_t st = (hipStream_t)stream;
    switch (kind) {
        case 0:  // blob -> planes
            hipLaunchKernelGGL(k_from_blob<FMT>, grid, dim3(256), 0, st, static_cast<const uint8_t*>(in0), nblocks,
                               static_cast<uint8_t*>(out0), static_cast<uint16_t*>(out1));
            break;
        case 1:  // f32 -> planes
            hipLaunchKernelGGL(k_quantize_w<FMT>, grid, dim3(256), 0, st, static_cast<const float*>(in0), nblocks,
                               static_cast<uint8_t*>(out0), static_cast<uint16_t*>(out1));
            break;
        case 2:  // planes -> blob
            hipLaunchKernelGGL(k_to_blob<FMT>, grid, dim3(256), 0, st, static_cast<const uint8_t*>(in0),
                               static_cast<const uint16_t*>(in1), nblocks, static_cast<uint8_t*>(out0));
            break;
        default:  // planes -> f32
            hipLaunchKernelGGL(k_dequantize<FMT>, grid, dim3(256), 0, st, static_cast<const uint8_t*>(in0),
                               static_cast<const uint16_t*>(in1), nblocks, static_cast<float*>(out0));
            break;
    }
    TN_LAUNCHED();
    return TN_OK;
}

template <int FMT>
tn_status linear_entry(void* stream, const void* x, int x_dtype, int64_t m, int64_t k, const uint8_t* qs,
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
        return linear_impl<FMT, float>(st, static_cast<const float*>(x), m, k, qs, d, n, bias, y, yb);
    return linear_impl<FMT, uint16_t>(st, static_cast<const uint16_t*>(x), m, k, qs, d, n, bias, y, yb);
}

}  // namespace

// One activation row through a q4_0 linear for the decode step, with the
// step's neighbouring elementwise ops fused in (see k_gemv): bit-identical to
// running tn_rmsnorm / tn_silu_mul, then tn_q4_0_linear, then tn_add.
tn_status linear_decode(hipStream_t st, const float* x, int64_t k, int pro, const GemvPro& po, const uint8_t* qs,
                        const uint16_t* d, int64_t n, const float* resid, float* y) {
    tn_status s = check_weight("linear_decode", "q4_0", n, k);
    if (s != TN_OK) return s;
    if (k > LINEAR_DECODE_MAX_K || n > INT32_MAX) return fail(TN_ENOTIMPL, "linear_decode: shape too large");
    if (n == 0) return TN_OK;
    switch (pro) {
        case PRO_RMSNORM:
            if (po.glu)
                s = launch_gemv<FMT_Q4_0, 1, float, PRO_RMSNORM, false, true>(st, x, (int)k, qs, d, (int)n, nullptr, y, 0,
                                                                             resid, po);
            else
                s = launch_gemv<FMT_Q4_0, 1, float, PRO_RMSNORM>(st, x, (int)k, qs, d, (int)n, nullptr, y, 0, resid, po);
            break;
        case PRO_SILU: s = launch_gemv<FMT_Q4_0, 1, float, PRO_SILU>(st, x, (int)k, qs, d, (int)n, nullptr, y, 0, resid, po); break;
        case PRO_COMBINE:
            // head_dim a power of two (the merge addresses by shifts), at least a 4-column piece
            if (po.head_dim < 4 || po.head_dim != (1 << po.head_shift) || k % po.head_dim != 0 || po.nsplit < 1 ||
                po.nsplit > STEP_MAX_SPLITS || !po.part_o || !po.part_ml || !po.len)
                return fail(TN_EINVAL, "linear_decode: bad attention partials");
            s = launch_gemv<FMT_Q4_0, 1, float, PRO_COMBINE>(st, po.part_o, (int)k, qs, d, (int)n, nullptr, y, 0, resid, po);
            break;
        default: s = launch_gemv<FMT_Q4_0, 1, float, PRO_NONE>(st, x, (int)k, qs, d, (int)n, nullptr, y, 0, resid, po); break;
    }
    if (s == TN_ENOTIMPL) return fail(TN_ENOTIMPL, "linear_decode: the activation row does not fit the GEMV");
    return s;
}

tn_status linear_decode_argmax(hipStream_t st, const float* x, int64_t k, const GemvPro& po, const uint8_t* qs,
                               const uint16_t* d, int64_t n, float* y) {
    tn_status s = check_weight("linear_decode_argmax", "q4_0", n, k);
    if (s != TN_OK) return s;
    if (k > LINEAR_DECODE_MAX_K || n > INT32_MAX || n < 1) return TN_ENOTIMPL;
    if (!po.arg_v || !po.arg_i || !po.state || !po.tokens || (po.prompt_len > 0 && !po.prompt))
        return fail(TN_EINVAL, "linear_decode_argmax: missing argmax operands");
    unsigned parts = 0;
    s = launch_gemv<FMT_Q4_0, 1, float, PRO_RMSNORM, true>(st, x, (int)k, qs, d, (int)n, nullptr, y, 0, nullptr, po,
                                                           &parts);
    if (s != TN_OK) return s;
    hipLaunchKernelGGL(k_argmax_parts, dim3(1), dim3(GEMV_THREADS), 0, st, po.arg_v, po.arg_i, (int)parts, (int)n,
                       po.state, po.tokens, po.prompt, po.prompt_len, po.cap);
    TN_LAUNCHED();
    return TN_OK;
}

// A prompt's projection through the q4 GEMM, its input in one of the
// prepass's layouts and the residual added in its epilogue.
tn_status linear_prefill(hipStream_t st, const float* x, int64_t m, int64_t k, int xm, int hd, const uint8_t* qs,
                         const uint16_t* d, int64_t n, const float* resid, float* y) {
    tn_status s = check_weight("linear_prefill", "q4_0", n, k);
    if (s != TN_OK) return s;
    if (m == 0 || n == 0) return TN_OK;
    if (reinterpret_cast<uintptr_t>(x) % 16 != 0) return fail(TN_EINVAL, "linear_prefill: x must be 16-byte aligned");
    if (xm == XM_HEADS && (hd <= 0 || hd % QK != 0 || k % hd != 0))
        return fail(TN_EINVAL, "linear_prefill: the head dim must divide the row and be a multiple of 32");
    const int nb = (int)(k / QK);
    const int64_t M_pad = cdiv(m, GM_BM) * GM_BM;
    if (M_pad > INT32_MAX || n > INT32_MAX || M_pad * k * (xm == XM_GLU ? 2 : 1) > INT32_MAX)
        return fail(TN_EVALUE, "linear_prefill: shape too large");
    const int64_t blocks = M_pad * nb;
    const size_t dx_bytes = (size_t)M_pad * nb * 4, xc_bytes = (size_t)M_pad * k * 2;
    void* ws = nullptr;
    s = workspace(st, xc_bytes + 2 * dx_bytes, &ws);
    if (s != TN_OK) return s;
    uint16_t* xc = static_cast<uint16_t*>(ws);
    float* dxT = reinterpret_cast<float*>(static_cast<char*>(ws) + xc_bytes);
    float* corrT = reinterpret_cast<float*>(static_cast<char*>(ws) + xc_bytes + dx_bytes);
    const dim3 vgrid((unsigned)cdiv(blocks, 64));  // 4 lanes per block
    if (xm == XM_GLU)
        hipLaunchKernelGGL((k_q8_rows_v<float, XM_GLU>), vgrid, dim3(256), 0, st, x, (int)m, (int)M_pad, (int)k, nb, xc,
                           dxT, corrT, 0);
    else if (xm == XM_HEADS)
        hipLaunchKernelGGL((k_q8_rows_v<float, XM_HEADS>), vgrid, dim3(256), 0, st, x, (int)m, (int)M_pad, (int)k, nb,
                           xc, dxT, corrT, hd);
    else
        hipLaunchKernelGGL((k_q8_rows_v<float, XM_ROWS>), vgrid, dim3(256), 0, st, x, (int)m, (int)M_pad, (int)k, nb,
                           xc, dxT, corrT, 0);
    TN_LAUNCHED();
    gemm_q4_launch(st, xc, dxT, corrT, m, M_pad, nb, qs, d, n, nullptr, y, 0, resid);
    TN_LAUNCHED();
    return TN_OK;
}

}  // namespace tn

using namespace tn;

extern "C" {

tn_status tn_q4_0_from_blob(void* stream, const uint8_t* blob, int64_t n, int64_t k, uint8_t* qs, uint16_t* d) {
    return codec_launch<FMT_Q4_0>("torch._C._quantized_to", stream, n, k, 0, blob, nullptr, qs, d);
}

tn_status tn_q4_0_to_blob(void* stream, const uint8_t* qs, const uint16_t* d, int64_t n, int64_t k, uint8_t* blob) {
    return codec_launch<FMT_Q4_0>("torch._C._quantized_blob", stream, n, k, 2, qs, d, blob, nullptr);
}

tn_status tn_q4_0_quantize(void* stream, const float* w, int64_t n, int64_t k, uint8_t* qs, uint16_t* d) {
    return codec_launch<FMT_Q4_0>("torch._C._quantize", stream, n, k, 1, w, nullptr, qs, d);
}

tn_status tn_q4_0_dequantize(void* stream, const uint8_t* qs, const uint16_t* d, int64_t n, int64_t k, float* out) {
    return codec_launch<FMT_Q4_0>("torch._C._dequantize", stream, n, k, 3, qs, d, out, nullptr);
}

tn_status tn_q8_0_from_blob(void* stream, const uint8_t* blob, int64_t n, int64_t k, int8_t* qs, uint16_t* d) {
    return codec_launch<FMT_Q8_0>("torch._C._quantized_to", stream, n, k, 0, blob, nullptr, qs, d);
}

tn_status tn_q8_0_to_blob(void* stream, const int8_t* qs, const uint16_t* d, int64_t n, int64_t k, uint8_t* blob) {
    return codec_launch<FMT_Q8_0>("torch._C._quantized_blob", stream, n, k, 2, qs, d, blob, nullptr);
}

tn_status tn_q8_0_quantize(void* stream, const float* w, int64_t n, int64_t k, int8_t* qs, uint16_t* d) {
    return codec_launch<FMT_Q8_0>("torch._C._quantize", stream, n, k, 1, w, nullptr, qs, d);
}

tn_status tn_q8_0_dequantize(void* stream, const int8_t* qs, const uint16_t* d, int64_t n, int64_t k, float* out) {
    return codec_launch<FMT_Q8_0>("torch._C._dequantize", stream, n, k, 3, qs, d, out, nullptr);
}

tn_status tn_q4_0_linear_decode(void* stream, const float* x, int64_t k, int prologue, const float* prologue_w,
                                double eps, const uint8_t* qs, const uint16_t* d, int64_t n, const float* resid,
                                float* y) {
    const char* op = "q4_0_linear_decode";
    if (prologue != TN_PRO_NONE && prologue != TN_PRO_RMSNORM && prologue != TN_PRO_SILU &&
        prologue != TN_PRO_RMSNORM_SILU)
        return fail(TN_EINVAL, std::string(op) + ": unknown prologue");
    if (k <= 0 || n < 0) return fail(TN_EINVAL, std::string(op) + ": bad sizes");
    const bool glu = prologue == TN_PRO_RMSNORM_SILU;
    if (glu && resid) return fail(TN_EINVAL, std::string(op) + ": the SiLU epilogue takes no residual");
    if (n == 0) return TN_OK;
    if (!x || !qs || !d || !y || ((prologue == TN_PRO_RMSNORM || glu) && !prologue_w))
        return fail(TN_EVALUE, std::string(op) + ": null pointer");
    // y is written while other workgroups still read x
    const char* xb = reinterpret_cast<const char*>(x);
    const char* yb = reinterpret_cast<const char*>(y);
    const int64_t xlen = (prologue == TN_PRO_SILU ? 2 * k : k) * 4;
    if (yb < xb + xlen && xb < yb + n * 4) return fail(TN_EINVAL, std::string(op) + ": y overlaps x");
    if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(prologue_w)) % 16 != 0)
        return fail(TN_EINVAL, std::string(op) + ": x and prologue_w must be 16-byte aligned");
    static_assert(TN_PRO_NONE == PRO_NONE && TN_PRO_RMSNORM == PRO_RMSNORM && TN_PRO_SILU == PRO_SILU, "prologues");
    GemvPro po;
    po.w = prologue_w;
    po.eps = (float)eps;
    po.glu = glu ? 1 : 0;
    return linear_decode((hipStream_t)stream, x, k, glu ? PRO_RMSNORM : prologue, po, qs, d, n, resid, y);
}

tn_status tn_q4_0_linear(void* stream, const void* x, int x_dtype, int64_t m, int64_t k, const uint8_t* qs,
                         const uint16_t* d, int64_t n, const float* bias, void* y, int y_dtype) {
    return linear_entry<FMT_Q4_0>(stream, x, x_dtype, m, k, qs, d, n, bias, y, y_dtype);
}

tn_status tn_q8_0_linear(void* stream, const void* x, int x_dtype, int64_t m, int64_t k, const int8_t* qs,
                         const uint16_t* d, int64_t n, const float* bias, void* y, int y_dtype) {
    return linear_entry<FMT_Q8_0>(stream, x, x_dtype, m, k, reinterpret_cast<const uint8_t*>(qs), d, n, bias, y,
                                  y_dtype);
}

}  // extern "C"
