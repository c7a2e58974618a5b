// Scaled dot-product attention on gfx950: flash prefill (bf16 and f32) and
// split-KV decode over per-sequence KV caches.
//
// Semantics are the reference's aten._scaled_dot_product_flash_attention_for_cpu
// (torchnative/rust/torch_c/src/aten.rs:10092-10440): softmax(q k^T * scale
// [+ upper-left causal -inf]) v with f32 accumulation, GQA by indexing key/value
// head h / (Hq/Hkv), logsumexp over the masked, scaled scores. The blocked
// online softmax follows the structure of upstream's CPU flash kernel that the
// reference reproduces in flash.rs:587-780 (accumulators rescaled by
// exp(m_old - m_new), P narrowed to the input dtype between the products for
// bf16).
//
// Layout shared by all kernels: scores are computed transposed, S^T = K . Q^T,
// so that in the 16x16 MFMA result layout (lane l holds C[4*(l>>4) + r][l & 15])
// each lane owns one query (column l & 15) and four keys per 16-key tile. Row
// statistics are then in-lane plus two cross-lane steps, and the output is
// accumulated transposed, O^T = V^T . P^T, where the lane's own probabilities
// are directly the B operand and the lane again owns its query's column, so
// the online rescale needs no data movement.
//
// Rescaling is lazy: a row keeps the maximum it last rescaled to until a tile
// raises it by more than 2^8 (in exp2 units), so probabilities stay <= 256 and
// the accumulators are touched only when a wave actually needs it. The result
// is the same softmax; only the common factor differs until the end.
#include <algorithm>
#include <type_traits>

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

__device__ inline float wave_xor_max(float v) {
    v = fmaxf(v, __shfl_xor(v, 16));
    v = fmaxf(v, __shfl_xor(v, 32));
    return v;
}

__device__ inline float wave_xor_sum(float v) {
    v = v + __shfl_xor(v, 16);
    v = v + __shfl_xor(v, 32);
    return v;
}

// two f32 -> packed bf16 pair, RNE (v_cvt_pk_bf16_f32); used for the
// probabilities, which are finite and non-negative
__device__ inline uint32_t pack2_bf16_hw(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, bf16x2));
}

// the same narrowing spelled out (reduced.rs:161-218: RNE, NaN quieted), for outputs
__device__ inline uint32_t pack2_bf16(float a, float b) {
    return (uint32_t)bf16_from_f32(a) | ((uint32_t)bf16_from_f32(b) << 16);
}

// ---------------------------------------------------------------------------
// bf16 prefill. Workgroup = 4 waves = 64 queries of one (batch, head); each
// wave owns 16 queries. K/V tiles of 64 keys are staged in LDS (K as is, V
// transposed), double-buffered: the next tile's global loads are issued into
// registers before the current tile is computed and stored to the other LDS
// buffer after it. Per tile and wave:
//   S^T  : 4 key-tiles x D/32 MFMA 16x16x32 (A = K rows, B = Q^T in registers)
//   P    : exp2(S * scale*log2e - m), narrowed to bf16
//   O^T += D/16 d-tiles x 2 MFMA 16x16x32 (A = V^T rows, B = P^T)
// MFMA K-slot order for a 32-key chunk u: lane group g holds keys
// {32u + 4g + r, 32u + 16 + 4g + r : r = 0..3}, which is where S^T put them.
//
// Long causal rows are split over `nsplit` workgroups (blockIdx.x encodes the
// (query block, split) pair); a split writes unnormalised (m, l, O) partials
// that k_prefill_combine merges. Rows that fit one split write the output
// directly.
// ---------------------------------------------------------------------------

constexpr int PF_BQ = 64, PF_BK = 64;

template <int D>
__global__ __launch_bounds__(256) void k_fa_bf16(const uint16_t* __restrict__ Qg, const uint16_t* __restrict__ Kg,
                                               const uint16_t* __restrict__ Vg, int Hq, int Hkv, int L, int S,
                                               float sl2, int causal, int tiles_per, int nsplit,
                                               uint16_t* __restrict__ Og, float* __restrict__ lse,
                                               float* __restrict__ part_o, float2* __restrict__ part_ml) {
    constexpr int BQ = PF_BQ, BK = PF_BK;
    constexpr int KS = D + 8;   // K tile row stride (bf16)
    constexpr int VS = BK + 8;  // V^T tile row stride (bf16)
    constexpr int KCH = (BK * D / 8) / 256;   // 16-byte K chunks per thread
    constexpr int VBL = (BK * D / 16) / 256;  // 4-key x 4-d V blocks per thread
    __shared__ __align__(16) uint16_t sK[2][BK * KS];
    __shared__ __align__(16) uint16_t sVt[2][D * VS];

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int lq = lane & 15, g = lane >> 4;
    // work decode: heaviest query blocks first, then their splits
    const int nqb = (L + BQ - 1) / BQ;
    const int item = (int)blockIdx.x;
    const int qt = nqb - 1 - item / nsplit;
    const int split = item % nsplit;
    const int h = blockIdx.y, b = blockIdx.z;
    const int kvh = h / (Hq / Hkv);
    const int q0 = qt * BQ;
    const int qi = q0 + w * 16 + lq;
    const int kend = causal ? min(S, q0 + BQ) : S;
    const int ntiles_row = (kend + BK - 1) / BK;
    const int nsplit_row = (ntiles_row + tiles_per - 1) / tiles_per;
    if (split >= nsplit_row) return;  // uniform over the workgroup
    const int t_begin = split * tiles_per;
    const int t_end = min(ntiles_row, t_begin + tiles_per);

    const uint16_t* qp = Qg + ((int64_t)b * Hq + h) * L * D;
    const uint16_t* kp = Kg + ((int64_t)b * Hkv + kvh) * S * D;
    const uint16_t* vp = Vg + ((int64_t)b * Hkv + kvh) * S * D;

    bf16x8 qf[D / 32];
#pragma unroll
    for (int c = 0; c < D / 32; c++) {
        uint4 v = make_uint4(0, 0, 0, 0);
        if (qi < L) v = *reinterpret_cast<const uint4*>(qp + (int64_t)qi * D + 32 * c + 8 * g);
        qf[c] = __builtin_bit_cast(bf16x8, v);
    }
    // o[0 .. D/16-1]: O^T tiles; o[D/16]: the row sums, accumulated by one more
    // MFMA against a tile of ones so that the normaliser sums exactly the
    // bf16 probabilities the numerator used (every element of it holds l)
    f32x4 o[D / 16 + 1];
#pragma unroll
    for (int i = 0; i <= D / 16; i++) o[i] = (f32x4){0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY;
    const bf16x8 ones = __builtin_bit_cast(bf16x8, make_uint4(0x3f803f80u, 0x3f803f80u, 0x3f803f80u, 0x3f803f80u));

    uint4 kr[KCH];
    uint2 vr[VBL][4];
    // the (key, column) each thread moves is fixed; only the tile base moves
    auto gload = [&](int k0) {
        const uint16_t* kb = kp + (int64_t)k0 * D;
        const uint16_t* vb = vp + (int64_t)k0 * D;
        if (k0 + BK <= S) {
#pragma unroll
            for (int it = 0; it < KCH; it++) {
                const int c = tid + it * 256;
                kr[it] = *reinterpret_cast<const uint4*>(kb + (c / (D / 8)) * D + (c % (D / 8)) * 8);
            }
#pragma unroll
            for (int it = 0; it < VBL; it++) {
                const int idx = tid + it * 256;
                const uint16_t* src = vb + (4 * (idx / (D / 4))) * D + 4 * (idx % (D / 4));
#pragma unroll
                for (int i = 0; i < 4; i++) vr[it][i] = *reinterpret_cast<const uint2*>(src + i * D);
            }
        } else {
#pragma unroll
            for (int it = 0; it < KCH; it++) {
                const int c = tid + it * 256;
                const int r = c / (D / 8), part = c % (D / 8);
                kr[it] = make_uint4(0, 0, 0, 0);
                if (k0 + r < S) kr[it] = *reinterpret_cast<const uint4*>(kb + r * D + part * 8);
            }
#pragma unroll
            for (int it = 0; it < VBL; it++) {
                const int idx = tid + it * 256;
                const int dg = idx % (D / 4), kg = idx / (D / 4);
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    vr[it][i] = make_uint2(0, 0);
                    if (k0 + 4 * kg + i < S) vr[it][i] = *reinterpret_cast<const uint2*>(vb + (4 * kg + i) * D + 4 * dg);
                }
            }
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int it = 0; it < KCH; it++) {
            const int c = tid + it * 256;
            const int r = c / (D / 8), part = c % (D / 8);
            *reinterpret_cast<uint4*>(&sK[buf][r * KS + part * 8]) = kr[it];
        }
#pragma unroll
        for (int it = 0; it < VBL; it++) {
            const int idx = tid + it * 256;
            const int dg = idx % (D / 4), kg = idx / (D / 4);
            // 4 keys x 4 d -> 4 d-rows x 4 keys (v_perm picks 16-bit halves)
            const uint2* rw = vr[it];
            const uint32_t c0 = __builtin_amdgcn_perm(rw[1].x, rw[0].x, 0x05040100u);
            const uint32_t c1 = __builtin_amdgcn_perm(rw[3].x, rw[2].x, 0x05040100u);
            const uint32_t c2 = __builtin_amdgcn_perm(rw[1].x, rw[0].x, 0x07060302u);
            const uint32_t c3 = __builtin_amdgcn_perm(rw[3].x, rw[2].x, 0x07060302u);
            const uint32_t c4 = __builtin_amdgcn_perm(rw[1].y, rw[0].y, 0x05040100u);
            const uint32_t c5 = __builtin_amdgcn_perm(rw[3].y, rw[2].y, 0x05040100u);
            const uint32_t c6 = __builtin_amdgcn_perm(rw[1].y, rw[0].y, 0x07060302u);
            const uint32_t c7 = __builtin_amdgcn_perm(rw[3].y, rw[2].y, 0x07060302u);
            uint16_t* base = &sVt[buf][(4 * dg) * VS + 4 * kg];
            *reinterpret_cast<uint2*>(base) = make_uint2(c0, c1);
            *reinterpret_cast<uint2*>(base + VS) = make_uint2(c2, c3);
            *reinterpret_cast<uint2*>(base + 2 * VS) = make_uint2(c4, c5);
            *reinterpret_cast<uint2*>(base + 3 * VS) = make_uint2(c6, c7);
        }
    };

    gload(t_begin * BK);
    lstore(0);
    __syncthreads();
    for (int t = t_begin; t < t_end; t++) {
        const int buf = (t - t_begin) & 1;
        const int k0 = t * BK;
        if (t + 1 < t_end) gload(k0 + BK);

        // S^T for 64 keys x this wave's 16 queries
        f32x4 s[4];
#pragma unroll
        for (int kt = 0; kt < 4; kt++) {
            s[kt] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < D / 32; c++) {
                const bf16x8 ka = *reinterpret_cast<const bf16x8*>(&sK[buf][(16 * kt + lq) * KS + 32 * c + 8 * g]);
                s[kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka, qf[c], s[kt], 0, 0, 0);
            }
        }
        if (k0 + BK > S || (causal && k0 + BK - 1 > q0 + w * 16)) {
#pragma unroll
            for (int kt = 0; kt < 4; kt++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int key = k0 + 16 * kt + 4 * g + r;
                    if (key >= S || (causal && key > qi)) s[kt][r] = -INFINITY;
                }
        }
        float mx = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < 4; kt++)
            mx = fmaxf(mx, fmaxf(fmaxf(s[kt][0], s[kt][1]), fmaxf(s[kt][2], s[kt][3])));
        mx = wave_xor_max(mx) * sl2;
        const bool need = mx > m + RESCALE_SLACK;
        if (__any(need)) {
            const float mn = need ? mx : m;
            const float alpha = __builtin_amdgcn_exp2f(m - mn);
#pragma unroll
            for (int i = 0; i <= D / 16; i++) o[i] = o[i] * alpha;
            m = mn;
        }
        const float mu = (m == -INFINITY) ? 0.0f : m;
        bf16x8 pf[2];
#pragma unroll
        for (int u = 0; u < 2; u++) {
            float p[8];
#pragma unroll
            for (int r = 0; r < 4; r++) {
                p[r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[2 * u][r], sl2, -mu));
                p[4 + r] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[2 * u + 1][r], sl2, -mu));
            }
            uint4 pk;
            pk.x = pack2_bf16_hw(p[0], p[1]);
            pk.y = pack2_bf16_hw(p[2], p[3]);
            pk.z = pack2_bf16_hw(p[4], p[5]);
            pk.w = pack2_bf16_hw(p[6], p[7]);
            pf[u] = __builtin_bit_cast(bf16x8, pk);
        }
#pragma unroll
        for (int dt = 0; dt < D / 16; dt++) {
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const uint16_t* row = &sVt[buf][(16 * dt + lq) * VS + 32 * u + 4 * g];
                const uint2 lo = *reinterpret_cast<const uint2*>(row);
                const uint2 hi = *reinterpret_cast<const uint2*>(row + 16);
                const bf16x8 va = __builtin_bit_cast(bf16x8, make_uint4(lo.x, lo.y, hi.x, hi.y));
                o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pf[u], o[dt], 0, 0, 0);
            }
        }
#pragma unroll
        for (int u = 0; u < 2; u++) o[D / 16] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ones, pf[u], o[D / 16], 0, 0, 0);
        if (t + 1 < t_end) lstore(buf ^ 1);
        __syncthreads();
    }

    const float l = o[D / 16][0];
    if (qi >= L) return;
    const int64_t row = ((int64_t)b * Hq + h) * L + qi;
    if (nsplit_row == 1) {
        const float inv = 1.0f / l;
        uint16_t* op = Og + row * D;
#pragma unroll
        for (int dt = 0; dt < D / 16; dt++) {
            // O^T[d = 16dt + 4g + r][q = lq]
            *reinterpret_cast<uint2*>(op + 16 * dt + 4 * g) =
                make_uint2(pack2_bf16(o[dt][0] * inv, o[dt][1] * inv), pack2_bf16(o[dt][2] * inv, o[dt][3] * inv));
        }
        if (lse && g == 0) lse[row] = m * LN2 + logf(l);
    } else {
        float* po = part_o + (row * nsplit + split) * D;
#pragma unroll
        for (int dt = 0; dt < D / 16; dt++)
            *reinterpret_cast<float4*>(po + 16 * dt + 4 * g) = make_float4(o[dt][0], o[dt][1], o[dt][2], o[dt][3]);
        if (g == 0) part_ml[row * nsplit + split] = make_float2(m, l);
    }
}

// ---------------------------------------------------------------------------
// f32 prefill: the same decomposition on v_mfma_f32_16x16x4_f32 (K = 4 per op).
//   S^T : lane (key lq, group g) feeds K[key][4c + g]; Q^T from registers.
//   O^T : for key slot r of tile kt, lane group g feeds V[16kt + 4g + r][d]
//         and its own P at (kt, r), so V stays in natural layout in LDS.
// Row strides are padded to 4 mod 64 dwords, so the 64 lanes of each LDS read
// hit 64 distinct banks.
// ---------------------------------------------------------------------------

template <int D, int BK>
__global__ __launch_bounds__(256) void k_fa_f32(const float* __restrict__ Qg, const float* __restrict__ Kg,
                                              const float* __restrict__ Vg, int Hq, int Hkv, int L, int S,
                                              float sl2, int causal, int tiles_per, int nsplit,
                                              float* __restrict__ Og, float* __restrict__ lse,
                                              float* __restrict__ part_o, float2* __restrict__ part_ml) {
    constexpr int BQ = PF_BQ;
    constexpr int RS = D + 4;
    constexpr int CH = (BK * D / 4) / 256;  // float4 chunks of K (and of V) per thread
    __shared__ __align__(16) float sK[2][BK * RS];
    __shared__ __align__(16) float sV[2][BK * RS];

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int lq = lane & 15, g = lane >> 4;
    const int nqb = (L + BQ - 1) / BQ;
    const int item = (int)blockIdx.x;
    const int qt = nqb - 1 - item / nsplit;
    const int split = item % nsplit;
    const int h = blockIdx.y, b = blockIdx.z;
    const int kvh = h / (Hq / Hkv);
    const int q0 = qt * BQ;
    const int qi = q0 + w * 16 + lq;
    const int kend = causal ? min(S, q0 + BQ) : S;
    const int ntiles_row = (kend + BK - 1) / BK;
    const int nsplit_row = (ntiles_row + tiles_per - 1) / tiles_per;
    if (split >= nsplit_row) return;
    const int t_begin = split * tiles_per;
    const int t_end = min(ntiles_row, t_begin + tiles_per);

    const float* qp = Qg + ((int64_t)b * Hq + h) * L * D;
    const float* kp = Kg + ((int64_t)b * Hkv + kvh) * S * D;
    const float* vp = Vg + ((int64_t)b * Hkv + kvh) * S * D;

    float qf[D / 4];
#pragma unroll
    for (int c = 0; c < D / 4; c++) qf[c] = (qi < L) ? qp[(int64_t)qi * D + 4 * c + g] : 0.0f;
    f32x4 o[D / 16];
#pragma unroll
    for (int i = 0; i < D / 16; i++) o[i] = (f32x4){0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY, l = 0.0f;

    float4 kr[CH], vr[CH];
    auto gload = [&](int k0) {
#pragma unroll
        for (int it = 0; it < CH; it++) {
            const int c = tid + it * 256;
            const int r = c / (D / 4), part = c % (D / 4);
            kr[it] = vr[it] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (k0 + r < S) {
                kr[it] = *reinterpret_cast<const float4*>(kp + (int64_t)(k0 + r) * D + part * 4);
                vr[it] = *reinterpret_cast<const float4*>(vp + (int64_t)(k0 + r) * D + part * 4);
            }
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int it = 0; it < CH; it++) {
            const int c = tid + it * 256;
            const int r = c / (D / 4), part = c % (D / 4);
            *reinterpret_cast<float4*>(&sK[buf][r * RS + part * 4]) = kr[it];
            *reinterpret_cast<float4*>(&sV[buf][r * RS + part * 4]) = vr[it];
        }
    };

    gload(t_begin * BK);
    lstore(0);
    __syncthreads();
    for (int t = t_begin; t < t_end; t++) {
        const int buf = (t - t_begin) & 1;
        const int k0 = t * BK;
        if (t + 1 < t_end) gload(k0 + BK);

        f32x4 s[BK / 16];
#pragma unroll
        for (int kt = 0; kt < BK / 16; kt++) {
            s[kt] = (f32x4){0.f, 0.f, 0.f, 0.f};
            const float* krow = &sK[buf][(16 * kt + lq) * RS + g];
#pragma unroll
            for (int c = 0; c < D / 4; c++) s[kt] = __builtin_amdgcn_mfma_f32_16x16x4f32(krow[4 * c], qf[c], s[kt], 0, 0, 0);
        }
        if (k0 + BK > S || (causal && k0 + BK - 1 > q0 + w * 16)) {
#pragma unroll
            for (int kt = 0; kt < BK / 16; kt++)
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    const int key = k0 + 16 * kt + 4 * g + r;
                    if (key >= S || (causal && key > qi)) s[kt][r] = -INFINITY;
                }
        }
        float mx = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < BK / 16; kt++)
            mx = fmaxf(mx, fmaxf(fmaxf(s[kt][0], s[kt][1]), fmaxf(s[kt][2], s[kt][3])));
        mx = wave_xor_max(mx) * sl2;
        const bool need = mx > m + RESCALE_SLACK;
        if (__any(need)) {
            const float mn = need ? mx : m;
            const float alpha = exp2f(m - mn);
            l = l * alpha;
#pragma unroll
            for (int i = 0; i < D / 16; i++) o[i] = o[i] * alpha;
            m = mn;
        }
        const float mu = (m == -INFINITY) ? 0.0f : m;
#pragma unroll
        for (int kt = 0; kt < BK / 16; kt++) {
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float p = exp2f(__builtin_fmaf(s[kt][r], sl2, -mu));
                l = l + p;
                const float* vrow = &sV[buf][(16 * kt + 4 * g + r) * RS + lq];
#pragma unroll
                for (int dt = 0; dt < D / 16; dt++)
                    o[dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(vrow[16 * dt], p, o[dt], 0, 0, 0);
            }
        }
        if (t + 1 < t_end) lstore(buf ^ 1);
        __syncthreads();
    }

    l = wave_xor_sum(l);
    if (qi >= L) return;
    const int64_t row = ((int64_t)b * Hq + h) * L + qi;
    if (nsplit_row == 1) {
        const float inv = 1.0f / l;
        float* op = Og + row * D;
#pragma unroll
        for (int dt = 0; dt < D / 16; dt++)
            *reinterpret_cast<float4*>(op + 16 * dt + 4 * g) =
                make_float4(o[dt][0] * inv, o[dt][1] * inv, o[dt][2] * inv, o[dt][3] * inv);
        if (lse && g == 0) lse[row] = m * LN2 + logf(l);
    } else {
        float* po = part_o + (row * nsplit + split) * D;
#pragma unroll
        for (int dt = 0; dt < D / 16; dt++)
            *reinterpret_cast<float4*>(po + 16 * dt + 4 * g) = make_float4(o[dt][0], o[dt][1], o[dt][2], o[dt][3]);
        if (g == 0) part_ml[row * nsplit + split] = make_float2(m, l);
    }
}

// Merge the split partials of the rows whose KV range was split: one wave
// per (row, head); lane covers D/64 output elements.
template <int D, typename OT>
__global__ __launch_bounds__(256) void k_prefill_combine(const float* __restrict__ part_o,
                                                       const float2* __restrict__ part_ml, int L, int S, int causal,
                                                       int bk, int tiles_per, int nsplit, int64_t rows,
                                                       OT* __restrict__ out, float* __restrict__ lse) {
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const int qi = (int)(row % L);
    const int q0 = qi / PF_BQ * PF_BQ;
    const int kend = causal ? min(S, q0 + PF_BQ) : S;
    const int ntiles_row = (kend + bk - 1) / bk;
    const int ns = (ntiles_row + tiles_per - 1) / tiles_per;
    if (ns <= 1) return;  // written directly by the prefill kernel
    const float2* ml = part_ml + row * nsplit;
    float mm = -INFINITY;
    for (int s = 0; s < ns; s++) mm = fmaxf(mm, ml[s].x);
    const float mu = (mm == -INFINITY) ? 0.0f : mm;
    float tl = 0.0f;
    float acc[D / 64];
#pragma unroll
    for (int e = 0; e < D / 64; e++) acc[e] = 0.0f;
    for (int s = 0; s < ns; s++) {
        const float f = exp2f(ml[s].x - mu);
        tl = tl + ml[s].y * f;
        const float* po = part_o + (row * nsplit + s) * D;
#pragma unroll
        for (int e = 0; e < D / 64; e++) acc[e] = acc[e] + po[lane + 64 * e] * f;
    }
    const float inv = 1.0f / tl;
#pragma unroll
    for (int e = 0; e < D / 64; e++) {
        const float v = acc[e] * inv;
        if constexpr (sizeof(OT) == 2)
            out[row * D + lane + 64 * e] = bf16_from_f32(v);
        else
            out[row * D + lane + 64 * e] = v;
    }
    if (lse && lane == 0) lse[row] = mu * LN2 + logf(tl);
}

// ---------------------------------------------------------------------------
// Decode (one query token per sequence), bf16, split-KV.
// Grid (splits of 256 keys, Hkv * groups, B); a workgroup of 4 waves covers
// one split of one sequence for NR query heads that share a key/value head;
// each wave takes 64 keys and issues all of its K and V loads at once (32 KB
// per wave at D=128), so the HBM stream is limited by occupancy, not by
// round trips. Per wave:
//   S^T  : MFMA 16x16x32 with K rows straight from HBM (16 B per lane),
//          query columns 0..NR-1 real, the rest zero;
//   P.V  : VALU, lane (key group g = lane>>4, d slice DL*(lane&15)) over its
//          16 V chunks, probabilities broadcast from LDS.
// The four waves merge in LDS and write one (m, l, O) partial per split;
// k_decode_combine merges the splits.
// ---------------------------------------------------------------------------

constexpr int DEC_WAVE_KEYS = 64;
constexpr int DEC_SPLIT = 4 * DEC_WAVE_KEYS;  // keys per workgroup

template <int D, int NR>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
void k_decode_bf16(const uint16_t* __restrict__ Qg, const uint16_t* __restrict__ Kc, const uint16_t* __restrict__ Vc,
                   int Hq, int Hkv, int nrep, int cap, const int32_t* __restrict__ lens, int nsplit, float sl2,
                   float* __restrict__ part_o, float2* __restrict__ part_ml) {
    static_assert(D == 128 || D == 64, "head dim");
    constexpr int DL = D / 16;  // d values per lane in P.V
    __shared__ float sP[4][NR][DEC_WAVE_KEYS];
    __shared__ float sO[4][NR][D];
    __shared__ float2 sML[4][NR];

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int lq = lane & 15, g = lane >> 4;
    const int groups = nrep / NR;
    const int kvh = blockIdx.y / groups, grp = blockIdx.y % groups;
    const int b = blockIdx.z, split = blockIdx.x;
    int len = lens[b];
    len = len < 0 ? 0 : (len > cap ? cap : len);
    if (split * DEC_SPLIT >= len) return;  // uniform over the workgroup
    const int k0 = split * DEC_SPLIT + w * DEC_WAVE_KEYS;
    const int nk = min(max(len - k0, 0), DEC_WAVE_KEYS);
    const int hq0 = kvh * nrep + grp * NR;
    const uint16_t* kp = Kc + ((int64_t)b * Hkv + kvh) * cap * D;
    const uint16_t* vp = Vc + ((int64_t)b * Hkv + kvh) * cap * D;

    // all loads of this wave up front
    uint4 kf[4][D / 32];
#pragma unroll
    for (int kt = 0; kt < 4; kt++) {
        const int key = 16 * kt + lq;
#pragma unroll
        for (int c = 0; c < D / 32; c++) {
            kf[kt][c] = make_uint4(0, 0, 0, 0);
            if (key < nk) kf[kt][c] = *reinterpret_cast<const uint4*>(kp + (int64_t)(k0 + key) * D + 32 * c + 8 * g);
        }
    }
    typedef typename std::conditional<DL == 8, uint4, uint2>::type vchunk;
    vchunk vv[16];
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int kk = 4 * i + g;
        vv[i] = vchunk{};
        if (kk < nk) vv[i] = *reinterpret_cast<const vchunk*>(vp + (int64_t)(k0 + kk) * D + DL * lq);
    }
    bf16x8 qf[D / 32];
#pragma unroll
    for (int c = 0; c < D / 32; c++) {
        uint4 v = make_uint4(0, 0, 0, 0);
        if (lq < NR) v = *reinterpret_cast<const uint4*>(Qg + ((int64_t)b * Hq + hq0 + lq) * D + 32 * c + 8 * g);
        qf[c] = __builtin_bit_cast(bf16x8, v);
    }

    f32x4 s[4];
#pragma unroll
    for (int kt = 0; kt < 4; kt++) {
        s[kt] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < D / 32; c++)
            s[kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, kf[kt][c]), qf[c], s[kt], 0, 0, 0);
    }
    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 4; kt++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            if (16 * kt + 4 * g + r >= nk) s[kt][r] = -INFINITY;
            mx = fmaxf(mx, s[kt][r]);
        }
    const float m = wave_xor_max(mx) * sl2;
    const float mu = (m == -INFINITY) ? 0.0f : m;
    float l = 0.0f;
#pragma unroll
    for (int kt = 0; kt < 4; kt++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const float p = exp2f(__builtin_fmaf(s[kt][r], sl2, -mu));
            l = l + p;
            if (lq < NR) sP[w][lq][16 * kt + 4 * g + r] = p;
        }
    l = wave_xor_sum(l);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

    float o[NR][DL];
#pragma unroll
    for (int hh = 0; hh < NR; hh++)
#pragma unroll
        for (int e = 0; e < DL; e++) o[hh][e] = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int kk = 4 * i + g;
        float vf[DL];
        uint32_t ws[DL / 2];
        __builtin_memcpy(ws, &vv[i], sizeof(ws));
#pragma unroll
        for (int e = 0; e < DL / 2; e++) {
            vf[2 * e] = __builtin_bit_cast(float, ws[e] << 16);
            vf[2 * e + 1] = __builtin_bit_cast(float, ws[e] & 0xffff0000u);
        }
#pragma unroll
        for (int hh = 0; hh < NR; hh++) {
            const float p = sP[w][hh][kk];  // 0 for keys past the end
#pragma unroll
            for (int e = 0; e < DL; e++) o[hh][e] = __builtin_fmaf(p, vf[e], o[hh][e]);
        }
    }
#pragma unroll
    for (int hh = 0; hh < NR; hh++)
#pragma unroll
        for (int e = 0; e < DL; e++) o[hh][e] = wave_xor_sum(o[hh][e]);
    if (g == 0) {
#pragma unroll
        for (int hh = 0; hh < NR; hh++)
#pragma unroll
            for (int e = 0; e < DL; e += 4)
                *reinterpret_cast<float4*>(&sO[w][hh][DL * lq + e]) =
                    make_float4(o[hh][e], o[hh][e + 1], o[hh][e + 2], o[hh][e + 3]);
        if (lq < NR) sML[w][lq] = make_float2(m, l);
    }
    __syncthreads();
    // merge the four waves: thread -> (head, d)
    for (int idx = tid; idx < NR * D; idx += 256) {
        const int hh = idx / D, d = idx % D;
        float mm = -INFINITY;
#pragma unroll
        for (int ww = 0; ww < 4; ww++) mm = fmaxf(mm, sML[ww][hh].x);
        const float mm_u = (mm == -INFINITY) ? 0.0f : mm;
        float tl = 0.0f, acc = 0.0f;
#pragma unroll
        for (int ww = 0; ww < 4; ww++) {
            const float f = exp2f(sML[ww][hh].x - mm_u);
            tl = tl + sML[ww][hh].y * f;
            acc = acc + sO[ww][hh][d] * f;
        }
        const int64_t prow = ((int64_t)b * Hq + hq0 + hh) * nsplit + split;
        part_o[prow * D + d] = acc;
        if (d == 0) part_ml[prow] = make_float2(mm, tl);
    }
}

template <int D>
__global__ __launch_bounds__(D) void k_decode_combine(const float* __restrict__ part_o,
                                                    const float2* __restrict__ part_ml,
                                                    const int32_t* __restrict__ lens, int Hq, int cap, int nsplit,
                                                    uint16_t* __restrict__ out, float* __restrict__ lse) {
    const int h = blockIdx.x, b = blockIdx.y, d = threadIdx.x;
    int len = lens[b];
    len = len < 0 ? 0 : (len > cap ? cap : len);
    int ns = (len + DEC_SPLIT - 1) / DEC_SPLIT;
    ns = ns < nsplit ? ns : nsplit;  // a length above max_len is truncated, never read past
    const int64_t base = ((int64_t)b * Hq + h) * nsplit;
    float mm = -INFINITY;
    for (int s = 0; s < ns; s++) mm = fmaxf(mm, part_ml[base + s].x);
    const float mu = (mm == -INFINITY) ? 0.0f : mm;
    float tl = 0.0f, acc = 0.0f;
    for (int s = 0; s < ns; s++) {
        const float2 ml = part_ml[base + s];
        const float f = exp2f(ml.x - mu);
        tl = tl + ml.y * f;
        acc = acc + part_o[(base + s) * D + d] * f;
    }
    out[((int64_t)b * Hq + h) * D + d] = bf16_from_f32(acc / tl);
    if (lse && d == 0) lse[(int64_t)b * Hq + h] = mu * LN2 + logf(tl);
}

const char* OP = "aten._scaled_dot_product_flash_attention_for_cpu.default";

tn_status refuse_head_dim(int64_t D) {
    char buf[256];
    std::snprintf(buf, sizeof buf,
                  "%s: head_dim %lld is not implemented on the hip device (kernels exist for 64 and 128)", OP,
                  (long long)D);
    return fail(TN_ENOTIMPL, buf);
}

// KV tiles per split for a prefill: long rows are split so that the longest
// work item is about a quarter of the longest row once there are fewer query
// blocks than it takes to fill the device; rows that fit stay whole.
int prefill_tiles_per_split(int64_t B, int64_t Hq, int64_t L, int64_t S, int causal, int bk) {
    const int64_t nqb = (L + PF_BQ - 1) / PF_BQ;
    const int64_t kend = causal ? std::min<int64_t>(S, nqb * PF_BQ) : S;
    const int64_t ntiles = (kend + bk - 1) / bk;
    const int64_t items = B * Hq * nqb;
    if (items >= 2048 || ntiles <= 8) return (int)std::max<int64_t>(ntiles, 1);
    return (int)std::max<int64_t>(8, (ntiles + 3) / 4);
}

}  // namespace
}  // namespace tn

using namespace tn;

extern "C" {

tn_status tn_sdpa_fwd(void* stream, int dtype, const void* q, const void* k, const void* v, int64_t B, int64_t Hq,
                      int64_t Hkv, int64_t L, int64_t S, int64_t D, const void* attn_mask, int mask_dtype,
                      int is_causal, double scale, void* out, float* lse) {
    if (dtype != TN_F32 && dtype != TN_BF16) {
        const char* name = dtype == TN_F16 ? "Half" : dtype == TN_F64 ? "Double" : "an unknown type";
        return fail(dtype == TN_F16 || dtype == TN_F64 ? TN_ENOTIMPL : TN_EINVAL,
                    std::string("scaled_dot_product_attention_flash_attention: ") + name +
                        " is not implemented on the hip device (float32 and bfloat16 are)");
    }
    if (B < 0 || Hq < 0 || L < 0 || S < 0 || D < 0 || Hkv < 0)
        return fail(TN_EINVAL, std::string(OP) + ": negative dimension");
    if (D == 0 || S == 0) {
        char buf[256];
        std::snprintf(buf, sizeof buf,
                      "%s: a zero key length or head dimension (query [%lld, %lld, %lld, %lld], key [%lld, %lld, "
                      "%lld, %lld]) is not implemented in torch._C shim",
                      OP, (long long)B, (long long)Hq, (long long)L, (long long)D, (long long)B, (long long)Hkv,
                      (long long)S, (long long)D);
        return fail(TN_ENOTIMPL, buf);
    }
    if (Hkv == 0 || Hq % Hkv != 0) {
        char buf[384];
        std::snprintf(buf, sizeof buf,
                      "%s: grouped-query attention with %lld query heads and %lld key/value heads is not implemented "
                      "in torch._C shim -- the head counts do not divide",
                      OP, (long long)Hq, (long long)Hkv);
        return fail(TN_ENOTIMPL, buf);
    }
    if (attn_mask) {
        (void)mask_dtype;
        return fail(TN_ENOTIMPL, std::string(OP) + ": an attn_mask is not implemented on the hip device yet "
                                                   "(is_causal is); pass the mask to the CPU device");
    }
    if (D != 64 && D != 128) return refuse_head_dim(D);
    if (B * Hq * L == 0) return TN_OK;  // nothing to write (aten.rs:10242-10259 returns empty zeros)
    if (!q || !k || !v || !out) return fail(TN_EVALUE, std::string(OP) + ": null pointer");
    if (L > INT32_MAX || S > INT32_MAX || Hq > 65535 || B > 65535)
        return fail(TN_EVALUE, std::string(OP) + ": shape too large");
    const double sc = std::isnan(scale) ? 1.0 / std::sqrt((double)D) : scale;
    const float sl2 = (float)sc * LOG2E;
    hipStream_t st = (hipStream_t)stream;
    const int c = is_causal ? 1 : 0;
    const int bk = (dtype == TN_F32 && D == 128) ? 32 : PF_BK;
    const int64_t nqb = cdiv(L, PF_BQ);
    const int64_t kend_max = is_causal ? std::min<int64_t>(S, nqb * PF_BQ) : S;
    const int tiles_per = prefill_tiles_per_split(B, Hq, L, S, c, bk);
    const int nsplit = (int)cdiv(cdiv(kend_max, bk), tiles_per);
    float* part_o = nullptr;
    float2* part_ml = nullptr;
    const int64_t rows = B * Hq * L;
    if (nsplit > 1) {
        const size_t po = (size_t)rows * nsplit * D * sizeof(float);
        const size_t pm = (size_t)rows * nsplit * sizeof(float2);
        void* ws = nullptr;
        tn_status s = workspace(st, po + pm, &ws);
        if (s != TN_OK) return s;
        part_o = static_cast<float*>(ws);
        part_ml = reinterpret_cast<float2*>(static_cast<char*>(ws) + po);
    }
    if (nqb * nsplit > INT32_MAX) return fail(TN_EVALUE, std::string(OP) + ": shape too large");
    dim3 grid((unsigned)(nqb * nsplit), (unsigned)Hq, (unsigned)B);
    if (dtype == TN_BF16) {
        auto qq = static_cast<const uint16_t*>(q);
        auto kk = static_cast<const uint16_t*>(k);
        auto vv = static_cast<const uint16_t*>(v);
        auto oo = static_cast<uint16_t*>(out);
        if (D == 64)
            hipLaunchKernelGGL(k_fa_bf16<64>, grid, dim3(256), 0, st, qq, kk, vv, (int)Hq, (int)Hkv, (int)L, (int)S,
                               sl2, c, tiles_per, nsplit, oo, lse, part_o, part_ml);
        else
            hipLaunchKernelGGL(k_fa_bf16<128>, grid, dim3(256), 0, st, qq, kk, vv, (int)Hq, (int)Hkv, (int)L,
                               (int)S, sl2, c, tiles_per, nsplit, oo, lse, part_o, part_ml);
        TN_LAUNCHED();
        if (nsplit > 1) {
            const unsigned g2 = (unsigned)cdiv(rows, 4);
            if (D == 64)
                hipLaunchKernelGGL((k_prefill_combine<64, uint16_t>), dim3(g2), dim3(256), 0, st, part_o, part_ml,
                                   (int)L, (int)S, c, bk, tiles_per, nsplit, rows, oo, lse);
            else
                hipLaunchKernelGGL((k_prefill_combine<128, uint16_t>), dim3(g2), dim3(256), 0, st, part_o, part_ml,
                                   (int)L, (int)S, c, bk, tiles_per, nsplit, rows, oo, lse);
            TN_LAUNCHED();
        }
    } else {
        auto qq = static_cast<const float*>(q);
        auto kk = static_cast<const float*>(k);
        auto vv = static_cast<const float*>(v);
        auto oo = static_cast<float*>(out);
        if (D == 64)
            hipLaunchKernelGGL((k_fa_f32<64, 64>), grid, dim3(256), 0, st, qq, kk, vv, (int)Hq, (int)Hkv, (int)L,
                               (int)S, sl2, c, tiles_per, nsplit, oo, lse, part_o, part_ml);
        else
            hipLaunchKernelGGL((k_fa_f32<128, 32>), grid, dim3(256), 0, st, qq, kk, vv, (int)Hq, (int)Hkv, (int)L,
                               (int)S, sl2, c, tiles_per, nsplit, oo, lse, part_o, part_ml);
        TN_LAUNCHED();
        if (nsplit > 1) {
            const unsigned g2 = (unsigned)cdiv(rows, 4);
            if (D == 64)
                hipLaunchKernelGGL((k_prefill_combine<64, float>), dim3(g2), dim3(256), 0, st, part_o, part_ml,
                                   (int)L, (int)S, c, bk, tiles_per, nsplit, rows, oo, lse);
            else
                hipLaunchKernelGGL((k_prefill_combine<128, float>), dim3(g2), dim3(256), 0, st, part_o, part_ml,
                                   (int)L, (int)S, c, bk, tiles_per, nsplit, rows, oo, lse);
            TN_LAUNCHED();
        }
    }
    return TN_OK;
}

tn_status tn_sdpa_decode(void* stream, int dtype, const void* q, const void* k_cache, const void* v_cache, int64_t B,
                         int64_t Hq, int64_t Hkv, int64_t cap, int64_t D, const int32_t* lens, int64_t max_len,
                         double scale, void* out, float* lse) {
    if (dtype != TN_BF16)
        return fail(TN_ENOTIMPL, "sdpa_decode: only bfloat16 KV caches are implemented on the hip device");
    if (B < 0 || Hq < 0 || Hkv <= 0 || cap <= 0 || D <= 0 || max_len < 1 || max_len > cap)
        return fail(TN_EINVAL, "sdpa_decode: need Hkv > 0, cap > 0 and 1 <= max_len <= cap");
    if (Hq % Hkv != 0) {
        char buf[256];
        std::snprintf(buf, sizeof buf,
                      "sdpa_decode: grouped-query attention with %lld query heads and %lld key/value heads -- the "
                      "head counts do not divide",
                      (long long)Hq, (long long)Hkv);
        return fail(TN_ENOTIMPL, buf);
    }
    if (D != 64 && D != 128) return refuse_head_dim(D);
    if (B == 0 || Hq == 0) return TN_OK;
    if (!q || !k_cache || !v_cache || !out || !lens) return fail(TN_EVALUE, "sdpa_decode: null pointer");
    if (B > 65535 || Hq > 65535 || cap > INT32_MAX) return fail(TN_EVALUE, "sdpa_decode: shape too large");
    const int nrep = (int)(Hq / Hkv);
    // query heads per workgroup: the largest of 8, 4, 3, 2, 1 that divides the group
    const int nr = nrep % 8 == 0 ? 8 : nrep % 4 == 0 ? 4 : nrep % 3 == 0 ? 3 : nrep % 2 == 0 ? 2 : 1;
    const int nsplit = (int)cdiv(max_len, DEC_SPLIT);
    const size_t po = (size_t)B * Hq * nsplit * D * sizeof(float);
    const size_t pm = (size_t)B * Hq * nsplit * sizeof(float2);
    void* ws = nullptr;
    hipStream_t st = (hipStream_t)stream;
    tn_status s = workspace(st, po + pm, &ws);
    if (s != TN_OK) return s;
    float* part_o = static_cast<float*>(ws);
    float2* part_ml = reinterpret_cast<float2*>(static_cast<char*>(ws) + po);
    const double sc = std::isnan(scale) ? 1.0 / std::sqrt((double)D) : scale;
    const float sl2 = (float)sc * LOG2E;
    auto qq = static_cast<const uint16_t*>(q);
    auto kk = static_cast<const uint16_t*>(k_cache);
    auto vv = static_cast<const uint16_t*>(v_cache);
    dim3 grid((unsigned)nsplit, (unsigned)(Hkv * (nrep / nr)), (unsigned)B);
#define TN_DEC(DD, NR)                                                                                            \
    hipLaunchKernelGGL((k_decode_bf16<DD, NR>), grid, dim3(256), 0, st, qq, kk, vv, (int)Hq, (int)Hkv, nrep,      \
                       (int)cap, lens, nsplit, sl2, part_o, part_ml)
#define TN_DEC_D(DD)                       \
    switch (nr) {                          \
        case 8: TN_DEC(DD, 8); break;      \
        case 4: TN_DEC(DD, 4); break;      \
        case 3: TN_DEC(DD, 3); break;      \
        case 2: TN_DEC(DD, 2); break;      \
        default: TN_DEC(DD, 1); break;     \
    }
    if (D == 128) {
        TN_DEC_D(128)
    } else {
        TN_DEC_D(64)
    }
#undef TN_DEC_D
#undef TN_DEC
    TN_LAUNCHED();
    auto oo = static_cast<uint16_t*>(out);
    if (D == 128)
        hipLaunchKernelGGL(k_decode_combine<128>, dim3((unsigned)Hq, (unsigned)B), dim3(128), 0, st, part_o, part_ml,
                           lens, (int)Hq, (int)cap, nsplit, oo, lse);
    else
        hipLaunchKernelGGL(k_decode_combine<64>, dim3((unsigned)Hq, (unsigned)B), dim3(64), 0, st, part_o, part_ml,
                           lens, (int)Hq, (int)cap, nsplit, oo, lse);
    TN_LAUNCHED();
    return TN_OK;
}

}  // extern "C"
