// Scaled dot-product attention on gfx950: flash prefill (bf16 and f32) and
// split-KV decode over per-sequence KV caches.
//
// Semantics are the reference's aten._scaled_dot_product_flash_attention_for_cpu
// (torchnative/rust/torch_c/src/aten.rs:10092-10440): softmax(q k^T * scale
// [+ upper-left causal -inf]) v with f32 accumulation, GQA by indexing key/value
// head h / (Hq/Hkv), logsumexp over the masked, scaled scores. The blocked
// online softmax follows the structure of upstream's CPU flash kernel that the
// reference reproduces in flash.rs:587-780 (rescale by exp(m_old - m_new), P
// narrowed to the input dtype between the products for bf16).
//
// Layout trick shared by all kernels: scores are computed transposed,
// S^T = K . Q^T, so that in the 16x16 MFMA result layout (lane l holds
// C[4*(l>>4) + r][l & 15]) each lane owns one query (column l & 15) and four
// keys per 16-key tile. Row statistics are then in-lane plus two cross-lane
// steps, and the output is accumulated transposed, O^T = V^T . P^T, where the
// lane's own probabilities are directly the B operand and the lane again owns
// its query's column, so the online rescale needs no data movement.
#include "tn_common.h"

namespace tn {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr float LOG2E = 1.4426950408889634f;
constexpr float LN2 = 0.69314718055994531f;

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

__device__ inline uint32_t pack2_bf16(float a, float b) {
    return (uint32_t)bf16_from_f32(a) | ((uint32_t)bf16_from_f32(b) << 16);
}

// ---------------------------------------------------------------------------
// bf16 prefill. Workgroup = 4 waves = 64 queries of one (batch, head); each
// wave owns 16 queries. K/V tiles of 64 keys are staged in LDS (K as is, V
// transposed), then per tile:
//   S^T  : 4 key-tiles x D/32 MFMA 16x16x32 (A = K rows, B = Q^T in registers)
//   P    : exp2(S * scale*log2e - m), narrowed to bf16
//   O^T += D/16 d-tiles x 2 MFMA 16x16x32 (A = V^T rows, B = P^T)
// MFMA K-slot order for a 32-key chunk u: lane group g holds keys
// {32u + 4g + r, 32u + 16 + 4g + r : r = 0..3}, which is where S^T put them.
// ---------------------------------------------------------------------------

template <int D>
__global__ __launch_bounds__(256) void k_fa_bf16(const uint16_t* __restrict__ Qg, const uint16_t* __restrict__ Kg,
                                               const uint16_t* __restrict__ Vg, int Hq, int Hkv, int L, int S,
                                               float sl2, int causal, uint16_t* __restrict__ Og,
                                               float* __restrict__ lse) {
    constexpr int BQ = 64, BK = 64;
    constexpr int KS = D + 8;   // K tile row stride (bf16)
    constexpr int VS = BK + 8;  // V^T tile row stride (bf16)
    __shared__ __align__(16) uint16_t sK[BK * KS];
    __shared__ __align__(16) uint16_t sVt[D * VS];

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int lq = lane & 15, g = lane >> 4;
    const int qt = (int)gridDim.x - 1 - (int)blockIdx.x;  // longest causal rows first
    const int h = blockIdx.y, b = blockIdx.z;
    const int kvh = h / (Hq / Hkv);
    const int q0 = qt * BQ;
    const int qi = q0 + w * 16 + lq;
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
    f32x4 o[D / 16];
#pragma unroll
    for (int i = 0; i < D / 16; i++) o[i] = (f32x4){0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY, l = 0.0f;

    const int kend = causal ? min(S, q0 + BQ) : S;
    const int ntiles = (kend + BK - 1) / BK;
    for (int t = 0; t < ntiles; t++) {
        const int k0 = t * BK;
        // stage K rows
#pragma unroll
        for (int it = 0; it < (BK * D / 8) / 256; it++) {
            const int c = tid + it * 256;
            const int r = c / (D / 8), part = c % (D / 8);
            uint4 v = make_uint4(0, 0, 0, 0);
            if (k0 + r < S) v = *reinterpret_cast<const uint4*>(kp + (int64_t)(k0 + r) * D + part * 8);
            *reinterpret_cast<uint4*>(sK + r * KS + part * 8) = v;
        }
        // stage V transposed: each thread moves a 4-key x 4-d block
#pragma unroll
        for (int it = 0; it < (BK * D / 16) / 256; it++) {
            const int idx = tid + it * 256;
            const int dg = idx % (D / 4), kg = idx / (D / 4);
            uint2 rows[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int key = k0 + 4 * kg + i;
                rows[i] = make_uint2(0, 0);
                if (key < S) rows[i] = *reinterpret_cast<const uint2*>(vp + (int64_t)key * D + 4 * dg);
            }
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const int sh = (j & 1) * 16;
                const uint32_t e0 = ((j < 2 ? rows[0].x : rows[0].y) >> sh) & 0xffffu;
                const uint32_t e1 = ((j < 2 ? rows[1].x : rows[1].y) >> sh) & 0xffffu;
                const uint32_t e2 = ((j < 2 ? rows[2].x : rows[2].y) >> sh) & 0xffffu;
                const uint32_t e3 = ((j < 2 ? rows[3].x : rows[3].y) >> sh) & 0xffffu;
                *reinterpret_cast<uint2*>(sVt + (4 * dg + j) * VS + 4 * kg) = make_uint2(e0 | (e1 << 16), e2 | (e3 << 16));
            }
        }
        __syncthreads();

        // S^T for 64 keys x this wave's 16 queries
        f32x4 s[4];
#pragma unroll
        for (int kt = 0; kt < 4; kt++) {
            s[kt] = (f32x4){0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < D / 32; c++) {
                const bf16x8 ka = *reinterpret_cast<const bf16x8*>(sK + (16 * kt + lq) * KS + 32 * c + 8 * g);
                s[kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka, qf[c], s[kt], 0, 0, 0);
            }
        }
        // masks (upper-left causal, key tail)
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
#pragma unroll
            for (int r = 0; r < 4; r++) mx = fmaxf(mx, s[kt][r]);
        mx = wave_xor_max(mx);
        const float mnew = fmaxf(m, mx * sl2);
        const float mu = (mnew == -INFINITY) ? 0.0f : mnew;
        const float alpha = exp2f(m - mu);
        l = l * alpha;
#pragma unroll
        for (int i = 0; i < D / 16; i++) o[i] = o[i] * alpha;
        float p[4][4];
#pragma unroll
        for (int kt = 0; kt < 4; kt++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                p[kt][r] = exp2f(__builtin_fmaf(s[kt][r], sl2, -mu));
                l = l + p[kt][r];
            }
        m = mnew;
        bf16x8 pf[2];
#pragma unroll
        for (int u = 0; u < 2; u++) {
            uint4 pk;
            pk.x = pack2_bf16(p[2 * u][0], p[2 * u][1]);
            pk.y = pack2_bf16(p[2 * u][2], p[2 * u][3]);
            pk.z = pack2_bf16(p[2 * u + 1][0], p[2 * u + 1][1]);
            pk.w = pack2_bf16(p[2 * u + 1][2], p[2 * u + 1][3]);
            pf[u] = __builtin_bit_cast(bf16x8, pk);
        }
#pragma unroll
        for (int dt = 0; dt < D / 16; dt++) {
#pragma unroll
            for (int u = 0; u < 2; u++) {
                const uint16_t* row = sVt + (16 * dt + lq) * VS + 32 * u + 4 * g;
                const uint2 lo = *reinterpret_cast<const uint2*>(row);
                const uint2 hi = *reinterpret_cast<const uint2*>(row + 16);
                const bf16x8 va = __builtin_bit_cast(bf16x8, make_uint4(lo.x, lo.y, hi.x, hi.y));
                o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va, pf[u], o[dt], 0, 0, 0);
            }
        }
        __syncthreads();
    }

    l = wave_xor_sum(l);
    if (qi < L) {
        const float inv = 1.0f / l;
        uint16_t* op = Og + (((int64_t)b * Hq + h) * L + qi) * D;
#pragma unroll
        for (int dt = 0; dt < D / 16; dt++) {
            // O^T[d = 16dt + 4g + r][q = lq]
            uint2 v;
            v.x = pack2_bf16(o[dt][0] * inv, o[dt][1] * inv);
            v.y = pack2_bf16(o[dt][2] * inv, o[dt][3] * inv);
            *reinterpret_cast<uint2*>(op + 16 * dt + 4 * g) = v;
        }
        if (lse && g == 0) lse[((int64_t)b * Hq + h) * L + qi] = m * LN2 + logf(l);
    }
}

// ---------------------------------------------------------------------------
// f32 prefill: same decomposition on v_mfma_f32_16x16x4_f32 (K = 4 per op).
//   S^T : lane (key lq, group g) feeds K[key][4c + g]; Q^T from registers.
//   O^T : for key slot r of tile kt, lane group g feeds V[16kt + 4g + r][d]
//         and its own P at (kt, r), so V stays in natural layout in LDS.
// Row strides are padded to 4 mod 64 dwords, so the 64 lanes of each LDS read
// hit 64 distinct banks.
// ---------------------------------------------------------------------------

template <int D, int BK>
__global__ __launch_bounds__(256) void k_fa_f32(const float* __restrict__ Qg, const float* __restrict__ Kg,
                                              const float* __restrict__ Vg, int Hq, int Hkv, int L, int S,
                                              float sl2, int causal, float* __restrict__ Og,
                                              float* __restrict__ lse) {
    constexpr int BQ = 64;
    constexpr int RS = D + 4;
    __shared__ __align__(16) float sK[BK * RS];
    __shared__ __align__(16) float sV[BK * RS];

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int lq = lane & 15, g = lane >> 4;
    const int qt = (int)gridDim.x - 1 - (int)blockIdx.x;
    const int h = blockIdx.y, b = blockIdx.z;
    const int kvh = h / (Hq / Hkv);
    const int q0 = qt * BQ;
    const int qi = q0 + w * 16 + lq;
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

    const int kend = causal ? min(S, q0 + BQ) : S;
    const int ntiles = (kend + BK - 1) / BK;
    for (int t = 0; t < ntiles; t++) {
        const int k0 = t * BK;
#pragma unroll
        for (int it = 0; it < (BK * D / 4) / 256; it++) {
            const int c = tid + it * 256;
            const int r = c / (D / 4), part = c % (D / 4);
            float4 kv = make_float4(0.f, 0.f, 0.f, 0.f), vv = kv;
            if (k0 + r < S) {
                kv = *reinterpret_cast<const float4*>(kp + (int64_t)(k0 + r) * D + part * 4);
                vv = *reinterpret_cast<const float4*>(vp + (int64_t)(k0 + r) * D + part * 4);
            }
            *reinterpret_cast<float4*>(sK + r * RS + part * 4) = kv;
            *reinterpret_cast<float4*>(sV + r * RS + part * 4) = vv;
        }
        __syncthreads();

        f32x4 s[BK / 16];
#pragma unroll
        for (int kt = 0; kt < BK / 16; kt++) {
            s[kt] = (f32x4){0.f, 0.f, 0.f, 0.f};
            const float* krow = sK + (16 * kt + lq) * RS + g;
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
#pragma unroll
            for (int r = 0; r < 4; r++) mx = fmaxf(mx, s[kt][r]);
        mx = wave_xor_max(mx);
        const float mnew = fmaxf(m, mx * sl2);
        const float mu = (mnew == -INFINITY) ? 0.0f : mnew;
        const float alpha = exp2f(m - mu);
        l = l * alpha;
#pragma unroll
        for (int i = 0; i < D / 16; i++) o[i] = o[i] * alpha;
        m = mnew;
#pragma unroll
        for (int kt = 0; kt < BK / 16; kt++) {
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float p = exp2f(__builtin_fmaf(s[kt][r], sl2, -mu));
                l = l + p;
                const float* vrow = sV + (16 * kt + 4 * g + r) * RS + lq;
#pragma unroll
                for (int dt = 0; dt < D / 16; dt++)
                    o[dt] = __builtin_amdgcn_mfma_f32_16x16x4f32(vrow[16 * dt], p, o[dt], 0, 0, 0);
            }
        }
        __syncthreads();
    }

    l = wave_xor_sum(l);
    if (qi < L) {
        const float inv = 1.0f / l;
        float* op = Og + (((int64_t)b * Hq + h) * L + qi) * D;
#pragma unroll
        for (int dt = 0; dt < D / 16; dt++)
            *reinterpret_cast<float4*>(op + 16 * dt + 4 * g) =
                make_float4(o[dt][0] * inv, o[dt][1] * inv, o[dt][2] * inv, o[dt][3] * inv);
        if (lse && g == 0) lse[((int64_t)b * Hq + h) * L + qi] = m * LN2 + logf(l);
    }
}

// ---------------------------------------------------------------------------
// Decode (one query token per sequence), bf16, split-KV.
// Grid (split groups, Hkv, B); each wave is one split of SPLIT keys of one
// sequence and serves the NREP query heads that share the key/value head:
//   S^T  : MFMA 16x16x32 with K rows read straight from HBM (16 B per lane),
//          query columns 0..NREP-1 real, the rest zero;
//   P.V  : VALU, lane (key group kq = lane>>4, d slice 8*(lane&15)) reads
//          16-byte V chunks, four keys per load instruction across the wave.
// Each wave writes (m, l, O) partials; k_decode_combine merges the splits.
// ---------------------------------------------------------------------------

constexpr int DEC_SPLIT = 128;  // keys per wave
constexpr int DEC_WAVES = 4;

template <int D, int NREP>
__global__ __launch_bounds__(256) void k_decode_bf16(const uint16_t* __restrict__ Qg, const uint16_t* __restrict__ Kc,
                                                   const uint16_t* __restrict__ Vc, int Hq, int Hkv, int cap,
                                                   const int32_t* __restrict__ lens, int nsplit, float sl2,
                                                   float* __restrict__ part_o, float2* __restrict__ part_ml) {
    static_assert(D == 128 || D == 64, "head dim");
    constexpr int DL = D / 16;  // d values per lane in P.V (8 for D=128)
    __shared__ float sP[DEC_WAVES][NREP][64];
    __shared__ float sA[DEC_WAVES][NREP];

    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int lq = lane & 15, g = lane >> 4;
    const int kvh = blockIdx.y, b = blockIdx.z;
    const int split = blockIdx.x * DEC_WAVES + w;
    int len = lens[b];
    len = len < 0 ? 0 : (len > cap ? cap : len);
    const int ks = split * DEC_SPLIT;
    if (split >= nsplit) return;
    const int ke = min(len, ks + DEC_SPLIT);
    const int hq0 = kvh * NREP;
    const uint16_t* kp = Kc + ((int64_t)b * Hkv + kvh) * cap * D;
    const uint16_t* vp = Vc + ((int64_t)b * Hkv + kvh) * cap * D;

    bf16x8 qf[D / 32];
#pragma unroll
    for (int c = 0; c < D / 32; c++) {
        uint4 v = make_uint4(0, 0, 0, 0);
        if (lq < NREP) v = *reinterpret_cast<const uint4*>(Qg + ((int64_t)b * Hq + hq0 + lq) * D + 32 * c + 8 * g);
        qf[c] = __builtin_bit_cast(bf16x8, v);
    }
    float o[NREP][DL];
#pragma unroll
    for (int hh = 0; hh < NREP; hh++)
#pragma unroll
        for (int e = 0; e < DL; e++) o[hh][e] = 0.0f;
    float m = -INFINITY, l = 0.0f;  // per query column lq (lanes lq < NREP meaningful)

    for (int k0 = ks; k0 < ke; k0 += 64) {
        f32x4 s[4];
#pragma unroll
        for (int kt = 0; kt < 4; kt++) {
            s[kt] = (f32x4){0.f, 0.f, 0.f, 0.f};
            const int key = k0 + 16 * kt + lq;
#pragma unroll
            for (int c = 0; c < D / 32; c++) {
                uint4 kv = make_uint4(0, 0, 0, 0);
                if (key < ke) kv = *reinterpret_cast<const uint4*>(kp + (int64_t)key * D + 32 * c + 8 * g);
                s[kt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, kv), qf[c], s[kt], 0, 0, 0);
            }
        }
        float mx = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < 4; kt++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                if (k0 + 16 * kt + 4 * g + r >= ke) s[kt][r] = -INFINITY;
                mx = fmaxf(mx, s[kt][r]);
            }
        mx = wave_xor_max(mx);
        const float mnew = fmaxf(m, mx * sl2);
        const float mu = (mnew == -INFINITY) ? 0.0f : mnew;
        const float alpha = exp2f(m - mu);
        l = l * alpha;
        m = mnew;
#pragma unroll
        for (int kt = 0; kt < 4; kt++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const float p = exp2f(__builtin_fmaf(s[kt][r], sl2, -mu));
                l = l + p;
                if (lq < NREP) sP[w][lq][16 * kt + 4 * g + r] = p;
            }
        if (lq < NREP && g == 0) sA[w][lq] = alpha;
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // P.V: lane covers keys k0 + 4i + g (i = 0..15), d = DL*lq .. +DL
#pragma unroll
        for (int hh = 0; hh < NREP; hh++) {
            const float a = sA[w][hh];
#pragma unroll
            for (int e = 0; e < DL; e++) o[hh][e] = o[hh][e] * a;
        }
        const int nk = ke - k0;
#pragma unroll 4
        for (int i = 0; i < 16; i++) {
            const int kk = 4 * i + g;
            if (kk < nk) {
                float vf[DL];
                if constexpr (DL == 8) {
                    const uint4 vv = *reinterpret_cast<const uint4*>(vp + (int64_t)(k0 + kk) * D + DL * lq);
                    const uint32_t ws[4] = {vv.x, vv.y, vv.z, vv.w};
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        vf[2 * e] = bf16_to_f32((uint16_t)(ws[e] & 0xffffu));
                        vf[2 * e + 1] = bf16_to_f32((uint16_t)(ws[e] >> 16));
                    }
                } else {
                    const uint2 vv = *reinterpret_cast<const uint2*>(vp + (int64_t)(k0 + kk) * D + DL * lq);
                    const uint32_t ws[2] = {vv.x, vv.y};
#pragma unroll
                    for (int e = 0; e < 2; e++) {
                        vf[2 * e] = bf16_to_f32((uint16_t)(ws[e] & 0xffffu));
                        vf[2 * e + 1] = bf16_to_f32((uint16_t)(ws[e] >> 16));
                    }
                }
#pragma unroll
                for (int hh = 0; hh < NREP; hh++) {
                    const float p = sP[w][hh][kk];
#pragma unroll
                    for (int e = 0; e < DL; e++) o[hh][e] = __builtin_fmaf(p, vf[e], o[hh][e]);
                }
            }
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    // reduce the four key groups of P.V, and the four lane groups of l
#pragma unroll
    for (int hh = 0; hh < NREP; hh++)
#pragma unroll
        for (int e = 0; e < DL; e++) o[hh][e] = wave_xor_sum(o[hh][e]);
    l = wave_xor_sum(l);
    const int64_t base = ((int64_t)b * Hq + hq0) * nsplit + split;
    if (g == 0) {
#pragma unroll
        for (int hh = 0; hh < NREP; hh++) {
            float* dst = part_o + (base + (int64_t)hh * nsplit) * D + DL * lq;
#pragma unroll
            for (int e = 0; e < DL; e += 4)
                *reinterpret_cast<float4*>(dst + e) = make_float4(o[hh][e], o[hh][e + 1], o[hh][e + 2], o[hh][e + 3]);
        }
        if (lq < NREP) part_ml[base + (int64_t)lq * nsplit] = make_float2(m, l);
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
    dim3 grid((unsigned)cdiv(L, 64), (unsigned)Hq, (unsigned)B);
    const int c = is_causal ? 1 : 0;
    if (dtype == TN_BF16) {
        auto qq = static_cast<const uint16_t*>(q);
        auto kk = static_cast<const uint16_t*>(k);
        auto vv = static_cast<const uint16_t*>(v);
        auto oo = static_cast<uint16_t*>(out);
        if (D == 64)
            hipLaunchKernelGGL(k_fa_bf16<64>, grid, dim3(256), 0, st, qq, kk, vv, (int)Hq, (int)Hkv, (int)L, (int)S,
                               sl2, c, oo, lse);
        else
            hipLaunchKernelGGL(k_fa_bf16<128>, grid, dim3(256), 0, st, qq, kk, vv, (int)Hq, (int)Hkv, (int)L,
                               (int)S, sl2, c, oo, lse);
    } else {
        auto qq = static_cast<const float*>(q);
        auto kk = static_cast<const float*>(k);
        auto vv = static_cast<const float*>(v);
        auto oo = static_cast<float*>(out);
        if (D == 64)
            hipLaunchKernelGGL((k_fa_f32<64, 64>), grid, dim3(256), 0, st, qq, kk, vv, (int)Hq, (int)Hkv, (int)L,
                               (int)S, sl2, c, oo, lse);
        else
            hipLaunchKernelGGL((k_fa_f32<128, 32>), grid, dim3(256), 0, st, qq, kk, vv, (int)Hq, (int)Hkv, (int)L,
                               (int)S, sl2, c, oo, lse);
    }
    TN_LAUNCHED();
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
    const int64_t nrep = Hq / Hkv;
    if (nrep != 1 && nrep != 2 && nrep != 4 && nrep != 8 && nrep != 16)
        return fail(TN_ENOTIMPL, "sdpa_decode: query heads per key/value head must be 1, 2, 4, 8 or 16");
    if (B == 0 || Hq == 0) return TN_OK;
    if (!q || !k_cache || !v_cache || !out || !lens) return fail(TN_EVALUE, "sdpa_decode: null pointer");
    if (B > 65535 || Hkv > 65535 || cap > INT32_MAX) return fail(TN_EVALUE, "sdpa_decode: shape too large");
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
    dim3 grid((unsigned)cdiv(nsplit, DEC_WAVES), (unsigned)Hkv, (unsigned)B);
#define TN_DEC(DD, NR)                                                                                            \
    hipLaunchKernelGGL((k_decode_bf16<DD, NR>), grid, dim3(256), 0, st, qq, kk, vv, (int)Hq, (int)Hkv, (int)cap, \
                       lens, nsplit, sl2, part_o, part_ml)
#define TN_DEC_D(DD)                       \
    switch (nrep) {                        \
        case 1: TN_DEC(DD, 1); break;      \
        case 2: TN_DEC(DD, 2); break;      \
        case 4: TN_DEC(DD, 4); break;      \
        case 8: TN_DEC(DD, 8); break;      \
        default: TN_DEC(DD, 16); break;    \
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
