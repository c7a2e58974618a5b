// The per-token ops of a Llama-style decode step (f32) and the step driver
// for a q4_0 decoder: embedding, RMSNorm, rotary embedding, SiLU-gated
// product, residual add, argmax, KV-cache append; tn_llama_step chains them
// with tn_q4_0_linear and the f32 decode attention, with every per-step
// quantity (position, token) on the device so that a run of steps can be
// captured as one HIP graph.
//
// Semantics follow the reference's ops as transformers' LlamaForCausalLM
// calls them on an f32 model (torchnative/rust/torch_c/src/aten.rs; each
// entry point in include/tnhip.h cites its lines). These are small, latency-
// bound kernels: one workgroup per row for the reductions, one thread per
// element elsewhere.
#include <algorithm>
#include <cmath>

#include "tn_common.h"

namespace tn {
namespace {

__global__ __launch_bounds__(256) void k_embedding(const int32_t* __restrict__ ids, const float* __restrict__ table,
                                                   int64_t vocab, int dim, float* __restrict__ out) {
    const int i = blockIdx.y;
    const int c = blockIdx.x * 256 + threadIdx.x;
    if (c >= dim) return;
    const int32_t id = ids[i];
    out[(int64_t)i * dim + c] = (id >= 0 && id < vocab) ? table[(int64_t)id * dim + c] : NAN;
}

// The decode step's first launch: the token's embedding row into h (as
// k_embedding), and the cosine and sine of this position's RoPE angles,
// cosf/sinf of pos * inv_freq[j] as k_rope computes them, so that every
// layer's rotation reads them instead of evaluating both functions again.
__global__ __launch_bounds__(256) void k_step_begin(const int32_t* __restrict__ state,
                                                    const float* __restrict__ table, int64_t vocab, int dim,
                                                    float* __restrict__ h, const float* __restrict__ inv_freq,
                                                    int half, float2* __restrict__ rope) {
    const int c = blockIdx.x * 256 + threadIdx.x;
    const int32_t id = state[2];
    if (c < dim) h[c] = (id >= 0 && id < vocab) ? table[(int64_t)id * dim + c] : NAN;
    if (blockIdx.x == 0 && threadIdx.x < half) {
        const float f = (float)state[0] * inv_freq[threadIdx.x];
        rope[threadIdx.x] = make_float2(cosf(f), sinf(f));
    }
}

// thread t adds the squares of elements 1024p + 4t .. 1024p + 4t + 3, p =
// 0, 1, ..., in order, then block_sum256: the order the q4_0 GEMV's fused
// RMSNorm prologue reproduces
__global__ __launch_bounds__(256) void k_rmsnorm(const float* x, int n, const float* __restrict__ w, float eps,
                                                 float* y) {
    __shared__ float red[4];
    const float* xr = x + (int64_t)blockIdx.x * n;
    float* yr = y + (int64_t)blockIdx.x * n;
    float ss = 0.0f;
    for (int64_t c0 = threadIdx.x * 4; c0 < n; c0 += 1024) {
        const int64_t ce = c0 + 4 < n ? c0 + 4 : n;
        for (int64_t c = c0; c < ce; c++) {
            const float v = xr[c];
            ss = ss + v * v;
        }
    }
    // every read of the row precedes the barrier inside, so y may alias x
    const float r = rms_scale(block_sum256(ss, red), n, eps);
    for (int c = threadIdx.x; c < n; c += 256) yr[c] = w[c] * (xr[c] * r);
}

// one workgroup of d/2 threads per (token, head) row
__global__ void k_rope(float* __restrict__ x, int heads, int d, const float* __restrict__ inv_freq,
                       const int32_t* __restrict__ pos) {
    const int row = blockIdx.x, i = threadIdx.x, half = d / 2;
    float* xr = x + (int64_t)row * d;
    const float f = (float)pos[row / heads] * inv_freq[i];
    const float c = cosf(f), s = sinf(f);
    const float x1 = xr[i], x2 = xr[i + half];
    xr[i] = x1 * c + (-x2) * s;
    xr[i + half] = x2 * c + x1 * s;
}

// The decode step's RoPE and KV-cache append in one launch, d/2 threads per
// row of the token's qkv vector [hq + 2 hkv][d]: q rows are rotated in place,
// k rows are rotated into the k cache at the device position, v rows are
// copied into the v cache. The rotation is k_rope's, bit for bit.
__global__ void k_rope_append(float* __restrict__ qkv, int hq, int hkv, int d, const float* __restrict__ inv_freq,
                              const int32_t* __restrict__ pos, float* __restrict__ kc, float* __restrict__ vc,
                              int cap) {
    const int row = blockIdx.x, i = threadIdx.x, half = d / 2;
    const int p = pos[0];
    float* xr = qkv + (int64_t)row * d;
    if (row >= hq + hkv) {
        if (p < 0 || p >= cap) return;
        float* dst = vc + ((int64_t)(row - hq - hkv) * cap + p) * d;
        dst[i] = xr[i];
        dst[i + half] = xr[i + half];
        return;
    }
    const float f = (float)p * inv_freq[i];
    const float c = cosf(f), s = sinf(f);
    const float x1 = xr[i], x2 = xr[i + half];
    const float y1 = x1 * c + (-x2) * s, y2 = x2 * c + x1 * s;
    if (row < hq) {
        xr[i] = y1;
        xr[i + half] = y2;
        return;
    }
    if (p < 0 || p >= cap) return;
    float* dst = kc + ((int64_t)(row - hq) * cap + p) * d;
    dst[i] = y1;
    dst[i + half] = y2;
}

// The decode step's attention for caches of at most STEP_MAX_SPLITS splits of
// STEP_SPLIT keys, with the step's RoPE and KV append folded in. One
// workgroup per (split, kv head) covers the NR query heads that share the kv
// head: it rotates their queries (into LDS) and, in the split that holds the
// new position, rotates the new key, writes it and the new value to the
// caches and uses them for that row (other rows come from the caches); the
// rotation's cosines and sines come from the step's table (k_step_begin). D/4
// lanes share a row, a float4 each, all of the split's K and V rows in flight
// at once; row dot products reduce with DPP. Each split writes an (O, m, l)
// partial per query head (m in log2 units), merged by the o projection's
// PRO_COMBINE prologue. The rotation is k_rope's, bit for bit.
constexpr float STEP_LOG2E = 1.4426950408889634f;

template <int D, int NR>
__global__ __launch_bounds__(256) void k_step_attn(const float* __restrict__ qkv, int hq, int hkv,
                                                  const float2* __restrict__ rope,
                                                  const int32_t* __restrict__ state, float* __restrict__ kc,
                                                  float* __restrict__ vc, int cap, float sl2, int nsplit,
                                                  float* __restrict__ part_o, float2* __restrict__ part_ml) {
    constexpr int TPK = D / 4;             // lanes per row
    constexpr int SLOTS = 256 / TPK;       // rows per load instruction of the workgroup
    constexpr int U = STEP_SPLIT / SLOTS;  // rows per lane
    static_assert(U * SLOTS == STEP_SPLIT && (TPK == 16 || TPK == 32), "shape");
    // the rotated query heads [NR][D], then two words per thread where idle
    // threads store (the rotation has no branch for the compiler to sink the
    // query loads into, behind the cache rows)
    __shared__ __align__(16) float sq[NR * D + 2 * 256];
    // the new key (rotated) and value [2][D], then four words per thread where
    // the other threads store (as sq's padding)
    __shared__ __align__(16) float snew[2 * D + 4 * 256];
    __shared__ float smax[NR][4], ssum[NR][4];
    __shared__ float4 so[4][NR][TPK];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int c = tid % TPK, kl = tid / TPK;
    const int sp = blockIdx.x, kvh = blockIdx.y;
    const int k0 = sp * STEP_SPLIT;
    // Every load is an unconditional buffer load (an idle lane's offset lies
    // past its descriptor and reads zero), so the compiler counts the loads
    // in flight exactly. The rotation's operands go first -- thread i <
    // NR * D/2 rotates pair i of the query heads, thread i < D/2 also pair i
    // of the new key -- then the split's K and V rows below cap, before the
    // position is known (rows at or past it are replaced or masked where
    // they are used), so that the rotation waits only for its own operands
    // while the cache rows are in flight. A split past the length runs
    // through with every row masked (its partial is never merged): an early
    // exit there let the compiler sink every load below the position's
    // read, so that all of them waited for it.
    constexpr int half = D / 2;
    constexpr int QP = (NR * half + 255) / 256;  // query pairs per thread
    const buf_rsrc rq = make_rsrc(qkv + (int64_t)kvh * NR * D, (uint32_t)(NR * D * 4));
    const buf_rsrc rkn = make_rsrc(qkv + (int64_t)(hq + kvh) * D, (uint32_t)(D * 4));
    const buf_rsrc rvn = make_rsrc(qkv + (int64_t)(hq + hkv + kvh) * D, (uint32_t)(D * 4));
    const buf_rsrc rrope = make_rsrc(rope, (uint32_t)(half * 8));
    float qx1[QP], qx2[QP];
    float2 qcs[QP];
#pragma unroll
    for (int i = 0; i < QP; i++) {
        const int pi = tid + 256 * i;
        const int hh = pi / half, j = pi - hh * half;
        const bool on = pi < NR * half;
        qx1[i] = buf_load_f(rq, on ? (uint32_t)(hh * D + j) * 4u : BUF_OOB);
        qx2[i] = buf_load_f(rq, on ? (uint32_t)(hh * D + j + half) * 4u : BUF_OOB);
        qcs[i] = buf_load_f2(rrope, on ? (uint32_t)j * 8u : BUF_OOB);
    }
    const bool kon = tid < half;
    const float kx1 = buf_load_f(rkn, kon ? (uint32_t)tid * 4u : BUF_OOB);
    const float kx2 = buf_load_f(rkn, kon ? (uint32_t)(tid + half) * 4u : BUF_OOB);
    const float kvv1 = buf_load_f(rvn, kon ? (uint32_t)tid * 4u : BUF_OOB);
    const float kvv2 = buf_load_f(rvn, kon ? (uint32_t)(tid + half) * 4u : BUF_OOB);
    const float2 kcs = buf_load_f2(rrope, kon ? (uint32_t)tid * 8u : BUF_OOB);
    const buf_rsrc rk = make_rsrc(kc + (int64_t)kvh * cap * D, (uint32_t)cap * (uint32_t)(D * 4));
    const buf_rsrc rv = make_rsrc(vc + (int64_t)kvh * cap * D, (uint32_t)cap * (uint32_t)(D * 4));
    const float4 zero = make_float4(0.f, 0.f, 0.f, 0.f);
    float4 kr[U], vr[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
        const int t = k0 + u * SLOTS + kl;
        const uint32_t off = t < cap ? (uint32_t)(t * D + 4 * c) * 4u : BUF_OOB;
        kr[u] = buf_load_f4(rk, off);
        vr[u] = buf_load_f4(rv, off);
    }
    __builtin_amdgcn_sched_barrier(0);  // every load issued before the rotation waits for its operands
    const int pos = state[0];
    const int len = pos < 0 ? 0 : (pos + 1 < cap ? pos + 1 : cap);
    const int ncached = pos < len ? pos : len;  // rows taken from the caches
    const bool fresh = pos >= k0 && pos < k0 + STEP_SPLIT && pos < len;
#pragma unroll
    for (int i = 0; i < QP; i++) {
        const int pi = tid + 256 * i;
        const int hh = pi / half, j = pi - hh * half;
        const bool on = pi < NR * half;
        const float cs = qcs[i].x, sn = qcs[i].y;
        const float x1 = qx1[i], x2 = qx2[i];
        sq[on ? hh * D + j : NR * D + 2 * tid] = x1 * cs + (-x2) * sn;
        sq[on ? hh * D + j + half : NR * D + 2 * tid + 1] = x2 * cs + x1 * sn;
    }
    // the new key's rotation in every split, without a branch (only the
    // fresh split reads it back; behind a branch its loads were sunk there,
    // after the cache rows)
    const float ny1 = kx1 * kcs.x + (-kx2) * kcs.y, ny2 = kx2 * kcs.x + kx1 * kcs.y;
    snew[kon ? tid : 2 * D + 4 * tid] = ny1;
    snew[kon ? tid + half : 2 * D + 4 * tid + 1] = ny2;
    snew[kon ? D + tid : 2 * D + 4 * tid + 2] = kvv1;
    snew[kon ? D + tid + half : 2 * D + 4 * tid + 3] = kvv2;
    if (fresh && kon) {
        const float y1 = ny1, y2 = ny2, v1 = kvv1, v2 = kvv2;
        float* kd = kc + ((int64_t)kvh * cap + pos) * D;
        float* vd = vc + ((int64_t)kvh * cap + pos) * D;
        kd[tid] = y1;
        kd[tid + half] = y2;
        vd[tid] = v1;
        vd[tid + half] = v2;
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < U; u++) {
        // the new row from LDS; rows past the cached ones hold stale or
        // unwritten values: zero them (a NaN there would survive a zero
        // probability)
        const int t = k0 + u * SLOTS + kl;
        if (fresh && t == pos) {
            kr[u] = reinterpret_cast<const float4*>(snew)[c];
            vr[u] = reinterpret_cast<const float4*>(snew + D)[c];
        } else if (t >= ncached) {
            kr[u] = zero;
            vr[u] = zero;
        }
    }
    float4 qv[NR];
#pragma unroll
    for (int hh = 0; hh < NR; hh++) qv[hh] = reinterpret_cast<const float4*>(sq + hh * D)[c];

    // scores (log2 units), then the split's max per head
    float sc[NR][U];
#pragma unroll
    for (int u = 0; u < U; u++) {
        const bool valid = k0 + u * SLOTS + kl < len;
#pragma unroll
        for (int hh = 0; hh < NR; hh++) {
            float d = qv[hh].x * kr[u].x;
            d = d + qv[hh].y * kr[u].y;
            d = d + qv[hh].z * kr[u].z;
            d = d + qv[hh].w * kr[u].w;
            d = row16_sum(d);
            if constexpr (TPK == 32) d = xor16_sum(d);
            sc[hh][u] = valid ? d * sl2 : -INFINITY;
        }
    }
#pragma unroll
    for (int hh = 0; hh < NR; hh++) {
        float m = sc[hh][0];
#pragma unroll
        for (int u = 1; u < U; u++) m = fmaxf(m, sc[hh][u]);
        if constexpr (TPK == 16) m = xor16_max(m);
        m = xor32_max(m);
        if (lane == 0) smax[hh][w] = m;
    }
    __syncthreads();
    float4 acc[NR];
#pragma unroll
    for (int hh = 0; hh < NR; hh++) {
        const float m = fmaxf(fmaxf(smax[hh][0], smax[hh][1]), fmaxf(smax[hh][2], smax[hh][3]));
        const float mu = (m == -INFINITY) ? 0.0f : m;
        float l = 0.0f;
        acc[hh] = zero;
#pragma unroll
        for (int u = 0; u < U; u++) {
            const float p = exp2f(sc[hh][u] - mu);  // 0 past the end
            l = l + p;
            acc[hh].x = acc[hh].x + p * vr[u].x;
            acc[hh].y = acc[hh].y + p * vr[u].y;
            acc[hh].z = acc[hh].z + p * vr[u].z;
            acc[hh].w = acc[hh].w + p * vr[u].w;
        }
        // over the wave's row slots (lanes c, c + TPK, ...)
        if constexpr (TPK == 16) {
            l = xor16_sum(l);
            acc[hh].x = xor16_sum(acc[hh].x);
            acc[hh].y = xor16_sum(acc[hh].y);
            acc[hh].z = xor16_sum(acc[hh].z);
            acc[hh].w = xor16_sum(acc[hh].w);
        }
        l = xor32_sum(l);
        acc[hh].x = xor32_sum(acc[hh].x);
        acc[hh].y = xor32_sum(acc[hh].y);
        acc[hh].z = xor32_sum(acc[hh].z);
        acc[hh].w = xor32_sum(acc[hh].w);
        if (lane == 0) ssum[hh][w] = l;
        if (lane < TPK) so[w][hh][lane] = acc[hh];
    }
    __syncthreads();
    for (int i = tid; i < NR * TPK; i += 256) {
        const int hh = i / TPK, cc = i - hh * TPK;
        float4 o = so[0][hh][cc];
#pragma unroll
        for (int ww = 1; ww < 4; ww++) {
            o.x = o.x + so[ww][hh][cc].x;
            o.y = o.y + so[ww][hh][cc].y;
            o.z = o.z + so[ww][hh][cc].z;
            o.w = o.w + so[ww][hh][cc].w;
        }
        const int64_t prow = (int64_t)(kvh * NR + hh) * nsplit + sp;
        reinterpret_cast<float4*>(part_o + prow * D)[cc] = o;
        if (cc == 0) {
            const float m = fmaxf(fmaxf(smax[hh][0], smax[hh][1]), fmaxf(smax[hh][2], smax[hh][3]));
            part_ml[prow] = make_float2(m, (ssum[hh][0] + ssum[hh][1]) + (ssum[hh][2] + ssum[hh][3]));
        }
    }
}

__global__ __launch_bounds__(256) void k_silu_mul(const float* gate, const float* up, int64_t n, float* out) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    const float g = gate[i];
    out[i] = (g / (1.0f + expf(-g))) * up[i];
}

__global__ __launch_bounds__(256) void k_add(const float* a, const float* b, int64_t n, float* out) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) out[i] = a[i] + b[i];
}

// (v, i) before (w, j) in argmax order: a NaN first (the earliest), then the
// larger value, then the smaller index
constexpr int ARGMAX_THREADS = 1024;
constexpr int ARGMAX_U = 12;  // loads in flight per thread (49152 f32 = one batch of float4s)

// One workgroup per row. arg_before is a strict total order on (value,
// index) pairs, so the winner does not depend on how the pairs are reduced:
// each thread scans its elements with ARGMAX_U loads in flight (16-byte
// pieces when VEC4: rows 16-byte aligned, n % 4 == 0), then waves reduce by
// shuffles and wave 0 merges the 16 waves.
// ADVANCE (one row): the winner goes to state[3] and the decode step's
// position advances.
template <bool ADVANCE, bool VEC4>
__global__ __launch_bounds__(ARGMAX_THREADS) void k_argmax(const float* __restrict__ x, int n,
                                                          int32_t* __restrict__ out, int32_t* state,
                                                          int32_t* tokens, const int32_t* prompt, int prompt_len,
                                                          int cap) {
    __shared__ float sv[ARGMAX_THREADS / 64];
    __shared__ int si[ARGMAX_THREADS / 64];
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const float* xr = x + (int64_t)blockIdx.x * n;
    float bv = -INFINITY;
    int bi = n;  // loses every tie against a real element
    auto take = [&](float v, int c) {
        if (arg_before(v, c, bv, bi)) {
            bv = v;
            bi = c;
        }
    };
    if (VEC4) {
        // the row in 16-byte pieces, ARGMAX_U pieces per thread in flight
        const float4* x4 = reinterpret_cast<const float4*>(xr);
        const int n4 = n / 4;
        for (int c0 = tid; c0 < n4; c0 += ARGMAX_THREADS * ARGMAX_U) {
            float4 v[ARGMAX_U];
#pragma unroll
            for (int u = 0; u < ARGMAX_U; u++) {
                const int c = c0 + u * ARGMAX_THREADS;
                v[u] = c < n4 ? x4[c] : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
            }
#pragma unroll
            for (int u = 0; u < ARGMAX_U; u++) {
                const int c = c0 + u * ARGMAX_THREADS;
                if (c < n4) {
                    take(v[u].x, 4 * c);
                    take(v[u].y, 4 * c + 1);
                    take(v[u].z, 4 * c + 2);
                    take(v[u].w, 4 * c + 3);
                }
            }
        }
    } else {
        for (int c0 = tid; c0 < n; c0 += ARGMAX_THREADS * ARGMAX_U) {
            float v[ARGMAX_U];
#pragma unroll
            for (int u = 0; u < ARGMAX_U; u++) {
                const int c = c0 + u * ARGMAX_THREADS;
                v[u] = c < n ? xr[c] : -INFINITY;
            }
#pragma unroll
            for (int u = 0; u < ARGMAX_U; u++) {
                const int c = c0 + u * ARGMAX_THREADS;
                if (c < n) take(v[u], c);
            }
        }
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float ov = __shfl_xor(bv, off);
        const int oi = __shfl_xor(bi, off);
        if (arg_before(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
        }
    }
    if (lane == 0) {
        sv[w] = bv;
        si[w] = bi;
    }
    __syncthreads();
    if (w != 0) return;
    constexpr int NW = ARGMAX_THREADS / 64;
    bv = lane < NW ? sv[lane] : -INFINITY;
    bi = lane < NW ? si[lane] : n;
#pragma unroll
    for (int off = NW / 2; off >= 1; off >>= 1) {
        const float ov = __shfl_xor(bv, off);
        const int oi = __shfl_xor(bi, off);
        if (arg_before(ov, oi, bv, bi)) {
            bv = ov;
            bi = oi;
        }
    }
    if (lane != 0) return;
    const int idx = bi < n ? bi : 0;
    if (ADVANCE) {
        state[3] = idx;
        llama_advance(state, tokens, prompt, prompt_len, cap);
    } else {
        out[blockIdx.x] = idx;
    }
}

// one workgroup of d threads per (row, kv head)
__global__ void k_kv_append(const float* __restrict__ k, const float* __restrict__ v, int hkv, int d,
                            float* __restrict__ kc, float* __restrict__ vc, int cap, const int32_t* __restrict__ pos0) {
    const int i = blockIdx.x / hkv, h = blockIdx.x % hkv, c = threadIdx.x;
    const int p = pos0[0] + i;
    if (p < 0 || p >= cap) return;
    const int64_t src = ((int64_t)i * hkv + h) * d + c;
    const int64_t dst = ((int64_t)h * cap + p) * d + c;
    kc[dst] = k[src];
    vc[dst] = v[src];
}

// ---- the prompt in one batched pass (tn_llama_prefill) ----

// Token t of the prompt: its embedding row into h[t], its input id into
// tokens[t], and the cosine and sine of position pos0 + t's RoPE angles
// (cosf/sinf of pos * inv_freq[j], k_rope's arithmetic) into rope[t].
__global__ __launch_bounds__(256) void k_prefill_begin(const int32_t* __restrict__ prompt, int T, int pos0,
                                                       const float* __restrict__ table, int64_t vocab, int dim,
                                                       float* __restrict__ h, int32_t* __restrict__ tokens,
                                                       const float* __restrict__ inv_freq, int half,
                                                       float2* __restrict__ rope) {
    const int t = blockIdx.x;
    const int32_t id = prompt[t];
    for (int c = threadIdx.x; c < dim; c += 256)
        h[(int64_t)t * dim + c] = (id >= 0 && id < vocab) ? table[(int64_t)id * dim + c] : NAN;
    if (threadIdx.x < half) {
        const float f = (float)(pos0 + t) * inv_freq[threadIdx.x];
        rope[(int64_t)t * half + threadIdx.x] = make_float2(cosf(f), sinf(f));
    }
    if (threadIdx.x == 0) tokens[pos0 + t] = id;
}

// The prompt's projected rows qkv [T][hq + 2 hkv][d] split for the batched
// attention and the caches: q heads rotated into q [hq][T][d], k heads
// rotated into kt [hkv][T][d] and the k cache at positions pos0 + t, v heads
// copied into vt [hkv][T][d] and the v cache. d/2 threads per (token, head),
// each a rotated pair (j, j + d/2): k_rope's arithmetic on the prefill's
// cos/sin table, bit for bit.
__global__ void k_prefill_qkv(const float* __restrict__ qkv, int T, int hq, int hkv, int d,
                              const float2* __restrict__ rope, float* __restrict__ q, float* __restrict__ kt,
                              float* __restrict__ vt, float* __restrict__ kc, float* __restrict__ vc, int cap,
                              int pos0) {
    const int t = blockIdx.x, hd = blockIdx.y, i = threadIdx.x, half = d / 2;
    const float* src = qkv + ((int64_t)t * (hq + 2 * hkv) + hd) * d;
    const float x1 = src[i], x2 = src[i + half];
    if (hd < hq + hkv) {
        const float2 cs = rope[(int64_t)t * half + i];
        const float r1 = x1 * cs.x + (-x2) * cs.y;
        const float r2 = x2 * cs.x + x1 * cs.y;
        if (hd < hq) {
            float* dst = q + ((int64_t)hd * T + t) * d;
            dst[i] = r1;
            dst[i + half] = r2;
        } else {
            const int kh = hd - hq;
            float* dst = kt + ((int64_t)kh * T + t) * d;
            dst[i] = r1;
            dst[i + half] = r2;
            if (pos0 + t < cap) {
                float* c = kc + ((int64_t)kh * cap + pos0 + t) * d;
                c[i] = r1;
                c[i + half] = r2;
            }
        }
    } else {
        const int vh = hd - hq - hkv;
        float* dst = vt + ((int64_t)vh * T + t) * d;
        dst[i] = x1;
        dst[i + half] = x2;
        if (pos0 + t < cap) {
            float* c = vc + ((int64_t)vh * cap + pos0 + t) * d;
            c[i] = x1;
            c[i + half] = x2;
        }
    }
}

// The batched attention's output [heads][T][d] back to token rows [T][heads d]
// for the o projection.
__global__ void k_heads_to_rows(const float* __restrict__ a, int T, int heads, int d, float* __restrict__ rows) {
    const int t = blockIdx.x, h = blockIdx.y;
    for (int c = threadIdx.x; c < d; c += blockDim.x)
        rows[((int64_t)t * heads + h) * d + c] = a[((int64_t)h * T + t) * d + c];
}

// the decode state before the prompt's last position: position T - 1 is the
// one being processed, so the lm_head's advance moves to T
__global__ void k_prefill_state(int32_t* state, int last) {
    state[0] = last;
    state[1] = last + 1;
}

}  // namespace

// scratch layout of a decode step, in floats
struct LlamaWork {
    int64_t h, qkv, attn, gu, part_o, part_ml, rope, arg_v, arg_i, total;
};

static LlamaWork llama_work(const tn_llama* m) {
    LlamaWork w;
    // partials of either attention path: splits of DECODE_SPLIT_KEYS or of STEP_SPLIT keys
    const int64_t nsplit = std::max(cdiv(m->cap, DECODE_SPLIT_KEYS), cdiv(m->cap, STEP_SPLIT));
    const int64_t qkv = (m->n_heads + 2 * m->n_kv_heads) * m->head_dim;
    int64_t o = 0;
    auto take = [&](int64_t n) {
        const int64_t at = o;
        o += (n + 63) / 64 * 64;  // 256-byte aligned
        return at;
    };
    w.h = take(m->hidden);
    w.qkv = take(qkv);
    w.attn = take(m->n_heads * m->head_dim);
    w.gu = take(2 * m->inter);
    w.part_o = take(m->n_heads * nsplit * m->head_dim);
    w.part_ml = take(m->n_heads * nsplit * 2);
    w.rope = take(m->head_dim);  // (cos, sin) of the step's position per rotated pair
    w.arg_v = take(GEMV_ARG_MAX_PARTS);   // the lm_head's per-workgroup argmax (values
    w.arg_i = take(GEMV_ARG_MAX_PARTS);   // and indices, as int32)
    w.total = o;
    return w;
}

static tn_status check_model(const tn_llama* m) {
    if (!m || !m->layers || !m->embed || !m->norm || !m->lm_head.qs || !m->lm_head.d || !m->inv_freq ||
        !m->state || !m->tokens || !m->logits || !m->work || (m->prompt_len > 0 && !m->prompt))
        return fail(TN_EVALUE, "tn_llama: null pointer in the model");
    if (m->n_layers < 1 || m->hidden < 1 || m->n_heads < 1 || m->n_kv_heads < 1 || m->inter < 1 || m->vocab < 1 ||
        m->cap < 1 || m->prompt_len < 1 || m->prompt_len > m->cap)
        return fail(TN_EINVAL, "tn_llama: need positive sizes and 1 <= prompt_len <= cap");
    if (m->n_heads * m->head_dim != m->hidden)
        return fail(TN_ENOTIMPL, "tn_llama: n_heads * head_dim must equal hidden");
    if (m->head_dim % 2 != 0 || m->head_dim > 1024)
        return fail(TN_ENOTIMPL, "tn_llama: head_dim must be even and at most 1024");
    if (m->vocab > INT32_MAX - ARGMAX_THREADS * ARGMAX_U || m->cap > INT32_MAX)
        return fail(TN_EVALUE, "tn_llama: shape too large");
    if (m->hidden % 32 != 0 || m->inter % 32 != 0 || m->hidden > LINEAR_DECODE_MAX_K || m->inter > LINEAR_DECODE_MAX_K)
        return fail(TN_ENOTIMPL, "tn_llama: hidden and inter must be multiples of 32 and at most 24576");
    for (int64_t l = 0; l < m->n_layers; l++) {
        const tn_llama_layer& L = m->layers[l];
        if (!L.qkv.qs || !L.qkv.d || !L.o.qs || !L.o.d || !L.gate_up.qs || !L.gate_up.d || !L.down.qs ||
            !L.down.d || !L.ln1 || !L.ln2 || !L.k_cache || !L.v_cache)
            return fail(TN_EVALUE, "tn_llama: null pointer in a layer");
    }
    return decode_check(TN_F32, 1, m->n_heads, m->n_kv_heads, m->cap, m->head_dim, m->cap);
}

}  // namespace tn

using namespace tn;

extern "C" {

tn_status tn_embedding(void* stream, const int32_t* ids, int64_t m, const float* table, int64_t vocab, int64_t dim,
                       float* out) {
    if (m < 0 || vocab < 1 || dim < 1) return fail(TN_EINVAL, "aten.embedding.default: bad sizes");
    if (m == 0) return TN_OK;
    if (!ids || !table || !out) return fail(TN_EVALUE, "aten.embedding.default: null pointer");
    if (m > 65535 || dim > INT32_MAX) return fail(TN_EVALUE, "aten.embedding.default: shape too large");
    hipLaunchKernelGGL(k_embedding, dim3((unsigned)cdiv(dim, 256), (unsigned)m), dim3(256), 0, (hipStream_t)stream,
                       ids, table, vocab, (int)dim, out);
    TN_LAUNCHED();
    return TN_OK;
}

tn_status tn_rmsnorm(void* stream, const float* x, int64_t m, int64_t n, const float* weight, double eps, float* y) {
    if (m < 0 || n < 1) return fail(TN_EINVAL, "rms_norm: bad sizes");
    if (m == 0) return TN_OK;
    if (!x || !weight || !y) return fail(TN_EVALUE, "rms_norm: null pointer");
    if (m > INT32_MAX || n > INT32_MAX) return fail(TN_EVALUE, "rms_norm: shape too large");
    hipLaunchKernelGGL(k_rmsnorm, dim3((unsigned)m), dim3(256), 0, (hipStream_t)stream, x, (int)n, weight,
                       (float)eps, y);
    TN_LAUNCHED();
    return TN_OK;
}

tn_status tn_rope(void* stream, float* x, int64_t m, int64_t heads, int64_t d, const float* inv_freq,
                  const int32_t* pos) {
    if (m < 0 || heads < 1 || d < 2 || d % 2 != 0) return fail(TN_EINVAL, "rotary embedding: bad sizes");
    if (d > 2048) return fail(TN_ENOTIMPL, "rotary embedding: head_dim above 2048 is not implemented");
    if (m == 0) return TN_OK;
    if (!x || !inv_freq || !pos) return fail(TN_EVALUE, "rotary embedding: null pointer");
    if (m * heads > INT32_MAX) return fail(TN_EVALUE, "rotary embedding: shape too large");
    hipLaunchKernelGGL(k_rope, dim3((unsigned)(m * heads)), dim3((unsigned)(d / 2)), 0, (hipStream_t)stream, x,
                       (int)heads, (int)d, inv_freq, pos);
    TN_LAUNCHED();
    return TN_OK;
}

tn_status tn_silu_mul(void* stream, const float* gate, const float* up, int64_t n, float* out) {
    if (n < 0) return fail(TN_EINVAL, "silu_mul: bad size");
    if (n == 0) return TN_OK;
    if (!gate || !up || !out) return fail(TN_EVALUE, "silu_mul: null pointer");
    hipLaunchKernelGGL(k_silu_mul, dim3((unsigned)cdiv(n, 256)), dim3(256), 0, (hipStream_t)stream, gate, up, n,
                       out);
    TN_LAUNCHED();
    return TN_OK;
}

tn_status tn_add(void* stream, const float* a, const float* b, int64_t n, float* out) {
    if (n < 0) return fail(TN_EINVAL, "aten.add.Tensor: bad size");
    if (n == 0) return TN_OK;
    if (!a || !b || !out) return fail(TN_EVALUE, "aten.add.Tensor: null pointer");
    hipLaunchKernelGGL(k_add, dim3((unsigned)cdiv(n, 256)), dim3(256), 0, (hipStream_t)stream, a, b, n, out);
    TN_LAUNCHED();
    return TN_OK;
}

tn_status tn_argmax(void* stream, const float* x, int64_t m, int64_t n, int32_t* out) {
    if (m < 0 || n < 1) return fail(TN_EINVAL, "aten.argmax.default: bad sizes");
    if (m == 0) return TN_OK;
    if (!x || !out) return fail(TN_EVALUE, "aten.argmax.default: null pointer");
    if (m > INT32_MAX || n > INT32_MAX - ARGMAX_THREADS * ARGMAX_U)
        return fail(TN_EVALUE, "aten.argmax.default: shape too large");
    if (n % 4 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0)
        hipLaunchKernelGGL((k_argmax<false, true>), dim3((unsigned)m), dim3(ARGMAX_THREADS), 0, (hipStream_t)stream,
                           x, (int)n, out, nullptr, nullptr, nullptr, 0, 0);
    else
        hipLaunchKernelGGL((k_argmax<false, false>), dim3((unsigned)m), dim3(ARGMAX_THREADS), 0, (hipStream_t)stream,
                           x, (int)n, out, nullptr, nullptr, nullptr, 0, 0);
    TN_LAUNCHED();
    return TN_OK;
}

tn_status tn_kv_append(void* stream, const float* k, const float* v, int64_t m, int64_t hkv, int64_t d,
                       float* k_cache, float* v_cache, int64_t cap, const int32_t* pos0) {
    if (m < 0 || hkv < 1 || d < 1 || cap < 1) return fail(TN_EINVAL, "kv_append: bad sizes");
    if (d > 1024) return fail(TN_ENOTIMPL, "kv_append: head_dim above 1024 is not implemented");
    if (m == 0) return TN_OK;
    if (!k || !v || !k_cache || !v_cache || !pos0) return fail(TN_EVALUE, "kv_append: null pointer");
    if (m * hkv > INT32_MAX || cap > INT32_MAX) return fail(TN_EVALUE, "kv_append: shape too large");
    hipLaunchKernelGGL(k_kv_append, dim3((unsigned)(m * hkv)), dim3((unsigned)d), 0, (hipStream_t)stream, k, v,
                       (int)hkv, (int)d, k_cache, v_cache, (int)cap, pos0);
    TN_LAUNCHED();
    return TN_OK;
}

int64_t tn_llama_work_floats(const tn_llama* model) {
    if (!model) return 0;
    return llama_work(model).total;
}

// One decode step. Per layer, for a cache of at most STEP_MAX_SPLITS *
// STEP_SPLIT keys (five launches):
//   qkv = Q4(rmsnorm(h, ln1))                    linear_decode, RMSNorm prologue
//   rope q, k; append k, v; split attention      k_step_attn -> partials
//   h = h + Q4(merge(partials))                  linear_decode, PRO_COMBINE, residual
//   g = silu(gate) * up, gate_up = Q4(rmsnorm(h, ln2))
//                                                linear_decode, RMSNorm prologue, SiLU epilogue
//   h = h + Q4(g)                                linear_decode, residual
// A longer cache replaces the middle two by k_rope_append, the split-KV decode
// attention with its combine, and the o projection on its output.
// Then logits = Q4(rmsnorm(h, norm)) with per-workgroup argmax partials, and
// one workgroup reducing them and advancing the state.
// The fused linears are bit-identical to the separate ops (tn_rmsnorm,
// tn_q4_0_linear, tn_add, tn_silu_mul); RoPE is tn_rope's arithmetic.
tn_status tn_llama_step(void* stream, const tn_llama* m) {
    tn_status s = check_model(m);
    if (s != TN_OK) return s;
    hipStream_t st = (hipStream_t)stream;
    const LlamaWork w = llama_work(m);
    float* h = m->work + w.h;
    float* qkv = m->work + w.qkv;
    float* attn = m->work + w.attn;
    float* gu = m->work + w.gu;
    float* part_o = m->work + w.part_o;
    float2* part_ml = reinterpret_cast<float2*>(m->work + w.part_ml);
    float2* rope = reinterpret_cast<float2*>(m->work + w.rope);
    const int64_t H = m->hidden, D = m->head_dim, Hq = m->n_heads, Hkv = m->n_kv_heads, I = m->inter;
    const int64_t nqkv = (Hq + 2 * Hkv) * D;
    const float eps = (float)m->eps;
    int32_t* pos = m->state;      // [0]: position of this token
    int32_t* len = m->state + 1;  // [1]: KV length after appending it
    const double nan = std::nan("");
    GemvPro none, ln1, ln2g, fin, comb;
    ln1.eps = ln2g.eps = fin.eps = eps;
    ln2g.glu = 1;
    fin.w = m->norm;
    // short caches: the fused split attention, merged in the o projection
    const int nrep = (int)(Hq / Hkv);
    const int64_t nsplit_step = cdiv(m->cap, STEP_SPLIT);
    const bool fused = nsplit_step <= STEP_MAX_SPLITS && (D == 64 || D == 128) &&
                       (nrep == 1 || nrep == 2 || nrep == 3 || nrep == 4 || nrep == 8);
    comb.part_o = part_o;
    comb.part_ml = part_ml;
    comb.len = len;
    comb.nsplit = (int)nsplit_step;
    comb.head_dim = (int)D;
    while ((1 << comb.head_shift) < comb.head_dim) comb.head_shift++;  // the fused path's D is 64 or 128
    comb.cap = (int)m->cap;
    const float sl2 = (float)(1.0 / std::sqrt((double)D)) * STEP_LOG2E;
    hipLaunchKernelGGL(k_step_begin, dim3((unsigned)cdiv(H, 256)), dim3(256), 0, st, m->state, m->embed, m->vocab,
                       (int)H, h, m->inv_freq, (int)(D / 2), rope);
    TN_LAUNCHED();
    for (int64_t l = 0; l < m->n_layers; l++) {
        const tn_llama_layer& L = m->layers[l];
        ln1.w = L.ln1;
        ln2g.w = L.ln2;
        TN_TRY(linear_decode(st, h, H, PRO_RMSNORM, ln1, L.qkv.qs, L.qkv.d, nqkv, nullptr, qkv));
        if (fused) {
            const dim3 grid((unsigned)nsplit_step, (unsigned)Hkv);
#define TN_STEP_ATTN(DD, NR)                                                                                  \
    hipLaunchKernelGGL((k_step_attn<DD, NR>), grid, dim3(256), 0, st, qkv, (int)Hq, (int)Hkv, rope, pos,        \
                       L.k_cache, L.v_cache, (int)m->cap, sl2, (int)nsplit_step, part_o, part_ml)
#define TN_STEP_ATTN_D(DD)                    \
    switch (nrep) {                           \
        case 1: TN_STEP_ATTN(DD, 1); break;   \
        case 2: TN_STEP_ATTN(DD, 2); break;   \
        case 3: TN_STEP_ATTN(DD, 3); break;   \
        case 4: TN_STEP_ATTN(DD, 4); break;   \
        default: TN_STEP_ATTN(DD, 8); break;  \
    }
            if (D == 64) {
                TN_STEP_ATTN_D(64)
            } else {
                TN_STEP_ATTN_D(128)
            }
#undef TN_STEP_ATTN_D
#undef TN_STEP_ATTN
            TN_LAUNCHED();
            TN_TRY(linear_decode(st, nullptr, Hq * D, PRO_COMBINE, comb, L.o.qs, L.o.d, H, h, h));
        } else {
            hipLaunchKernelGGL(k_rope_append, dim3((unsigned)(Hq + 2 * Hkv)), dim3((unsigned)(D / 2)), 0, st, qkv,
                               (int)Hq, (int)Hkv, (int)D, m->inv_freq, pos, L.k_cache, L.v_cache, (int)m->cap);
            TN_LAUNCHED();
            TN_TRY(decode_launch(st, TN_F32, qkv, L.k_cache, L.v_cache, 1, Hq, Hkv, m->cap, D, len, m->cap, nan,
                                 attn, nullptr, part_o, part_ml));
            TN_TRY(linear_decode(st, attn, Hq * D, PRO_NONE, none, L.o.qs, L.o.d, H, h, h));
        }
        // silu(gate) * up in the gate_up GEMV's epilogue, once, into gu[0, I)
        TN_TRY(linear_decode(st, h, H, PRO_RMSNORM, ln2g, L.gate_up.qs, L.gate_up.d, I, nullptr, gu));
        TN_TRY(linear_decode(st, gu, I, PRO_NONE, none, L.down.qs, L.down.d, H, h, h));
    }
    // the logits with their argmax partials, then the argmax and the state's advance
    fin.arg_v = m->work + w.arg_v;
    fin.arg_i = reinterpret_cast<int32_t*>(m->work + w.arg_i);
    fin.state = m->state;
    fin.tokens = m->tokens;
    fin.prompt = m->prompt;
    fin.prompt_len = (int)m->prompt_len;
    fin.cap = (int)m->cap;
    s = linear_decode_argmax(st, h, H, fin, m->lm_head.qs, m->lm_head.d, m->vocab, m->logits);
    if (s != TN_ENOTIMPL) return s;
    // a row the GEMV does not hold (linear_decode refuses it by name): the
    // logits, then k_argmax
    TN_TRY(linear_decode(st, h, H, PRO_RMSNORM, fin, m->lm_head.qs, m->lm_head.d, m->vocab, nullptr, m->logits));
    if (m->vocab % 4 == 0 && reinterpret_cast<uintptr_t>(m->logits) % 16 == 0)
        hipLaunchKernelGGL((k_argmax<true, true>), dim3(1), dim3(ARGMAX_THREADS), 0, st, m->logits, (int)m->vocab,
                           nullptr, m->state, m->tokens, m->prompt, (int)m->prompt_len, (int)m->cap);
    else
        hipLaunchKernelGGL((k_argmax<true, false>), dim3(1), dim3(ARGMAX_THREADS), 0, st, m->logits, (int)m->vocab,
                           nullptr, m->state, m->tokens, m->prompt, (int)m->prompt_len, (int)m->cap);
    TN_LAUNCHED();
    return TN_OK;
}

// The prompt's first T tokens in one batched pass per layer (the reference's
// prefill: LlamaForCausalLM.forward over the prompt, bench_llama_cpp.py:484-523):
//   h = embed[prompt[0..T)]; per layer: x = rmsnorm(h, ln1); qkv = x W_qkv^T
//   (the q4_0 GEMM, M = T); rope q, k; k, v to the caches; a = causal SDPA
//   over the T positions (the f32 prefill); h += a W_o^T; x = rmsnorm(h, ln2);
//   gu = x W_gate_up^T; h += (silu(gate) * up) W_down^T;
// then the last position's logits and argmax and the state's advance as a
// decode step ends (linear_decode_argmax), so decode steps continue at T.
// Every q4 linear row is the decode GEMV's row bit for bit (the reference's
// batched == one-row property); the attention's summation order is the
// prefill kernel's.
struct PrefillWork {
    int64_t h, x, qkv, q, kt, vt, att, rows, gu, rope, total;
};
static PrefillWork prefill_work(const tn_llama* m, int64_t T) {
    PrefillWork w;
    const int64_t H = m->hidden, D = m->head_dim, Hq = m->n_heads, Hkv = m->n_kv_heads, I = m->inter;
    int64_t o = 0;
    auto take = [&](int64_t n) {
        const int64_t at = o;
        o += (n + 3) & ~(int64_t)3;  // 16-byte aligned pieces
        return at;
    };
    w.h = take(T * H);
    w.x = take(T * H);
    w.qkv = take(T * (Hq + 2 * Hkv) * D);
    w.q = take(T * Hq * D);
    w.kt = take(T * Hkv * D);
    w.vt = take(T * Hkv * D);
    w.att = take(T * Hq * D);
    w.rows = take(T * Hq * D);
    w.gu = take(T * 2 * I);
    w.rope = take(T * D);  // T * D/2 float2
    w.total = o;
    return w;
}

int64_t tn_llama_prefill_work_floats(const tn_llama* model, int64_t tokens) {
    if (!model || tokens < 1) return 0;
    return prefill_work(model, tokens).total;
}

tn_status tn_llama_prefill(void* stream, const tn_llama* m, int64_t T, float* work) {
    tn_status s = check_model(m);
    if (s != TN_OK) return s;
    if (!work) return fail(TN_EVALUE, "tn_llama_prefill: null work buffer");
    if (T < 1 || T > m->prompt_len || T > m->cap)
        return fail(TN_EINVAL, "tn_llama_prefill: need 1 <= tokens <= prompt_len <= cap");
    if (m->head_dim % 2 != 0 || m->head_dim > 1024)
        return fail(TN_ENOTIMPL, "tn_llama_prefill: head_dim must be even and at most 1024");
    hipStream_t st = (hipStream_t)stream;
    const PrefillWork w = prefill_work(m, T);
    const int64_t H = m->hidden, D = m->head_dim, Hq = m->n_heads, Hkv = m->n_kv_heads, I = m->inter;
    const int64_t nqkv = (Hq + 2 * Hkv) * D;
    if (T * std::max(nqkv, 2 * I) > INT32_MAX) return fail(TN_EVALUE, "tn_llama_prefill: prompt too long");
    float* h = work + w.h;
    float* x = work + w.x;
    float2* rope = reinterpret_cast<float2*>(work + w.rope);
    // the o projection reads the attention output in place when a head's
    // rows are whole 32-element blocks
    const bool heads_ok = D % 32 == 0;
    hipLaunchKernelGGL(k_prefill_begin, dim3((unsigned)T), dim3(256), 0, st, m->prompt, (int)T, 0, m->embed,
                       m->vocab, (int)H, h, m->tokens, m->inv_freq, (int)(D / 2), rope);
    TN_LAUNCHED();
    for (int64_t l = 0; l < m->n_layers; l++) {
        const tn_llama_layer& L = m->layers[l];
        TN_TRY(tn_rmsnorm(stream, h, T, H, L.ln1, m->eps, x));
        TN_TRY(linear_prefill(st, x, T, H, XM_ROWS, 0, L.qkv.qs, L.qkv.d, nqkv, nullptr, work + w.qkv));
        hipLaunchKernelGGL(k_prefill_qkv, dim3((unsigned)T, (unsigned)(Hq + 2 * Hkv)), dim3((unsigned)(D / 2)), 0, st,
                           work + w.qkv, (int)T, (int)Hq, (int)Hkv, (int)D, rope, work + w.q, work + w.kt,
                           work + w.vt, L.k_cache, L.v_cache, (int)m->cap, 0);
        TN_LAUNCHED();
        TN_TRY(tn_sdpa_fwd(stream, TN_F32, work + w.q, work + w.kt, work + w.vt, 1, Hq, Hkv, T, T, D, nullptr, 0,
                           nullptr, 1, std::nan(""), work + w.att, nullptr));
        // the o projection reads the attention's [heads][T][D] output as
        // token rows and adds the residual in its epilogue: h += o
        if (heads_ok) {
            TN_TRY(linear_prefill(st, work + w.att, T, Hq * D, XM_HEADS, (int)D, L.o.qs, L.o.d, H, h, h));
        } else {
            hipLaunchKernelGGL(k_heads_to_rows, dim3((unsigned)T, (unsigned)Hq),
                               dim3((unsigned)std::min<int64_t>(D, 256)), 0, st, work + w.att, (int)T, (int)Hq, (int)D,
                               work + w.rows);
            TN_LAUNCHED();
            TN_TRY(linear_prefill(st, work + w.rows, T, Hq * D, XM_ROWS, 0, L.o.qs, L.o.d, H, h, h));
        }
        TN_TRY(tn_rmsnorm(stream, h, T, H, L.ln2, m->eps, x));
        TN_TRY(linear_prefill(st, x, T, H, XM_ROWS, 0, L.gate_up.qs, L.gate_up.d, 2 * I, nullptr, work + w.gu));
        // the down projection takes silu(gate) * up of the gate_up rows in
        // its prepass and adds the residual in its epilogue: h += down(...)
        TN_TRY(linear_prefill(st, work + w.gu, T, I, XM_GLU, 0, L.down.qs, L.down.d, H, h, h));
    }
    // the last position as a decode step ends it: the logits, their argmax
    // and the advance to position T (the prompt's token there, else the argmax)
    hipLaunchKernelGGL(k_prefill_state, dim3(1), dim3(1), 0, st, m->state, (int)(T - 1));
    TN_LAUNCHED();
    const LlamaWork lw = llama_work(m);
    GemvPro fin;
    fin.eps = (float)m->eps;
    fin.w = m->norm;
    fin.arg_v = m->work + lw.arg_v;
    fin.arg_i = reinterpret_cast<int32_t*>(m->work + lw.arg_i);
    fin.state = m->state;
    fin.tokens = m->tokens;
    fin.prompt = m->prompt;
    fin.prompt_len = (int)m->prompt_len;
    fin.cap = (int)m->cap;
    const float* hl = h + (T - 1) * H;
    s = linear_decode_argmax(st, hl, H, fin, m->lm_head.qs, m->lm_head.d, m->vocab, m->logits);
    if (s != TN_ENOTIMPL) return s;
    TN_TRY(linear_decode(st, hl, H, PRO_RMSNORM, fin, m->lm_head.qs, m->lm_head.d, m->vocab, nullptr, m->logits));
    if (m->vocab % 4 == 0 && reinterpret_cast<uintptr_t>(m->logits) % 16 == 0)
        hipLaunchKernelGGL((k_argmax<true, true>), dim3(1), dim3(ARGMAX_THREADS), 0, st, m->logits, (int)m->vocab,
                           nullptr, m->state, m->tokens, m->prompt, (int)m->prompt_len, (int)m->cap);
    else
        hipLaunchKernelGGL((k_argmax<true, false>), dim3(1), dim3(ARGMAX_THREADS), 0, st, m->logits, (int)m->vocab,
                           nullptr, m->state, m->tokens, m->prompt, (int)m->prompt_len, (int)m->cap);
    TN_LAUNCHED();
    return TN_OK;
}

tn_status tn_llama_capture(void* stream, const tn_llama* m, int64_t steps, void** graph) {
    if (!graph) return fail(TN_EVALUE, "tn_llama_capture: null output");
    *graph = nullptr;
    if (!stream) return fail(TN_EINVAL, "tn_llama_capture: capture needs a created stream, not the null stream");
    if (steps < 1) return fail(TN_EINVAL, "tn_llama_capture: steps must be positive");
    tn_status s = check_model(m);
    if (s != TN_OK) return s;
    hipStream_t st = (hipStream_t)stream;
    // capture records the stream's work from here on: it must be idle
    TN_HIP(hipStreamSynchronize(st));
    TN_HIP(hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal));
    for (int64_t i = 0; i < steps; i++) {
        s = tn_llama_step(stream, m);
        if (s != TN_OK) break;
    }
    hipGraph_t g = nullptr;
    const hipError_t e = hipStreamEndCapture(st, &g);
    if (s != TN_OK) {
        if (g) (void)hipGraphDestroy(g);
        return s;
    }
    if (e != hipSuccess) return hip_fail(e, "hipStreamEndCapture");
    hipGraphExec_t exec = nullptr;
    const hipError_t ei = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (ei != hipSuccess) return hip_fail(ei, "hipGraphInstantiate");
    *graph = exec;
    return TN_OK;
}

tn_status tn_graph_launch(void* stream, void* graph) {
    if (!graph) return fail(TN_EVALUE, "tn_graph_launch: null graph");
    TN_HIP(hipGraphLaunch((hipGraphExec_t)graph, (hipStream_t)stream));
    return TN_OK;
}

tn_status tn_graph_destroy(void* graph) {
    if (graph) TN_HIP(hipGraphExecDestroy((hipGraphExec_t)graph));
    return TN_OK;
}

}  // extern "C"
