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

// sum over the 256 threads of a workgroup, in a fixed order
__device__ inline float block_sum256(float v, float* red) {
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) v = v + __shfl_xor(v, off);
    const int w = threadIdx.x >> 6;
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

__global__ __launch_bounds__(256) void k_rmsnorm(const float* x, int n, const float* __restrict__ w, float eps,
                                                 float* y) {
    __shared__ float red[4];
    const float* xr = x + (int64_t)blockIdx.x * n;
    float* yr = y + (int64_t)blockIdx.x * n;
    float ss = 0.0f;
    for (int c = threadIdx.x; c < n; c += 256) {
        const float v = xr[c];
        ss = ss + v * v;
    }
    // every read of the row precedes the barrier inside, so y may alias x
    const float var = block_sum256(ss, red) / (float)n;
    const float r = 1.0f / sqrtf(var + eps);
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
__device__ inline bool arg_before(float v, int i, float w, int j) {
    const bool nv = v != v, nw = w != w;
    if (nv || nw) return nv && (!nw || i < j);
    return v > w || (v == w && i < j);
}

__global__ __launch_bounds__(1024) void k_argmax(const float* __restrict__ x, int n, int32_t* __restrict__ out) {
    __shared__ float sv[1024];
    __shared__ int si[1024];
    const float* xr = x + (int64_t)blockIdx.x * n;
    float bv = -INFINITY;
    int bi = n;  // loses every tie against a real element
    for (int c = threadIdx.x; c < n; c += 1024) {
        const float v = xr[c];
        if (arg_before(v, c, bv, bi)) {
            bv = v;
            bi = c;
        }
    }
    sv[threadIdx.x] = bv;
    si[threadIdx.x] = bi;
    __syncthreads();
    for (int half = 512; half >= 1; half >>= 1) {
        if ((int)threadIdx.x < half) {
            const int o = threadIdx.x + half;
            if (arg_before(sv[o], si[o], sv[threadIdx.x], si[threadIdx.x])) {
                sv[threadIdx.x] = sv[o];
                si[threadIdx.x] = si[o];
            }
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) out[blockIdx.x] = si[0] < n ? si[0] : 0;
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

// end of a decode step: advance the position, pick the next input token
__global__ void k_llama_advance(int32_t* state, int32_t* tokens, const int32_t* prompt, int prompt_len, int cap) {
    if (threadIdx.x != 0) return;
    const int pos = state[0] + 1;
    const int next = pos < prompt_len ? prompt[pos] : state[3];
    if (pos < cap) tokens[pos] = next;
    state[0] = pos;
    state[1] = pos + 1;
    state[2] = next;
}

}  // namespace

// scratch layout of a decode step, in floats
struct LlamaWork {
    int64_t h, x, qkv, attn, tmp, gu, part_o, part_ml, total;
};

static LlamaWork llama_work(const tn_llama* m) {
    LlamaWork w;
    const int64_t nsplit = cdiv(m->cap, DECODE_SPLIT_KEYS);
    const int64_t qkv = (m->n_heads + 2 * m->n_kv_heads) * m->head_dim;
    int64_t o = 0;
    auto take = [&](int64_t n) {
        const int64_t at = o;
        o += (n + 63) / 64 * 64;  // 256-byte aligned
        return at;
    };
    w.h = take(m->hidden);
    w.x = take(std::max(m->hidden, m->inter));
    w.qkv = take(qkv);
    w.attn = take(m->n_heads * m->head_dim);
    w.tmp = take(m->hidden);
    w.gu = take(2 * m->inter);
    w.part_o = take(m->n_heads * nsplit * m->head_dim);
    w.part_ml = take(m->n_heads * nsplit * 2);
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
    if (m->hidden > INT32_MAX || m->inter > INT32_MAX || m->vocab > INT32_MAX || m->cap > INT32_MAX)
        return fail(TN_EVALUE, "tn_llama: shape too large");
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
    if (m > INT32_MAX || n > INT32_MAX - 1024) return fail(TN_EVALUE, "aten.argmax.default: shape too large");
    hipLaunchKernelGGL(k_argmax, dim3((unsigned)m), dim3(1024), 0, (hipStream_t)stream, x, (int)n, out);
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

tn_status tn_llama_step(void* stream, const tn_llama* m) {
    tn_status s = check_model(m);
    if (s != TN_OK) return s;
    hipStream_t st = (hipStream_t)stream;
    const LlamaWork w = llama_work(m);
    float* h = m->work + w.h;
    float* x = m->work + w.x;
    float* qkv = m->work + w.qkv;
    float* attn = m->work + w.attn;
    float* tmp = m->work + w.tmp;
    float* gu = m->work + w.gu;
    float* part_o = m->work + w.part_o;
    float2* part_ml = reinterpret_cast<float2*>(m->work + w.part_ml);
    const int64_t H = m->hidden, D = m->head_dim, Hq = m->n_heads, Hkv = m->n_kv_heads, I = m->inter;
    const int64_t nqkv = (Hq + 2 * Hkv) * D;
    int32_t* pos = m->state;      // [0]: position of this token
    int32_t* len = m->state + 1;  // [1]: KV length after appending it
    int32_t* tok = m->state + 2;  // [2]: this token
    const double nan = std::nan("");
#define TN_TRY(call)                   \
    do {                               \
        tn_status e_ = (call);         \
        if (e_ != TN_OK) return e_;    \
    } while (0)
    TN_TRY(tn_embedding(st, tok, 1, m->embed, m->vocab, H, h));
    for (int64_t l = 0; l < m->n_layers; l++) {
        const tn_llama_layer& L = m->layers[l];
        TN_TRY(tn_rmsnorm(st, h, 1, H, L.ln1, m->eps, x));
        TN_TRY(tn_q4_0_linear(st, x, TN_F32, 1, H, L.qkv.qs, L.qkv.d, nqkv, nullptr, qkv, TN_F32));
        TN_TRY(tn_rope(st, qkv, 1, Hq + Hkv, D, m->inv_freq, pos));  // q heads, then k heads
        TN_TRY(tn_kv_append(st, qkv + Hq * D, qkv + (Hq + Hkv) * D, 1, Hkv, D, L.k_cache, L.v_cache, m->cap, pos));
        TN_TRY(decode_launch(st, TN_F32, qkv, L.k_cache, L.v_cache, 1, Hq, Hkv, m->cap, D, len, m->cap, nan, attn,
                             nullptr, part_o, part_ml));
        TN_TRY(tn_q4_0_linear(st, attn, TN_F32, 1, Hq * D, L.o.qs, L.o.d, H, nullptr, tmp, TN_F32));
        TN_TRY(tn_add(st, h, tmp, H, h));
        TN_TRY(tn_rmsnorm(st, h, 1, H, L.ln2, m->eps, x));
        TN_TRY(tn_q4_0_linear(st, x, TN_F32, 1, H, L.gate_up.qs, L.gate_up.d, 2 * I, nullptr, gu, TN_F32));
        TN_TRY(tn_silu_mul(st, gu, gu + I, I, x));
        TN_TRY(tn_q4_0_linear(st, x, TN_F32, 1, I, L.down.qs, L.down.d, H, nullptr, tmp, TN_F32));
        TN_TRY(tn_add(st, h, tmp, H, h));
    }
    TN_TRY(tn_rmsnorm(st, h, 1, H, m->norm, m->eps, x));
    TN_TRY(tn_q4_0_linear(st, x, TN_F32, 1, H, m->lm_head.qs, m->lm_head.d, m->vocab, nullptr, m->logits, TN_F32));
    TN_TRY(tn_argmax(st, m->logits, 1, m->vocab, m->state + 3));
    hipLaunchKernelGGL(k_llama_advance, dim3(1), dim3(64), 0, st, m->state, m->tokens, m->prompt,
                       (int)m->prompt_len, (int)m->cap);
    TN_LAUNCHED();
#undef TN_TRY
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
