// The dense "quantised" formats f32 / f16 / bf16 and the dense linear.
//
// `_quantize(t, "f32" | "f16" | "bf16")` stores the weight element by element
// (candle k_quants.rs:2778-2910: GgmlType for f32 copies, for f16 and bf16
// narrows with half's round-to-nearest-even), and `_quantized_linear` on such
// a weight is the exactness control: QMatMul::from_arc widens it to f32 up
// front and takes a plain matmul (candle quantized/mod.rs:836-852), so the
// call must give exactly the bits of the dense linear on the widened weight
// (quant.rs:273-279). Here both go through one kernel, k_dense_linear, whose
// every output is one fixed chain: acc = 0, then acc = fma(x[k], w[k], acc)
// for k = 0, 1, ..., K-1, then acc + bias (the addmm that nn.Linear's bias
// branch emits, aten.rs:9686-9700, adds the bias once after the product).
// The chain does not depend on the tiling, the launch or the row count, so
// a batched call equals its one-row calls and the C oracle's sequential fmaf
// loop gives the same bits.

#include "tn_common.h"

namespace tn {
namespace {

constexpr int DL_TM = 64;   // rows of x per workgroup
constexpr int DL_TN = 64;   // output features per workgroup
constexpr int DL_TK = 16;   // k per LDS stage
constexpr int DL_LD = 68;   // LDS row stride in floats (float4-aligned, staggers the banks)

// half's to_f32 (the reference's widening): exact, and a NaN comes back with
// its payload and the quiet bit set (0x7fc00000 | sign | payload << 13 for
// f16, (h | 0x40) << 16 for bf16).
template <int WT>
__device__ inline float widen_w(const void* w, int64_t i) {
    if constexpr (WT == TN_F32) {
        return reinterpret_cast<const float*>(w)[i];
    } else if constexpr (WT == TN_F16) {
        const uint16_t h = reinterpret_cast<const uint16_t*>(w)[i];
        const float f = f16_bits_hw(h);
        if (f == f) return f;
        return __builtin_bit_cast(float, ((uint32_t)(h & 0x8000u) << 16) | 0x7fc00000u | ((uint32_t)(h & 0x3ffu) << 13));
    } else {
        const uint16_t h = reinterpret_cast<const uint16_t*>(w)[i];
        return bf16_to_f32((h & 0x7fffu) > 0x7f80u ? (uint16_t)(h | 0x40u) : h);
    }
}

// y[m, n] = (sequential fma chain over k of x[m, k] * w[n, k]) (+ bias[n]).
// 256 threads; thread (tx, ty) = (t % 16, t / 16) owns rows ty*4..ty*4+3 and
// features tx*4..tx*4+3 of the 64 x 64 tile. Stage s holds x[:, 16s..16s+15]
// and w[:, 16s..16s+15] k-major in LDS; only k < K is ever accumulated.
template <int WT>
__global__ void __launch_bounds__(256) k_dense_linear(const float* __restrict__ x, int M, int K,
                                                      const void* __restrict__ w, int N,
                                                      const float* __restrict__ bias, float* __restrict__ y) {
    __shared__ __align__(16) float xs[DL_TK][DL_LD];
    __shared__ __align__(16) float ws[DL_TK][DL_LD];
    const int t = threadIdx.x;
    const int tx = t % 16, ty = t / 16;
    const int n0 = blockIdx.x * DL_TN, m0 = blockIdx.y * DL_TM;
    const int lk = t % DL_TK, lr = t / DL_TK;  // loader: k column, first row (rows lr + 16i)
    float acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = 0.0f;
    for (int k0 = 0; k0 < K; k0 += DL_TK) {
        const int kk = k0 + lk;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = lr + 16 * i;
            const int m = m0 + r, n = n0 + r;
            xs[lk][r] = (m < M && kk < K) ? x[(int64_t)m * K + kk] : 0.0f;
            ws[lk][r] = (n < N && kk < K) ? widen_w<WT>(w, (int64_t)n * K + kk) : 0.0f;
        }
        __syncthreads();
        const int kend = min(DL_TK, K - k0);  // the same for every thread
        for (int k = 0; k < kend; ++k) {
            const float4 a = *reinterpret_cast<const float4*>(&xs[k][ty * 4]);
            const float4 b = *reinterpret_cast<const float4*>(&ws[k][tx * 4]);
            const float av[4] = {a.x, a.y, a.z, a.w}, bv[4] = {b.x, b.y, b.z, b.w};
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_fmaf(av[i], bv[j], acc[i][j]);
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int m = m0 + ty * 4 + i;
        if (m >= M) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int n = n0 + tx * 4 + j;
            if (n < N) y[(int64_t)m * N + n] = bias ? acc[i][j] + bias[n] : acc[i][j];
        }
    }
}

template <int WT>
__global__ void k_dense_store(const float* __restrict__ x, int64_t count, void* __restrict__ out) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < count; i += (int64_t)gridDim.x * blockDim.x) {
        if constexpr (WT == TN_F32) reinterpret_cast<float*>(out)[i] = x[i];
        else if constexpr (WT == TN_F16) reinterpret_cast<uint16_t*>(out)[i] = f16_from_f32(x[i]);
        else reinterpret_cast<uint16_t*>(out)[i] = bf16_from_f32(x[i]);
    }
}

template <int WT>
__global__ void k_dense_widen(const void* __restrict__ w, int64_t count, float* __restrict__ out) {
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < count; i += (int64_t)gridDim.x * blockDim.x)
        out[i] = widen_w<WT>(w, i);
}

tn_status dense_dtype(const char* op, int dtype) {
    if (dtype == TN_F32 || dtype == TN_F16 || dtype == TN_BF16) return TN_OK;
    return fail(TN_ENOTIMPL, std::string(op) + ": the dense formats are f32, f16 and bf16 (dtype code " +
                                 std::to_string(dtype) + " is none of them)");
}

unsigned stride_grid(int64_t count) { return (unsigned)std::min<int64_t>(cdiv(count, 256), 8192); }

}  // namespace
}  // namespace tn

using namespace tn;

extern "C" {

tn_status tn_dense_quantize(void* stream, const float* x, int64_t count, int dtype, void* out) {
    const char* op = "torch._C._quantize";
    TN_TRY(dense_dtype(op, dtype));
    if (count < 0) return fail(TN_EINVAL, std::string(op) + ": negative element count");
    if (count == 0) return TN_OK;
    if (!x || !out) return fail(TN_EVALUE, std::string(op) + ": null pointer");
    hipStream_t st = (hipStream_t)stream;
    if (dtype == TN_F32) hipLaunchKernelGGL(k_dense_store<TN_F32>, dim3(stride_grid(count)), dim3(256), 0, st, x, count, out);
    else if (dtype == TN_F16) hipLaunchKernelGGL(k_dense_store<TN_F16>, dim3(stride_grid(count)), dim3(256), 0, st, x, count, out);
    else hipLaunchKernelGGL(k_dense_store<TN_BF16>, dim3(stride_grid(count)), dim3(256), 0, st, x, count, out);
    TN_LAUNCHED();
    return TN_OK;
}

tn_status tn_dense_dequantize(void* stream, const void* w, int dtype, int64_t count, float* out) {
    const char* op = "torch._C._dequantize";
    TN_TRY(dense_dtype(op, dtype));
    if (count < 0) return fail(TN_EINVAL, std::string(op) + ": negative element count");
    if (count == 0) return TN_OK;
    if (!w || !out) return fail(TN_EVALUE, std::string(op) + ": null pointer");
    hipStream_t st = (hipStream_t)stream;
    if (dtype == TN_F32) hipLaunchKernelGGL(k_dense_widen<TN_F32>, dim3(stride_grid(count)), dim3(256), 0, st, w, count, out);
    else if (dtype == TN_F16) hipLaunchKernelGGL(k_dense_widen<TN_F16>, dim3(stride_grid(count)), dim3(256), 0, st, w, count, out);
    else hipLaunchKernelGGL(k_dense_widen<TN_BF16>, dim3(stride_grid(count)), dim3(256), 0, st, w, count, out);
    TN_LAUNCHED();
    return TN_OK;
}

tn_status tn_dense_linear(void* stream, const float* x, int64_t m, int64_t k, const void* w, int w_dtype,
                          int64_t n, const float* bias, float* y) {
    const char* op = "torch._C._quantized_linear";
    TN_TRY(dense_dtype(op, w_dtype));
    if (m < 0 || n < 0 || k < 1)
        return fail(TN_EINVAL, std::string(op) + ": mat1 and mat2 shapes cannot be multiplied ([" +
                                   std::to_string(m) + ", " + std::to_string(k) + "] and " + std::to_string(k) +
                                   "x" + std::to_string(n) + ")");
    if (m == 0 || n == 0) return TN_OK;
    if (!x || !w || !y) return fail(TN_EVALUE, std::string(op) + ": null pointer");
    if (m > INT32_MAX || n > INT32_MAX || k > INT32_MAX || cdiv(m, DL_TM) > 65535)
        return fail(TN_EVALUE, std::string(op) + ": shape too large");
    dim3 grid((unsigned)cdiv(n, DL_TN), (unsigned)cdiv(m, DL_TM));
    hipStream_t st = (hipStream_t)stream;
    if (w_dtype == TN_F32)
        hipLaunchKernelGGL(k_dense_linear<TN_F32>, grid, dim3(256), 0, st, x, (int)m, (int)k, w, (int)n, bias, y);
    else if (w_dtype == TN_F16)
        hipLaunchKernelGGL(k_dense_linear<TN_F16>, grid, dim3(256), 0, st, x, (int)m, (int)k, w, (int)n, bias, y);
    else
        hipLaunchKernelGGL(k_dense_linear<TN_BF16>, grid, dim3(256), 0, st, x, (int)m, (int)k, w, (int)n, bias, y);
    TN_LAUNCHED();
    return TN_OK;
}

}  // extern "C"
