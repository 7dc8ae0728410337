// decoder_ops.h — the decoder-layer operators on either side of MatMulNBits, so that
// activations stay in HBM between projections:
//
//   rmsnorm_kernel       SimplifiedLayerNormalization
//                        (Cpu/Kernels/Llm/SimplifiedLayerNormalizationKernel.cs:24-64):
//                        inv = 1 / sqrt(sum(x^2) / norm + eps), y = (x * inv) * scale
//   skip_rmsnorm_kernel  SkipSimplifiedLayerNormalization
//                        (SkipSimplifiedLayerNormalizationKernel.cs:29-86):
//                        t = (input + skip) + bias, y = (t * inv) * gamma + beta, with t,
//                        inv and (optionally) t written out
//   silu_mul_kernel      the MLP gate of Llama-family exports, Sigmoid -> Mul -> Mul
//                        (Activations/SigmoidKernel.cs:13-22, the elementwise Mul):
//                        y = (g * (1 / (1 + exp(-g)))) * u
//   add_kernel           the elementwise Add of the residual stream
//   sigmoid_kernel,      the unfused Sigmoid and Mul nodes, y = 1 / (1 + exp(-x)) and
//   mul_kernel           y = a * b, for graphs the fusion does not match
//
// One workgroup per row for the norms (the row's sum of squares is one fixed-order tree
// over the workgroup's partial sums, so a row's result does not depend on the launch);
// grid-stride loops for the elementwise kernels. Every operation is rounded on its own
// (the library is built with -ffp-contract=off); sqrt and the divisions are IEEE.
#pragma once
#include "nbits_device.h"

namespace msnb {

constexpr int kNormThreads = 256;

// Sum over the workgroup in a fixed order: each wave's sum by a DPP scan (one VALU op per
// level, the sum in lane 63), then the four wave sums in index order. The closing barrier
// lets a caller reuse red.
__device__ __forceinline__ float block_sum256(float v, float* red)
{
    v = group_sum_to_last<64>(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 63) red[wave] = v;
    __syncthreads();
    const float s = ((red[0] + red[1]) + red[2]) + red[3];
    __syncthreads();
    return s;
}

// Rows of up to kNormRegs * 4 * kNormThreads floats (vec: norm % 4 == 0, every buffer
// 16-byte aligned)
// are held in registers between the two passes: every load of a row is issued before any
// store, which the compiler cannot arrange by itself when the output may alias an input.
constexpr int kNormRegs = 8;

__device__ __forceinline__ float4 f4add(float4 a, float4 b)
{
    return float4{a.x + b.x, a.y + b.y, a.z + b.z, a.w + b.w};
}

__device__ __forceinline__ float f4sq(float4 t, float ss)
{
    ss = ss + t.x * t.x;
    ss = ss + t.y * t.y;
    ss = ss + t.z * t.z;
    return ss + t.w * t.w;
}

__device__ __forceinline__ float4 f4norm(float4 t, float inv, float4 g)
{
    return float4{(t.x * inv) * g.x, (t.y * inv) * g.y, (t.z * inv) * g.z, (t.w * inv) * g.w};
}

// y may alias x (each element is read before it is written, by the same thread).
__global__ __launch_bounds__(kNormThreads) void rmsnorm_kernel(const float* x, const float* __restrict__ scale,
                                                               float* y, float* __restrict__ inv_std, int norm,
                                                               float eps, int vec)
{
    __shared__ float red[4];
    const int64_t off = (int64_t)blockIdx.x * norm;
    if (vec && (norm & 3) == 0 && norm <= 4 * kNormThreads * kNormRegs) {
        const int n4 = norm >> 2;
        const float4* x4 = reinterpret_cast<const float4*>(x + off);
        float4 t[kNormRegs];
        float ss = 0.0f;
        // the scale is loaded with x, before the reduction's barrier (one round trip to memory)
        float4 sc[kNormRegs];
#pragma unroll
        for (int u = 0; u < kNormRegs; ++u) {
            const int i = threadIdx.x + u * kNormThreads;
            t[u] = i < n4 ? x4[i] : float4{0.0f, 0.0f, 0.0f, 0.0f};
            sc[u] = i < n4 ? reinterpret_cast<const float4*>(scale)[i] : float4{0.0f, 0.0f, 0.0f, 0.0f};
        }
#pragma unroll
        for (int u = 0; u < kNormRegs; ++u) ss = f4sq(t[u], ss);
        const float inv = 1.0f / __builtin_sqrtf(block_sum256(ss, red) / (float)norm + eps);
        if (inv_std && threadIdx.x == 0) inv_std[blockIdx.x] = inv;
        float4* y4 = reinterpret_cast<float4*>(y + off);
#pragma unroll
        for (int u = 0; u < kNormRegs; ++u) {
            const int i = threadIdx.x + u * kNormThreads;
            if (i < n4) y4[i] = f4norm(t[u], inv, sc[u]);
        }
        return;
    }
    float ss = 0.0f;
    for (int i = threadIdx.x; i < norm; i += kNormThreads) {
        const float v = x[off + i];
        ss = ss + v * v;
    }
    const float sum_sq = block_sum256(ss, red);
    const float inv = 1.0f / __builtin_sqrtf(sum_sq / (float)norm + eps);
    if (inv_std && threadIdx.x == 0) inv_std[blockIdx.x] = inv;
    for (int i = threadIdx.x; i < norm; i += kNormThreads) y[off + i] = (x[off + i] * inv) * scale[i];
}

// out and sum_out may alias input or skip (the residual stream updated in place): every
// element is read and written by one thread, and the second pass reads t back from
// sum_out when it was written.
__global__ __launch_bounds__(kNormThreads) void skip_rmsnorm_kernel(
    const float* input, const float* skip, const float* __restrict__ gamma, const float* __restrict__ beta,
    const float* __restrict__ bias, float* out, float* sum_out, float* __restrict__ inv_std, int norm, float eps,
    int vec)
{
    __shared__ float red[4];
    const int64_t off = (int64_t)blockIdx.x * norm;
    if (vec && (norm & 3) == 0 && norm <= 4 * kNormThreads * kNormRegs) {
        const int n4 = norm >> 2;
        const float4* a4 = reinterpret_cast<const float4*>(input + off);
        const float4* b4 = reinterpret_cast<const float4*>(skip + off);
        float4 t[kNormRegs], gm[kNormRegs];
        float ss = 0.0f;
        // gamma is loaded with the inputs, before the reduction's barrier (one round trip)
#pragma unroll
        for (int u = 0; u < kNormRegs; ++u) {
            const int i = threadIdx.x + u * kNormThreads;
            t[u] = i < n4 ? f4add(a4[i], b4[i]) : float4{0.0f, 0.0f, 0.0f, 0.0f};
            if (bias && i < n4) t[u] = f4add(t[u], reinterpret_cast<const float4*>(bias)[i]);
            gm[u] = i < n4 ? reinterpret_cast<const float4*>(gamma)[i] : float4{0.0f, 0.0f, 0.0f, 0.0f};
        }
#pragma unroll
        for (int u = 0; u < kNormRegs; ++u) ss = f4sq(t[u], ss);
        if (sum_out) {
#pragma unroll
            for (int u = 0; u < kNormRegs; ++u) {
                const int i = threadIdx.x + u * kNormThreads;
                if (i < n4) reinterpret_cast<float4*>(sum_out + off)[i] = t[u];
            }
        }
        const float inv = 1.0f / __builtin_sqrtf(block_sum256(ss, red) / (float)norm + eps);
        if (inv_std && threadIdx.x == 0) inv_std[blockIdx.x] = inv;
#pragma unroll
        for (int u = 0; u < kNormRegs; ++u) {
            const int i = threadIdx.x + u * kNormThreads;
            if (i < n4) {
                float4 v = f4norm(t[u], inv, gm[u]);
                if (beta) v = f4add(v, reinterpret_cast<const float4*>(beta)[i]);
                reinterpret_cast<float4*>(out + off)[i] = v;
            }
        }
        return;
    }
    float ss = 0.0f;
    for (int i = threadIdx.x; i < norm; i += kNormThreads) {
        float t = input[off + i] + skip[off + i];
        if (bias) t = t + bias[i];
        if (sum_out) sum_out[off + i] = t;
        ss = ss + t * t;
    }
    const float sum_sq = block_sum256(ss, red);
    const float inv = 1.0f / __builtin_sqrtf(sum_sq / (float)norm + eps);
    if (inv_std && threadIdx.x == 0) inv_std[blockIdx.x] = inv;
    for (int i = threadIdx.x; i < norm; i += kNormThreads) {
        float t;
        if (sum_out) {
            t = sum_out[off + i];
        } else {   // recomputed: the same roundings
            t = input[off + i] + skip[off + i];
            if (bias) t = t + bias[i];
        }
        float v = (t * inv) * gamma[i];
        if (beta) v = v + beta[i];
        out[off + i] = v;
    }
}

// Elementwise: y may alias an input.
__global__ __launch_bounds__(256) void silu_mul_kernel(const float* g, const float* u, float* y, int64_t n)
{
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const float x = g[i];
        const float s = 1.0f / (1.0f + expf(-x));
        y[i] = (x * s) * u[i];
    }
}

__global__ __launch_bounds__(256) void add_kernel(const float* a, const float* b, float* y, int64_t n)
{
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        y[i] = a[i] + b[i];
}

__global__ __launch_bounds__(256) void sigmoid_kernel(const float* x, float* y, int64_t n)
{
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        y[i] = 1.0f / (1.0f + expf(-x[i]));
}

__global__ __launch_bounds__(256) void mul_kernel(const float* a, const float* b, float* y, int64_t n)
{
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        y[i] = a[i] * b[i];
}

}  // namespace msnb
