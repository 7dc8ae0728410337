// gemv_w4_m1.h — dequant-fused INT4 GEMV for a single activation row (M = 1,
// the token-by-token decode path).
//
// Work mapping:
//   * K is cut into KW slices of whole 32-code chunks. A wave owns one slice;
//     lane l of the wave owns the chunks slice_start + l + 64*i (i < T). The
//     activations of those chunks live in the lane's VGPRs for the wave's whole
//     life (loaded once from global memory, no LDS staging, no barrier).
//   * A wave streams YT weight rows per step: per row and owned chunk one
//     16-byte load (the 64 lanes read 1 KiB contiguous per row), plus the
//     block's scale and zero-point nibble; the next step's loads are issued
//     before the current step is reduced. Every activation register is reused
//     by the YT rows of a step.
//   * The YT partial sums of a step are combined across the 64 lanes with one
//     transposed butterfly (reduce_rows); with KW > 1 the KW slice totals of a
//     row meet in LDS and are added in slice order. Fixed orders throughout:
//     results are deterministic.
// Arithmetic per chunk (32 codes, zero point zp, scale s, activations a_k):
//   A code q placed in the low mantissa bits of an fp16 lane is the exact
//   subnormal q * 2^-24 (bits 0-3) or 16q * 2^-24 (bits 4-7). With the lane's
//   activations stored pre-multiplied by 2^24 (even k) and 2^20 (odd k) — exact,
//   powers of two — an fp32 fma of the widened lane (v_fma_mix_f32) adds
//   exactly a_k * q_k. Then
//       blk = sum_k a_k q_k - zp * sum_k a_k,   acc += s * blk,
//   which is sum_k a_k (q_k - zp) s, the row's dot product with the dequantized
//   weights W = (q - zp) s, summed per block. Cost: 13 VALU ops per 8 codes.
#pragma once
#include "nbits_device.h"

namespace msnb {

struct GemvM1Params {
    const uint8_t* b;
    const float* scales;
    const uint8_t* zp;       // nullptr: zp = 8
    const float* a;          // [K]
    float* y;                // [N]
    int64_t row_bytes;
    int N, K, C, log2cpb, nb, zrb;
    int kw;                  // K slices (waves per row stream)
    int rs;                  // row streams per workgroup
    int steps;               // row steps per wave
};

// sum_k a'_k * q_k * 2^-24 over the 8 codes of dword x (a' pre-scaled as above,
// a8[0..7] for k = 8j .. 8j+7).
__device__ __forceinline__ float qdot8(uint32_t x, const float* a8, float acc)
{
    const uint32_t x8 = x >> 8;
    const uint32_t p0 = x & 0x000F000Fu;    // k0, k4   (q * 2^-24)
    const uint32_t p1 = x & 0x00F000F0u;    // k1, k5   (16 q * 2^-24)
    const uint32_t p2 = x8 & 0x000F000Fu;   // k2, k6
    const uint32_t p3 = x8 & 0x00F000F0u;   // k3, k7
    acc = mix_lo_acc(p0, a8[0], acc);
    acc = mix_lo_acc(p1, a8[1], acc);
    acc = mix_lo_acc(p2, a8[2], acc);
    acc = mix_lo_acc(p3, a8[3], acc);
    acc = mix_hi_acc(p0, a8[4], acc);
    acc = mix_hi_acc(p1, a8[5], acc);
    acc = mix_hi_acc(p2, a8[6], acc);
    acc = mix_hi_acc(p3, a8[7], acc);
    return acc;
}

// v[y] summed over the 64 lanes. On return v[0] of lane l holds the total of
// row (l >> (6 - log2 YT)); halves are exchanged first so every butterfly step
// moves at most YT/2 values.
template <int YT>
__device__ __forceinline__ float reduce_rows(float (&v)[YT], int lane)
{
    int mask = 32;
#pragma unroll
    for (int cnt = YT; cnt > 1; cnt >>= 1, mask >>= 1) {
        const bool upper = (lane & mask) != 0;
#pragma unroll
        for (int i = 0; i < cnt / 2; ++i) {
            const float keep = upper ? v[i + cnt / 2] : v[i];
            const float send = upper ? v[i] : v[i + cnt / 2];
            v[i] = keep + __shfl_xor(send, mask, kWave);
        }
    }
    float s = v[0];
    for (; mask > 0; mask >>= 1) s += __shfl_xor(s, mask, kWave);
    return s;
}

template <int YT, int T>
__global__ __launch_bounds__(512) void gemv_w4_m1_kernel(GemvM1Params p)
{
    extern __shared__ float part[];   // [rs * steps * YT][kw] when kw > 1
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int slice = wave % p.kw;
    const int stream = wave / p.kw;
    const int cs0 = (int)((int64_t)slice * p.C / p.kw);
    const int cs1 = (int)((int64_t)(slice + 1) * p.C / p.kw);

    // ---- the lane's chunks and their activations (pre-scaled), once ------------------
    int cidx[T];
    bool cok[T];
    float av[T][32];
    float asum[T];
#pragma unroll
    for (int i = 0; i < T; ++i) {
        const int c = cs0 + lane + kWave * i;
        cok[i] = c < cs1;
        cidx[i] = cok[i] ? c : cs0;
        const float4* src = reinterpret_cast<const float4*>(p.a + (int64_t)cidx[i] * 32);
        float sum = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float4 f = src[j];
            sum += f.x;
            sum += f.y;
            sum += f.z;
            sum += f.w;
            // float4 j holds k = 4j .. 4j+3: even k scaled by 2^24, odd k
            // (codes in bits 4-7, read as 16 q) by 2^20
            av[i][4 * j + 0] = f.x * kTwo24;
            av[i][4 * j + 1] = f.y * kTwo20;
            av[i][4 * j + 2] = f.z * kTwo24;
            av[i][4 * j + 3] = f.w * kTwo20;
        }
        asum[i] = sum;
    }

    const int rows_per_step = p.rs * YT;
    const int row0 = blockIdx.x * rows_per_step * p.steps;

    struct Step {
        uint4 q[YT][T];
        float s[YT][T];
        int z[YT][T];
    };
    auto load = [&](Step& st, int t) {
#pragma unroll
        for (int y = 0; y < YT; ++y) {
            const int n = min(row0 + (t * p.rs + stream) * YT + y, p.N - 1);
            const uint8_t* brow = p.b + (int64_t)n * p.row_bytes;
#pragma unroll
            for (int i = 0; i < T; ++i) {
                const int blk = cidx[i] >> p.log2cpb;
                st.q[y][i] = *reinterpret_cast<const uint4*>(brow + (int64_t)cidx[i] * 16);
                st.s[y][i] = p.scales[(int64_t)n * p.nb + blk];
                st.z[y][i] = p.zp ? zp_nibble(p.zp + (int64_t)n * p.zrb, blk) : 8;
            }
        }
    };

    // One step: reduce the YT rows of `st` (step t) and store or park the totals.
    auto finish = [&](const Step& st, int t) {
        float acc[YT];
#pragma unroll
        for (int y = 0; y < YT; ++y) {
            acc[y] = 0.0f;
#pragma unroll
            for (int i = 0; i < T; ++i) {
                if (cok[i]) {
                    const uint32_t qd[4] = {st.q[y][i].x, st.q[y][i].y, st.q[y][i].z, st.q[y][i].w};
                    float blk = 0.0f;
#pragma unroll
                    for (int j = 0; j < 4; ++j) blk = qdot8(qd[j], &av[i][8 * j], blk);
                    blk = __builtin_fmaf(-(float)st.z[y][i], asum[i], blk);
                    acc[y] = __builtin_fmaf(st.s[y][i], blk, acc[y]);
                }
            }
        }
        const float tot = reduce_rows<YT>(acc, lane);
        const int yrow = lane / (kWave / YT);
        const int n = row0 + (t * p.rs + stream) * YT + yrow;
        if ((lane & (kWave / YT - 1)) == 0) {
            if (p.kw == 1) {
                if (n < p.N) p.y[n] = tot;
            } else {
                part[((t * p.rs + stream) * YT + yrow) * p.kw + slice] = tot;
            }
        }
    };

    // Two step buffers in ping-pong: step t+1 is in flight while step t is reduced.
    Step s0, s1;
    load(s0, 0);
    for (int t = 0; t < p.steps; t += 2) {
        if (t + 1 < p.steps) load(s1, t + 1);
        finish(s0, t);
        if (t + 1 >= p.steps) break;
        if (t + 2 < p.steps) load(s0, t + 2);
        finish(s1, t + 1);
    }

    if (p.kw > 1) {
        __syncthreads();
        const int rows = rows_per_step * p.steps;
        for (int r = threadIdx.x; r < rows; r += blockDim.x) {
            const int n = row0 + r;
            float s = 0.0f;
            for (int j = 0; j < p.kw; ++j) s += part[r * p.kw + j];
            if (n < p.N) p.y[n] = s;
        }
    }
}

}  // namespace msnb
