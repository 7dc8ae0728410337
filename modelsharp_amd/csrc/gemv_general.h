// gemv_general.h — decode GEMV (M <= 16) for the weight formats the 4-bit kernels do not
// take: bits = 8, float zero points, block sizes other than 32/64/128/256, K not a
// multiple of 32 (K and the block size multiples of 8).
//
// Each lane dequantizes its weights exactly as the reference does (W = fl(fl(q - zp) * s),
// generic_nbits.h: the same fp32 values bit for bit) and accumulates a * W in fp32 with
// explicit fma: the reference's sum in another order.
//
// Mapping: 16 lanes per weight row, 4 rows per wave, 16 rows per workgroup of 4 waves.
// Lane g of a row takes the 8-code groups g, g + 16, g + 32, ... of its row (8 codes lie
// in one quantization block when the block size is a multiple of 8): one 4-byte (bits 4)
// or 8-byte (bits 8) load of codes, the block's scale and zero point, and two 16-byte
// loads of activations per row of A (the rows of a workgroup read the same activations,
// served by L1). The 16 partial sums of a row meet in a DPP scan (fixed order).
#pragma once
#include "generic_nbits.h"

namespace msnb {

constexpr int kGenRowsPerWg = 16;

template <int M>
__global__ __launch_bounds__(256) void gemv_general_kernel(RawLayout L, const float* __restrict__ a,
                                                           float* __restrict__ y)
{
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int g = lane & 15, r = lane >> 4;
    const int n = blockIdx.x * kGenRowsPerWg + wave * 4 + r;
    const int64_t row_bytes = (int64_t)L.nb * L.blob;
    float acc[M];
#pragma unroll
    for (int m = 0; m < M; ++m) acc[m] = 0.0f;
    if (n < L.N) {
        const int groups = L.K >> 3;
        for (int t = g; t < groups; t += 16) {
            const int k0 = t << 3;
            const int bk = k0 / L.bs, i0 = k0 - bk * L.bs;
            const float s = L.scales[(int64_t)n * L.nb + bk];
            const float zp = block_zp(L, n, bk);
            const uint8_t* src = L.b + (int64_t)n * row_bytes + (int64_t)bk * L.blob;
            float w[8];
            if (L.bits == 4) {
                const uint32_t x = *reinterpret_cast<const uint32_t*>(src + (i0 >> 1));
#pragma unroll
                for (int i = 0; i < 8; ++i) w[i] = ((float)((x >> (4 * i)) & 0xFu) - zp) * s;
            } else {
                const uint2 x = *reinterpret_cast<const uint2*>(src + i0);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    w[i] = ((float)((x.x >> (8 * i)) & 0xFFu) - zp) * s;
                    w[i + 4] = ((float)((x.y >> (8 * i)) & 0xFFu) - zp) * s;
                }
            }
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const float4 a0 = *reinterpret_cast<const float4*>(a + (int64_t)m * L.K + k0);
                const float4 a1 = *reinterpret_cast<const float4*>(a + (int64_t)m * L.K + k0 + 4);
                float t0 = acc[m];
                t0 = __builtin_fmaf(a0.x, w[0], t0);
                t0 = __builtin_fmaf(a0.y, w[1], t0);
                t0 = __builtin_fmaf(a0.z, w[2], t0);
                t0 = __builtin_fmaf(a0.w, w[3], t0);
                t0 = __builtin_fmaf(a1.x, w[4], t0);
                t0 = __builtin_fmaf(a1.y, w[5], t0);
                t0 = __builtin_fmaf(a1.z, w[6], t0);
                t0 = __builtin_fmaf(a1.w, w[7], t0);
                acc[m] = t0;
            }
        }
    }
    // Every lane of the wave takes part in the scan (rows past N carry zeros).
#pragma unroll
    for (int m = 0; m < M; ++m) acc[m] = group_sum_to_last<16>(acc[m]);
    if (g == 15 && n < L.N) {
#pragma unroll
        for (int m = 0; m < M; ++m) y[(int64_t)m * L.N + n] = acc[m];
    }
}

}  // namespace msnb
