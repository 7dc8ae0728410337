// gemv_w4.h — dequant-fused INT4 GEMV for M <= 16 (the decode path).
//
// Work mapping (wave64-first):
//   * A workgroup is 4 waves. Each wave owns R = 64/G consecutive output rows
//     n; the G lanes of a row split that row's K into 32-code chunks (one
//     16-byte load each) taken round-robin, so one wave-wide load reads R
//     contiguous segments of G*16 bytes of packed B in the reference layout
//     B[n][K/2] (G >= 8 makes every segment a whole 128-byte line).
//   * The activation slice A[0..M)[panel] is staged once per workgroup in LDS
//     (a chunk is 32 floats padded to 36 so the G distinct chunk addresses of
//     one wave-wide read fall on different banks); lanes with the same chunk
//     index read the same address (broadcast).
//   * Per chunk: one dwordx4 load of codes, one scale, one zero-point nibble;
//     32 exact dequants W = (q - zp) * s (nbits_device.h), then M fp32 FMAs
//     per dequantized weight. The dequant is shared by all M rows.
//   * End: the G partial sums of a row are combined with a butterfly over the
//     G lanes (fixed order: deterministic), lane 0 of the row stores Y.
// HBM traffic is the algorithmic minimum: every byte of B, scales and zero
// points is read once; A is read once per workgroup (L2-resident).
#pragma once
#include "nbits_device.h"

namespace msnb {

struct GemvParams {
    const uint8_t* b;        // [N][row_bytes] packed codes (reference layout)
    const float* scales;     // [N][nb]
    const uint8_t* zp;       // [N][zrb] packed nibbles, or nullptr (zp = 8)
    const float* a;          // [M][K]
    float* y;                // [M][N]
    int64_t row_bytes;       // nb * block_size / 2
    int N, K;
    int C;                   // K / 32 chunks per row
    int log2cpb;             // log2(block_size / 32)
    int nb, zrb;
    int panel_chunks;        // chunks of A staged per LDS panel
};

constexpr int kGemvThreads = 256;
constexpr int kChunkStride4 = 9;   // float4 per staged chunk (8 + 1 pad)

template <int M, int G>
__global__ __launch_bounds__(kGemvThreads) void gemv_w4_kernel(GemvParams p)
{
    constexpr int R = kWave / G;   // rows per wave
    constexpr int U = 4;           // chunks per lane in flight
    extern __shared__ float4 lds_a4[];   // [M][panel_chunks][kChunkStride4]

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int g = lane % G;
    const int r = lane / G;
    const int n = (blockIdx.x * (kGemvThreads / kWave) + wave) * R + r;
    const bool row_ok = n < p.N;
    const int nl = row_ok ? n : p.N - 1;   // clamped row for loads

    const uint8_t* brow = p.b + (int64_t)nl * p.row_bytes;
    const float* srow = p.scales + (int64_t)nl * p.nb;
    const uint8_t* zrow = p.zp ? p.zp + (int64_t)nl * p.zrb : nullptr;

    float acc[M];
#pragma unroll
    for (int m = 0; m < M; ++m) acc[m] = 0.0f;

    const int P = p.panel_chunks;
    for (int c0 = 0; c0 < p.C; c0 += P) {
        const int pc = min(P, p.C - c0);
        // ---- stage A[:, c0*32 .. (c0+pc)*32) into LDS --------------------------------
        __syncthreads();
        const int per_row = pc * 8;   // float4 per A row in this panel
        for (int idx = threadIdx.x; idx < M * per_row; idx += kGemvThreads) {
            const int m = idx / per_row;
            const int rem = idx - m * per_row;
            const int cc = rem >> 3;
            const int q4 = rem & 7;
            const float4 v = *reinterpret_cast<const float4*>(
                p.a + (int64_t)m * p.K + (int64_t)(c0 + cc) * 32 + q4 * 4);
            lds_a4[(m * P + cc) * kChunkStride4 + q4] = v;
        }
        __syncthreads();

        // ---- stream this row's chunks of the panel, U at a time ------------------------
        for (int base = 0; base < pc; base += G * U) {
            uint4 q[U];
            float s[U];
            int z[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int cc = base + u * G + g;
                const int c = c0 + (cc < pc ? cc : 0);
                const int blk = c >> p.log2cpb;
                q[u] = *reinterpret_cast<const uint4*>(brow + (int64_t)c * 16);
                s[u] = srow[blk];
                z[u] = zrow ? zp_nibble(zrow, blk) : 8;
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int cc = base + u * G + g;
                if (cc < pc) {
                    const BlockDq dq = block_dq(z[u], s[u]);
                    const uint32_t qd[4] = {q[u].x, q[u].y, q[u].z, q[u].w};
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        float w[8];
                        dequant8(qd[j], dq, w);
#pragma unroll
                        for (int m = 0; m < M; ++m) {
                            const float4 a0 = lds_a4[(m * P + cc) * kChunkStride4 + 2 * j];
                            const float4 a1 = lds_a4[(m * P + cc) * kChunkStride4 + 2 * j + 1];
                            acc[m] = __builtin_fmaf(a0.x, w[0], acc[m]);
                            acc[m] = __builtin_fmaf(a0.y, w[1], acc[m]);
                            acc[m] = __builtin_fmaf(a0.z, w[2], acc[m]);
                            acc[m] = __builtin_fmaf(a0.w, w[3], acc[m]);
                            acc[m] = __builtin_fmaf(a1.x, w[4], acc[m]);
                            acc[m] = __builtin_fmaf(a1.y, w[5], acc[m]);
                            acc[m] = __builtin_fmaf(a1.z, w[6], acc[m]);
                            acc[m] = __builtin_fmaf(a1.w, w[7], acc[m]);
                        }
                    }
                }
            }
        }
    }

    // ---- combine the G lanes of each row (butterfly, fixed order) ----------------------
#pragma unroll
    for (int off = G / 2; off > 0; off >>= 1) {
#pragma unroll
        for (int m = 0; m < M; ++m) acc[m] += __shfl_xor(acc[m], off, kWave);
    }
    if (g == 0 && row_ok) {
#pragma unroll
        for (int m = 0; m < M; ++m) p.y[(int64_t)m * p.N + n] = acc[m];
    }
}

}  // namespace msnb
