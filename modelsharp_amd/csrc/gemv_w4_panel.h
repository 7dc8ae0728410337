// gemv_w4_panel.h — dequant-fused INT4 GEMV over LDS panels of A (the decode path
// for 5 <= M <= 16, for activation panels too large for one LDS pass, and for block
// sizes 64 and 256).
//
// Work mapping (wave64-first):
//   * A workgroup is 4 waves. Each wave owns R = 64/G consecutive output rows
//     n; the G lanes of a row split that row's K into 32-code chunks (one
//     16-byte load each) taken round-robin, so one wave-wide load reads R
//     contiguous segments of G*16 bytes of packed B in the reference layout
//     B[n][K/2]. Codes, scales and zero points are read with buffer loads
//     (32-bit offsets off one scalar resource each).
//   * The activation slice A[0..M)[panel] is staged once per workgroup in LDS:
//     a chunk is 32 activations, pre-scaled as below, in 8 float4 plus one float4 of
//     padding (so that the G distinct chunk addresses of one wave-wide read fall on
//     different banks). Lanes with the same chunk index read the same address.
//   * Weight loads are software-pipelined in two ping-pong batches of U chunks:
//     one batch is in flight while the other is reduced. The first batch is
//     issued before A is staged, so the two latencies overlap.
//   * End: the G partial sums of a row are combined with a butterfly over the
//     G lanes (fixed order: deterministic); lane 0 of the row stores Y.
// Arithmetic per chunk (32 codes q_k, zero point zp, scale s), as in gemv_w4.h:
//   the packed-half dequant leaves q_k - zp (even k) and 16 (q_k - zp) (odd k) exactly
//   in fp16, the activations are staged as a_k and a_k / 16, and one v_fma_mix_f32 per
//   code adds a_k (q_k - zp) exactly into an fp32 sum. Per row m,
//       blk = sum_k a_k (q_k - zp),   acc += s * blk,
//   the reference's dot product with the scale applied once per block, with no
//   cancelling terms. The differences (9 ops per 8 codes) are shared by the M rows;
//   each row costs one fma per code plus one per chunk.
// HBM traffic is the algorithmic minimum: every byte of B, scales and zero
// points is read once; A is read once per workgroup (L2-resident).
#pragma once
#include "nbits_device.h"

namespace msnb {

struct GemvPanelParams {
    const uint8_t* b;        // [N][row_bytes] packed codes (reference layout)
    const float* scales;     // [N][nb]
    const uint8_t* zp;       // [N][zrb] packed nibbles, or nullptr (zp = 8)
    const float* a;          // [M][K]
    float* y;                // [M][N]
    int row_bytes;           // nb * block_size / 2
    int N, K;
    int C;                   // K / 32 chunks per row
    int log2cpb;             // log2(block_size / 32)
    int nb, zrb;
    int panel_chunks;        // chunks of A staged per LDS panel
};

constexpr int kPanelThreads = 256;
constexpr int kPanelU = 4;          // chunks per lane per pipeline batch
struct PanelChunkBatch {
    u32x4_t q[kPanelU];
    float s[kPanelU];
    int z[kPanelU];    // zero-point byte (both nibbles); the block's nibble is picked at use
};

template <int M, int G>
__global__ __launch_bounds__(kPanelThreads) void gemv_w4_panel_kernel(GemvPanelParams p)
{
    constexpr int R = kWave / G;   // rows per wave
    constexpr int U = kPanelU;
    extern __shared__ float4 lds_a4[];   // [M][panel_chunks][kChunkStride4]

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int g = lane % G;
    const int r = lane / G;
    const int n = (blockIdx.x * (kPanelThreads / kWave) + wave) * R + r;
    const bool row_ok = n < p.N;
    const int nl = row_ok ? n : p.N - 1;   // clamped row for loads

    const __amdgpu_buffer_rsrc_t rb = buffer_rsrc(p.b, p.N * p.row_bytes);
    const __amdgpu_buffer_rsrc_t rsc = buffer_rsrc(p.scales, p.N * p.nb * 4);
    const __amdgpu_buffer_rsrc_t rz = buffer_rsrc(p.zp ? (const void*)p.zp : (const void*)p.scales,
                                                  p.zp ? p.N * p.zrb : 0);
    const int boff = nl * p.row_bytes;
    const int soff = nl * p.nb * 4;
    const int zoff = nl * p.zrb;

    float acc[M];
#pragma unroll
    for (int m = 0; m < M; ++m) acc[m] = 0.0f;

    const int P = p.panel_chunks;
    for (int c0 = 0; c0 < p.C; c0 += P) {
        const int pc = min(P, p.C - c0);
        // ---- this lane's chunks of the panel: cc = g + G*k, k < nk -----------------------
        const int nk = g < pc ? (pc - g + G - 1) / G : 0;
        auto load = [&](PanelChunkBatch& bt, int k0) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int k = k0 + u;
                const int c = c0 + (k < nk ? g + G * k : 0);
                const int blk = c >> p.log2cpb;
                bt.q[u] = __builtin_amdgcn_raw_buffer_load_b128(rb, boff + c * 16, 0, 0);
                bt.s[u] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rsc, soff + blk * 4, 0, 0));
                bt.z[u] = p.zp ? (int)__builtin_amdgcn_raw_buffer_load_b8(rz, zoff + (blk >> 1), 0, 0) : 0x88;
            }
        };
        PanelChunkBatch b0, b1;
        load(b0, 0);

        // ---- stage A[:, c0*32 .. (c0+pc)*32): one thread per (row, chunk) ----------------
        __syncthreads();
        for (int idx = threadIdx.x; idx < M * pc; idx += kPanelThreads) {
            const int m = idx / pc;
            const int cc = idx - m * pc;
            const float4* src = reinterpret_cast<const float4*>(p.a + (int64_t)m * p.K + (int64_t)(c0 + cc) * 32);
            float4* dst = &lds_a4[(m * P + cc) * kChunkStride4];
#pragma unroll
            for (int j = 0; j < 8; ++j) dst[j] = stage_odd16(src[j]);
        }
        __syncthreads();

        auto reduce = [&](const PanelChunkBatch& bt, int k0) {
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (k0 + u < nk) {
                    const int cc = g + G * (k0 + u);
                    const int blk = (c0 + cc) >> p.log2cpb;
                    const uint32_t zp = ((uint32_t)bt.z[u] >> ((blk & 1) * 4)) & 0x0Fu;
                    const uint32_t qd[4] = {bt.q[u].x, bt.q[u].y, bt.q[u].z, bt.q[u].w};
                    uint32_t pr[4][4];
#pragma unroll
                    for (int j = 0; j < 4; ++j) diffs8(qd[j], zp_half2(zp), zp16_half2(zp), pr[j]);
#pragma unroll
                    for (int m = 0; m < M; ++m) {
                        const float4* arow = &lds_a4[(m * P + cc) * kChunkStride4];
                        float blkacc = 0.0f;
#pragma unroll
                        for (int j = 0; j < 4; ++j) blkacc = dot8(pr[j], arow[2 * j], arow[2 * j + 1], blkacc);
                        acc[m] = __builtin_fmaf(bt.s[u], blkacc, acc[m]);
                    }
                }
            }
        };
        for (int k0 = 0; k0 < nk; k0 += 2 * U) {
            if (k0 + U < nk) load(b1, k0 + U);
            reduce(b0, k0);
            if (k0 + U >= nk) break;
            if (k0 + 2 * U < nk) load(b0, k0 + 2 * U);
            reduce(b1, k0 + U);
        }
    }

    // ---- combine the G lanes of each row (DPP scan, fixed order; sum in lane G - 1) -----
#pragma unroll
    for (int m = 0; m < M; ++m) acc[m] = group_sum_to_last<G>(acc[m]);
    if (g == G - 1 && row_ok) {
#pragma unroll
        for (int m = 0; m < M; ++m) p.y[(int64_t)m * p.N + n] = acc[m];
    }
}

}  // namespace msnb
