// gemv_w4.h — dequant-fused INT4 GEMV for 1 <= M <= 4 (the decode path).
//
// Work mapping (wave64-first):
//   * A workgroup of WAVES waves owns ROWS = (64/G) * (WAVES/KW) consecutive output
//     rows n. Inside a wave, G lanes share a row and R = 64/G rows sit side by
//     side; KW waves split the same rows' K. A step advances each lane by
//     SPAN = G*KW chunks of 32 codes (one 16-byte load per chunk), so one
//     wave-wide code load reads R contiguous segments of G*16 bytes of packed B
//     in the reference layout B[n][K/2].
//   * The whole activation panel A[0..M)[0..K) is staged once per workgroup in
//     LDS (pre-scaled, plus per-chunk sums; kChunkStride4 float4 per chunk).
//   * Load order is the design: every vector-memory load returns in issue order,
//     so the activation loads go first, then two batches of U steps of codes,
//     scales and zero points, and only then is A written to LDS. The staging
//     therefore waits for the activations alone while the weight stream is
//     already in flight. Loads are unconditional (a lane with no chunk at a step
//     loads from kOOB: zero, no memory request), which keeps the compiler's
//     wait counts exact; sched_barrier keeps the scheduler from reordering the
//     three groups. Addresses are one per-lane base plus compile-time step
//     strides (L = log2 chunks per block is a template parameter).
//   * End: the G partial sums of a row meet in a butterfly over the G lanes,
//     the KW wave partials in LDS (fixed orders: deterministic); one lane stores.
// Arithmetic per chunk (32 codes q_k, zero point zp, scale s):
//   A code in the low mantissa bits of an fp16 lane is the exact subnormal
//   q * 2^-24 (code bits 0-3) or 16q * 2^-24 (bits 4-7). With the activations
//   staged times 2^24 (even k) and 2^20 (odd k) — exact powers of two — one
//   v_fma_mix_f32 adds exactly a_k * q_k. Per activation row m,
//       blk = sum_k a_k q_k - zp * sum_k a_k,   acc += s * blk,
//   i.e. sum_k a_k (q_k - zp) s: the dot product with the dequantized weights
//   W = (q - zp) s, folded per block. For M <= 2 the 32 products go into two
//   partial sums (shorter dependency chains).
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
    int row_bytes;           // nb * block_size / 2
    int N, K;
    int C;                   // K / 32 chunks per row
    int nb, zrb;
};

template <int M, int G, int KW, int U, int L, int WAVES>
__global__ __launch_bounds__(WAVES * 64) void gemv_w4_kernel(GemvParams p)
{
    constexpr int R = kWave / G;
    constexpr int WR = WAVES / KW;
    constexpr int ROWS = R * WR;
    constexpr int SPAN = G * KW;
    constexpr int BSPAN = SPAN >> L;   // blocks per step
    static_assert((BSPAN << L) == SPAN && (BSPAN & 1) == 0, "a step covers an even number of whole blocks");
    static_assert(WR * KW == WAVES, "KW must divide WAVES");
    extern __shared__ float4 lds_a4[];  // [M][C][kChunkStride4]
    __shared__ float red[KW > 1 ? KW : 1][ROWS][M];

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int g = lane % G, r = lane / G;
    const int wk = wave % KW, wr = wave / KW;
    const int rl = wr * R + r;
    const int n = blockIdx.x * ROWS + rl;
    const int C = p.C;
    const int nsteps = (C + SPAN - 1) / SPAN;
    const int lofs = wk * G + g;                       // chunk offset within a step
    const int nvalid = (lofs < C && n < p.N) ? (C - lofs + SPAN - 1) / SPAN : 0;

    const __amdgpu_buffer_rsrc_t ra = buffer_rsrc(p.a, M * p.K * 4);
    const __amdgpu_buffer_rsrc_t rb = buffer_rsrc(p.b, p.N * p.row_bytes);
    const __amdgpu_buffer_rsrc_t rsc = buffer_rsrc(p.scales, p.N * p.nb * 4);
    const __amdgpu_buffer_rsrc_t rz = buffer_rsrc(p.zp ? (const void*)p.zp : (const void*)p.scales,
                                                  p.zp ? p.N * p.zrb : 0);

    // ---- 1. activation chunks: first in the load queue -------------------------------
    const int na = M * C;
    const int idx = threadIdx.x;                      // M * C <= 64 * WAVES (checked by the host)
    const int am = idx / C, ac = idx - am * C;
    const int aoff = idx < na ? (am * p.K + ac * 32) * 4 : kOOB;
    float4 av[8];
#pragma unroll
    for (int j = 0; j < 8; ++j)
        av[j] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(ra, aoff + 16 * j, 0, 0));
    __builtin_amdgcn_sched_barrier(0);

    // ---- 2. weight stream: two batches of U steps in flight ---------------------------
    const int nl = n < p.N ? n : p.N - 1;
    const int bbase = nl * p.row_bytes + lofs * 16;
    const int sbase = nl * p.nb * 4 + (lofs >> L) * 4;
    const int zbase = nl * p.zrb + ((lofs >> L) >> 1);
    const int zshift = ((lofs >> L) & 1) * 4;
    struct Batch {
        u32x4_t q[U];
        float s[U];
        uint32_t z[U];
    };
    auto load = [&](Batch& bt, int k0) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int k = k0 + u;
            const bool ok = k < nvalid;
            bt.q[u] = __builtin_amdgcn_raw_buffer_load_b128(rb, ok ? bbase + k * (SPAN * 16) : kOOB, 0, 0);
            bt.s[u] = __builtin_bit_cast(
                float, __builtin_amdgcn_raw_buffer_load_b32(rsc, ok ? sbase + k * (BSPAN * 4) : kOOB, 0, 0));
            bt.z[u] = __builtin_amdgcn_raw_buffer_load_b8(rz, ok ? zbase + k * (BSPAN / 2) : kOOB, 0, 0);
        }
    };
    Batch bA, bB;
    load(bA, 0);
    load(bB, U);
    __builtin_amdgcn_sched_barrier(0);

    // ---- 3. stage A: pre-scaled activations and chunk sums ------------------------------
    if (idx < na) {
        float4* dst = &lds_a4[idx * kChunkStride4];
        float sum = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float4 v = av[j];
            sum += v.x;
            sum += v.y;
            sum += v.z;
            sum += v.w;
            dst[j] = float4{v.x * kTwo24, v.y * kTwo20, v.z * kTwo24, v.w * kTwo20};
        }
        dst[8] = float4{sum, 0.0f, 0.0f, 0.0f};
    }
    __syncthreads();

    float acc[M];
#pragma unroll
    for (int m = 0; m < M; ++m) acc[m] = 0.0f;
    auto reduce = [&](const Batch& bt, int k0) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int k = k0 + u;
            if (k < nvalid) {
                const int c = k * SPAN + lofs;
                const float zpf = p.zp ? (float)((bt.z[u] >> zshift) & 0x0F) : 8.0f;
                const uint32_t qd[4] = {bt.q[u].x, bt.q[u].y, bt.q[u].z, bt.q[u].w};
                uint32_t pr[4][4];
#pragma unroll
                for (int j = 0; j < 4; ++j) code_pairs(qd[j], pr[j]);
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    const float4* arow = &lds_a4[(m * C + c) * kChunkStride4];
                    float blkacc;
                    if constexpr (M <= 2) {
                        float t0 = qdot8(pr[0], arow[0], arow[1], 0.0f);
                        float t1 = qdot8(pr[1], arow[2], arow[3], 0.0f);
                        t0 = qdot8(pr[2], arow[4], arow[5], t0);
                        t1 = qdot8(pr[3], arow[6], arow[7], t1);
                        blkacc = t0 + t1;
                    } else {
                        blkacc = 0.0f;
#pragma unroll
                        for (int j = 0; j < 4; ++j) blkacc = qdot8(pr[j], arow[2 * j], arow[2 * j + 1], blkacc);
                    }
                    blkacc = __builtin_fmaf(-zpf, arow[8].x, blkacc);
                    acc[m] = __builtin_fmaf(bt.s[u], blkacc, acc[m]);
                }
            }
        }
    };
    for (int k0 = 0; k0 < nsteps; k0 += 2 * U) {
        reduce(bA, k0);
        load(bA, k0 + 2 * U);
        if (k0 + U >= nsteps) break;
        reduce(bB, k0 + U);
        load(bB, k0 + 3 * U);
    }

    // ---- 4. combine: G lanes (butterfly), then KW waves (LDS, in wave order) -----------
#pragma unroll
    for (int off = G / 2; off > 0; off >>= 1) {
#pragma unroll
        for (int m = 0; m < M; ++m) acc[m] += __shfl_xor(acc[m], off, kWave);
    }
    if constexpr (KW > 1) {
        if (g == 0) {
#pragma unroll
            for (int m = 0; m < M; ++m) red[wk][rl][m] = acc[m];
        }
        __syncthreads();
        if (wk == 0 && g == 0) {
#pragma unroll
            for (int m = 0; m < M; ++m) {
                float s = red[0][rl][m];
#pragma unroll
                for (int j = 1; j < KW; ++j) s += red[j][rl][m];
                acc[m] = s;
            }
        }
    }
    if (wk == 0 && g == 0 && n < p.N) {
#pragma unroll
        for (int m = 0; m < M; ++m) p.y[(int64_t)m * p.N + n] = acc[m];
    }
}

// Launch configurations of gemv_w4_kernel (one instantiation each per M and L).
struct GemvConfig {
    int waves, G, KW, U;
};
constexpr GemvConfig kGemvConfigs[] = {
    {4, 16, 1, 2},  {4, 16, 1, 4},  {4, 32, 1, 4},  {4, 64, 1, 2},  {4, 16, 4, 2},  {4, 32, 2, 2},
    {8, 32, 1, 4},  {8, 16, 2, 4},  {8, 16, 4, 2},  {16, 16, 4, 2}, {16, 32, 2, 2}, {16, 32, 4, 2},
};
constexpr int kNumGemvConfigs = sizeof(kGemvConfigs) / sizeof(kGemvConfigs[0]);
constexpr int kGemvMaxM = 4;

}  // namespace msnb
