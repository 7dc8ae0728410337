// gemv_w8.h — dequant-fused 8-bit GEMV for 1 <= M <= 4 (decode), packed or default zero
// points, block size a power of two >= 16, K a multiple of 16.
//
// Work mapping (as gemv_w4, with 16-code chunks): a workgroup of WAVES waves owns
// ROWS = (64/G) * (WAVES/KW) * RL consecutive rows n. Inside a wave G lanes share a row and
// 64/G rows sit side by side; KW waves split the same rows' K; a lane owns RL rows,
// ROWS0 apart. A step advances a lane by SPAN = G*KW chunks (one 16-byte code load per
// chunk and row), so one wave-wide load reads 64/G contiguous segments of G*16 bytes of
// the reference layout B[n][nb * bs].
// Load order: the activation panel first (into registers when it fits AV float4 per
// thread), then two batches of U steps of codes, scales and zero points, and only then
// the panel goes to LDS, so the staging waits for the activations while the weight
// stream is already in flight (loads return in issue order). Loads are unconditional: a
// lane with no chunk at a step loads from kOOB (zero, no memory request).
// LDS layout of the panel: float4 i (codes 4i..4i+3) of chunk c of row m sits at
// (m * 4 + i) * C + c, so the G lanes of a row read consecutive 16-byte words.
// Arithmetic per chunk (16 codes q_k, zero point zp, scale s): v_perm places bytes 0, 2
// (resp. 1, 3) of a code dword under the fp16 exponent of 1024.0, reading 1024 + q; one
// packed subtract of 1024 + zp leaves q - zp exactly (|q - zp| <= 255). Each product
// a_k (q_k - zp) is formed and added inside one v_fma_mix_f32; per row of A,
//     blk = sum_k a_k (q_k - zp),   acc += s * blk,
// the dot product with the dequantized weights (q - zp) s in another order with no
// cancelling terms (error within eps * sum_k |a_k (q_k - zp) s| per term of the sum).
// End: the G partial sums of a row meet in a DPP scan, the KW wave partials in LDS
// (fixed orders: deterministic); one lane stores.
// HBM traffic: every byte of B, scales and zero points once; A once per workgroup (L2).
#pragma once
#include "nbits_device.h"

namespace msnb {

struct Gemv8Params {
    const uint8_t* b;        // [N][row_bytes] codes (reference layout, one byte per code)
    const float* scales;     // [N][nb]
    const uint8_t* zp;       // [N][zrb] zero points (one byte per block), or nullptr (128)
    const float* a;          // [M][K]
    float* y;                // [M][N]
    int N, K, C;             // C = K / 16 chunks per row
    int row_bytes, nb, zrb;
    int lcpb;                // log2(block size / 16)
};

// acc + a . (q - zp) over the 4 codes of one dword: d0 holds the differences of codes
// 0 and 2, d1 those of codes 1 and 3 (fp16 pairs).
__device__ __forceinline__ float dot4_w8(uint32_t d0, uint32_t d1, const float4& a, float acc)
{
    acc = fmac_lo(d0, a.x, acc);
    acc = fmac_lo(d1, a.y, acc);
    acc = fmac_hi(d0, a.z, acc);
    acc = fmac_hi(d1, a.w, acc);
    return acc;
}

constexpr uint32_t kExp1024Bytes = 0x64646464u;   // byte 0x64: the high byte of fp16 1024.0
constexpr uint32_t kSelEven = 0x04020400u;        // v_perm: (code 0, 0x64, code 2, 0x64)
constexpr uint32_t kSelOdd = 0x04030401u;         // v_perm: (code 1, 0x64, code 3, 0x64)

template <int M, int WAVES, int G, int KW, int U, int RL, int AV>
__global__ __launch_bounds__(WAVES * 64) void gemv_w8_kernel(Gemv8Params p)
{
    constexpr int NB = 2;
    constexpr int NT = WAVES * 64;
    constexpr int R = kWave / G;
    constexpr int WR = WAVES / KW;
    constexpr int ROWS0 = R * WR;
    constexpr int ROWS = RL * ROWS0;
    constexpr int SPAN = G * KW;
    static_assert(WR * KW == WAVES && SPAN >= 16, "KW divides the waves; a step covers >= 16 chunks");
    extern __shared__ float4 lds_a8[];   // [M][4][C]
    __shared__ float red[KW > 1 ? KW : 1][ROWS][M];

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1), wave = tid / kWave;
    const int g = lane % G, r = lane / G;
    const int wk = wave % KW, wr = wave / KW;
    const int rl = wr * R + r;
    const int n0 = blockIdx.x * ROWS + rl;
    bool vrow[RL];
#pragma unroll
    for (int j = 0; j < RL; ++j) vrow[j] = n0 + j * ROWS0 < p.N;
    const int C = p.C;
    const int nsteps = (C + SPAN - 1) / SPAN;
    const int lofs = wk * G + g;
    const int nvalid = lofs < C ? (C - lofs + SPAN - 1) / SPAN : 0;

    const __amdgpu_buffer_rsrc_t ra = buffer_rsrc(p.a, M * p.K * 4);
    const __amdgpu_buffer_rsrc_t rb = buffer_rsrc(p.b, p.N * p.row_bytes);
    const __amdgpu_buffer_rsrc_t rsc = buffer_rsrc(p.scales, p.N * p.nb * 4);
    const __amdgpu_buffer_rsrc_t rz =
        buffer_rsrc(p.zp ? (const void*)p.zp : (const void*)p.scales, p.zp ? p.N * p.zrb : 0);

    // ---- 1. activations: first in the load queue ------------------------------------
    const int na4 = M * C * 4;
    float4 av[AV > 0 ? AV : 1];
    if constexpr (AV > 0) {
#pragma unroll
        for (int j = 0; j < AV; ++j) {
            const int e = tid + NT * j;
            av[j] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(ra, e < na4 ? e * 16 : kOOB, 0, 0));
        }
    }
    __builtin_amdgcn_sched_barrier(0);

    // ---- 2. weight stream: NB batches of U steps in flight ----------------------------
    int bbase[RL], sbase[RL], zbase[RL];
#pragma unroll
    for (int j = 0; j < RL; ++j) {
        const int nl = vrow[j] ? n0 + j * ROWS0 : 0;
        bbase[j] = nl * p.row_bytes;
        sbase[j] = nl * p.nb * 4;
        zbase[j] = nl * p.zrb;
    }
    struct Batch {
        u32x4_t q[RL][U];
        float s[RL][U];
        uint8_t z[RL][U];
    };
    // Codes are read once per call: non-temporal, so they do not displace the
    // activations, scales and zero points (lines shared by several steps) in L2.
    auto load = [&](Batch& bt, int k0) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int k = k0 + u;
            const int c = lofs + k * SPAN;
            const int blk = c >> p.lcpb;
#pragma unroll
            for (int j = 0; j < RL; ++j) {
                const bool ok = k < nvalid && vrow[j];
                bt.q[j][u] = __builtin_amdgcn_raw_buffer_load_b128(rb, ok ? bbase[j] + c * 16 : kOOB, 0, kNonTemporal);
                bt.s[j][u] = __builtin_bit_cast(
                    float, __builtin_amdgcn_raw_buffer_load_b32(rsc, ok ? sbase[j] + blk * 4 : kOOB, 0, 0));
                bt.z[j][u] = __builtin_amdgcn_raw_buffer_load_b8(rz, ok ? zbase[j] + blk : kOOB, 0, 0);
            }
        }
    };
    Batch bt[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) load(bt[b], b * U);
    __builtin_amdgcn_sched_barrier(0);

    // ---- 3. stage A in LDS, chunk-transposed ------------------------------------------
    auto put = [&](int e, const float4& v) {
        const int m = e / (4 * C);
        const int rem = e - m * 4 * C;
        lds_a8[(m * 4 + (rem & 3)) * C + (rem >> 2)] = v;
    };
    if constexpr (AV > 0) {
#pragma unroll
        for (int j = 0; j < AV; ++j) {
            const int e = tid + NT * j;
            if (e < na4) put(e, av[j]);
        }
    } else {
        for (int e = tid; e < na4; e += NT)
            put(e, __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(ra, e * 16, 0, 0)));
    }
    __syncthreads();

    float acc[RL][M];
#pragma unroll
    for (int j = 0; j < RL; ++j) {
#pragma unroll
        for (int m = 0; m < M; ++m) acc[j][m] = 0.0f;
    }
    auto reduce = [&](const Batch& bt, int k0) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int k = k0 + u;
            if (k < nvalid) {
                const int c = lofs + k * SPAN;
                h2_t zb[RL];
#pragma unroll
                for (int j = 0; j < RL; ++j) zb[j] = zp_half2(p.zp ? (uint32_t)bt.z[j][u] : 128u);
                float t[RL][M][2];
#pragma unroll
                for (int j = 0; j < RL; ++j) {
#pragma unroll
                    for (int m = 0; m < M; ++m) t[j][m][0] = t[j][m][1] = 0.0f;
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    uint32_t d0[RL], d1[RL];
#pragma unroll
                    for (int j = 0; j < RL; ++j) {
                        const uint32_t qd = bt.q[j][u][i];
                        d0[j] = as_u32(as_h2(__builtin_amdgcn_perm(kExp1024Bytes, qd, kSelEven)) - zb[j]);
                        d1[j] = as_u32(as_h2(__builtin_amdgcn_perm(kExp1024Bytes, qd, kSelOdd)) - zb[j]);
                    }
#pragma unroll
                    for (int m = 0; m < M; ++m) {
                        const float4 a = lds_a8[(m * 4 + i) * C + c];
#pragma unroll
                        for (int j = 0; j < RL; ++j) t[j][m][i & 1] = dot4_w8(d0[j], d1[j], a, t[j][m][i & 1]);
                    }
                }
#pragma unroll
                for (int m = 0; m < M; ++m) {
#pragma unroll
                    for (int j = 0; j < RL; ++j)
                        acc[j][m] = __builtin_fmaf(bt.s[j][u], t[j][m][0] + t[j][m][1], acc[j][m]);
                }
            }
        }
    };
    // Leaving through goto keeps every path back to the loop head past a refill (a
    // `break` out of the inner loop alone makes the compiler drain all loads each turn).
    for (int k0 = 0;; k0 += NB * U) {
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            if (k0 + b * U >= nsteps) goto steps_done;
            reduce(bt[b], k0 + b * U);
            load(bt[b], k0 + (b + NB) * U);
        }
    }
steps_done:

    // ---- 4. combine: G lanes (DPP scan), then KW waves (LDS, in wave order) -----------
#pragma unroll
    for (int j = 0; j < RL; ++j) {
#pragma unroll
        for (int m = 0; m < M; ++m) acc[j][m] = group_sum_to_last<G>(acc[j][m]);
    }
    if constexpr (KW > 1) {
        if (g == G - 1) {
#pragma unroll
            for (int j = 0; j < RL; ++j) {
#pragma unroll
                for (int m = 0; m < M; ++m) red[wk][j * ROWS0 + rl][m] = acc[j][m];
            }
        }
        __syncthreads();
        if (wk == 0 && g == G - 1) {
#pragma unroll
            for (int j = 0; j < RL; ++j) {
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    float s = red[0][j * ROWS0 + rl][m];
#pragma unroll
                    for (int w = 1; w < KW; ++w) s += red[w][j * ROWS0 + rl][m];
                    acc[j][m] = s;
                }
            }
        }
    }
    if (wk == 0 && g == G - 1) {
#pragma unroll
        for (int j = 0; j < RL; ++j) {
            if (vrow[j]) {
#pragma unroll
                for (int m = 0; m < M; ++m) p.y[(int64_t)m * p.N + n0 + j * ROWS0] = acc[j][m];
            }
        }
    }
}

// Launch configurations of gemv_w8_kernel.
struct Gemv8Config {
    int waves, G, KW, U, RL;
};
constexpr Gemv8Config kGemv8Configs[] = {
    {8, 64, 1, 2, 1}, {8, 16, 2, 2, 2}, {4, 16, 1, 2, 2}, {16, 64, 1, 2, 1}, {8, 64, 1, 2, 2},
    {16, 16, 4, 2, 2}, {8, 32, 1, 2, 2}, {4, 64, 1, 2, 1}, {16, 32, 2, 2, 1},
};
constexpr int kNumGemv8Configs = sizeof(kGemv8Configs) / sizeof(kGemv8Configs[0]);
constexpr int gemv8_rows(const Gemv8Config& c) { return (kWave / c.G) * (c.waves / c.KW) * c.RL; }
// Activation panels of up to kGemv8Av float4 per thread (256 threads) go through registers first.
constexpr int kGemv8Av = 8;
constexpr int kGemv8MaxLds = 160 * 1024 - 1024;   // LDS for the panel (the rest: the KW partials)

}  // namespace msnb
