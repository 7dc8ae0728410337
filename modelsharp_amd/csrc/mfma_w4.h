// mfma_w4.h — INT4 MatMulNBits GEMM on the CDNA4 matrix cores (M > 16, the
// prefill path).
//
// Y[M,N] = A[M,K] * W[N,K]^T with W dequantized in-kernel:
//   * A workgroup owns a (4*WM) x BN tile of Y: 4 waves stacked along M, each
//     wave WM x BN as (WM/32) x (BN/32) v_mfma_f32_32x32x16_f16 fragments with
//     fp32 accumulators. K advances 32 codes (one 16-byte chunk per weight
//     row) per step.
//   * Producer: the 256 threads dequantize the step's BN x 32 weight tile —
//     each thread 32*BN/256 codes of one row, exactly in fp32
//     (W = (q - zp) * s, nbits_device.h dequant8), rounded once to fp16 — into a
//     double-buffered LDS tile Bs[BN][32 (+8 pad)]: one barrier per step. The
//     next step's codes, scales and zero points are loaded before the current
//     step's MFMAs are issued.
//   * Consumer: each wave loads its A rows straight from global memory in the
//     MFMA operand layout (8 consecutive k per lane), one step ahead, and rounds
//     them to fp16 in registers; weight fragments come from LDS.
//   * Tile order is XCD-aware: workgroups are dealt round-robin to the 8 XCDs,
//     so tile t goes to XCD t % 8; tiles are numbered so that each XCD walks a
//     contiguous m-major range of tiles, and the CUs of one XCD share the same
//     A row panel in their L2.
// Numerics: A and W each carry one fp16 rounding (relative 2^-11); products
// are exact and sums fp32.
#pragma once
#include <cmath>

#include "nbits_device.h"

namespace msnb {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float floatx16_t __attribute__((ext_vector_type(16)));

struct MfmaParams {
    const uint8_t* b;
    const float* scales;
    const uint8_t* zp;
    const float* a;
    float* y;
    int64_t row_bytes;
    int M, N, K;
    int C;          // K / 32
    int log2cpb;
    int nb, zrb;
    int tiles_m, tiles_n;
};

constexpr int kMfmaThreads = 256;
constexpr int kBsStride = 40;   // fp16 per LDS weight row (32 + 8 pad)
constexpr int kXcds = 8;

// tile index of workgroup `bid` among tiles_m*tiles_n tiles (m-major), so that
// XCD x = bid % 8 owns the contiguous tile range [x*per, (x+1)*per).
__device__ __forceinline__ int xcd_tile(int bid, int tiles)
{
    const int per = (tiles + kXcds - 1) / kXcds;
    return (bid % kXcds) * per + bid / kXcds;
}

template <int WM, int BN>
__global__ __launch_bounds__(kMfmaThreads) void mfma_w4_kernel(MfmaParams p)
{
    constexpr int MF = WM / 32;               // 32-row fragments per wave
    constexpr int NF = BN / 32;               // 32-col fragments per wave
    constexpr int BM = 4 * WM;
    constexpr int CPT = 32 * BN / kMfmaThreads;   // codes per producer thread (8, 16 or 32)
    constexpr int TPR = 32 / CPT;                 // producer threads per weight row
    static_assert(CPT == 8 || CPT == 16 || CPT == 32, "BN must be 64, 128 or 256");
    __shared__ __attribute__((aligned(16))) _Float16 Bs[2][BN][kBsStride];

    const int tile = xcd_tile(blockIdx.x, p.tiles_m * p.tiles_n);
    if (tile >= p.tiles_m * p.tiles_n) return;
    const int m0 = (tile / p.tiles_n) * BM;
    const int n0 = (tile % p.tiles_n) * BN;

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;

    // ---- producer: row pn, codes [ph*CPT, ph*CPT + CPT) of each 32-code chunk --------
    const int pn = tid / TPR;
    const int ph = tid % TPR;
    const int prow = min(n0 + pn, p.N - 1);
    const uint8_t* pb = p.b + (int64_t)prow * p.row_bytes + ph * (CPT / 2);
    const float* ps = p.scales + (int64_t)prow * p.nb;
    const uint8_t* pz = p.zp ? p.zp + (int64_t)prow * p.zrb : nullptr;

    // ---- consumer: lane -> A row (l % 32) of each fragment, 8-k slot (l / 32) ----------
    const float* pa[MF];
#pragma unroll
    for (int i = 0; i < MF; ++i) {
        const int am = min(m0 + wave * WM + 32 * i + (lane & 31), p.M - 1);
        pa[i] = p.a + (int64_t)am * p.K + 8 * (lane >> 5);
    }

    floatx16_t acc[MF][NF];
#pragma unroll
    for (int i = 0; i < MF; ++i)
#pragma unroll
        for (int j = 0; j < NF; ++j) acc[i][j] = floatx16_t{};

    struct Codes {
        uint32_t q[CPT / 8];
        float s;
        int z;
    };
    auto load_b = [&](int t, Codes& c) {
        const uint8_t* src = pb + (int64_t)t * 16;
        if constexpr (CPT == 32) {
            const uint4 v = *reinterpret_cast<const uint4*>(src);
            c.q[0] = v.x; c.q[1] = v.y; c.q[2] = v.z; c.q[3] = v.w;
        } else if constexpr (CPT == 16) {
            const uint2 v = *reinterpret_cast<const uint2*>(src);
            c.q[0] = v.x; c.q[1] = v.y;
        } else {
            c.q[0] = *reinterpret_cast<const uint32_t*>(src);
        }
        const int blk = t >> p.log2cpb;
        c.s = ps[blk];
        c.z = pz ? zp_nibble(pz, blk) : 8;
    };
    auto store_b = [&](int buf, const Codes& c) {
        const BlockDq dq = block_dq(c.z, c.s);
#pragma unroll
        for (int w8 = 0; w8 < CPT / 8; ++w8) {
            float w[8];
            dequant8(c.q[w8], dq, w);
            half8_t h;
#pragma unroll
            for (int e = 0; e < 8; ++e) h[e] = (_Float16)w[e];
            *reinterpret_cast<half8_t*>(&Bs[buf][pn][ph * CPT + 8 * w8]) = h;
        }
    };
    // A for step t: fragment i, k-substep s -> 8 floats
    auto load_a = [&](int t, float4 (&f)[MF][4]) {
#pragma unroll
        for (int i = 0; i < MF; ++i) {
            const float* src = pa[i] + (int64_t)t * 32;
            f[i][0] = *reinterpret_cast<const float4*>(src);
            f[i][1] = *reinterpret_cast<const float4*>(src + 4);
            f[i][2] = *reinterpret_cast<const float4*>(src + 16);
            f[i][3] = *reinterpret_cast<const float4*>(src + 20);
        }
    };

    Codes cn;
    float4 fa[MF][4];
    load_b(0, cn);
    load_a(0, fa);
    store_b(0, cn);
    __syncthreads();

    for (int t = 0; t < p.C; ++t) {
        const int buf = t & 1;
        const bool more = t + 1 < p.C;
        if (more) load_b(t + 1, cn);

        half8_t ah[MF][2];
#pragma unroll
        for (int i = 0; i < MF; ++i) {
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                const float4 lo = fa[i][2 * s], hi = fa[i][2 * s + 1];
                ah[i][s] = half8_t{(_Float16)lo.x, (_Float16)lo.y, (_Float16)lo.z, (_Float16)lo.w,
                                   (_Float16)hi.x, (_Float16)hi.y, (_Float16)hi.z, (_Float16)hi.w};
            }
        }
        if (more) load_a(t + 1, fa);

#pragma unroll
        for (int j = 0; j < NF; ++j) {
            const _Float16* brow = &Bs[buf][32 * j + (lane & 31)][8 * (lane >> 5)];
            const half8_t b0 = *reinterpret_cast<const half8_t*>(brow);
            const half8_t b1 = *reinterpret_cast<const half8_t*>(brow + 16);
#pragma unroll
            for (int i = 0; i < MF; ++i) {
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i][0], b0, acc[i][j], 0, 0, 0);
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i][1], b1, acc[i][j], 0, 0, 0);
            }
        }

        if (more) store_b(buf ^ 1, cn);
        __syncthreads();
    }

    // ---- epilogue: acc[i][j][v] is Y[row][col], col = lane % 32 and
    //      row = 8*(v/4) + 4*(lane/32) + v%4 within fragment (i, j).
#pragma unroll
    for (int i = 0; i < MF; ++i) {
        const int mrow0 = m0 + wave * WM + 32 * i + 4 * (lane >> 5);
#pragma unroll
        for (int j = 0; j < NF; ++j) {
            const int col = n0 + 32 * j + (lane & 31);
            if (col < p.N) {
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int row = mrow0 + 8 * (v >> 2) + (v & 3);
                    if (row < p.M) p.y[(int64_t)row * p.N + col] = acc[i][j][v];
                }
            }
        }
    }
}

struct MfmaShape {
    int WM, BN;
    int tiles_m, tiles_n;
};

// Tile choice: the largest tile that still gives every CU work, else the tile
// with the best tiles-per-CU quantisation.
inline MfmaShape mfma_shape(int M, int N)
{
    const int cus = 256;
    const int cand[][2] = {{64, 128}, {32, 128}, {32, 64}};
    MfmaShape best{32, 64, 0, 0};
    double best_score = -1;
    for (const auto& c : cand) {
        const int tm = (M + 4 * c[0] - 1) / (4 * c[0]);
        const int tn = (N + c[1] - 1) / c[1];
        const int tiles = tm * tn;
        const double waves = (double)tiles / cus;
        const double quant = waves / std::ceil(waves);                // CU-level load balance
        const double size = (double)(4 * c[0] * c[1]) / (256.0 * 128.0);  // reuse per tile
        const double pad = (double)M * N / ((double)tm * 4 * c[0] * tn * c[1]);
        const double score = quant * pad * (0.6 + 0.4 * size);
        if (score > best_score + 1e-9) {
            best_score = score;
            best = MfmaShape{c[0], c[1], tm, tn};
        }
    }
    return best;
}

inline void mfma_launch_shape(int N, int M, int* grid, int* block)
{
    const MfmaShape s = mfma_shape(M, N);
    const int tiles = s.tiles_m * s.tiles_n;
    *grid = ((tiles + kXcds - 1) / kXcds) * kXcds;
    *block = kMfmaThreads;
}

// Returns 0 on a successful launch, nonzero otherwise (hipGetLastError holds the cause).
inline int launch_mfma(const uint8_t* b, const float* scales, const uint8_t* zp, int64_t row_bytes, int N, int K,
                       int nb, int zrb, int log2cpb, const float* a, float* y, int M, hipStream_t stream)
{
    const MfmaShape s = mfma_shape(M, N);
    MfmaParams p;
    p.b = b;
    p.scales = scales;
    p.zp = zp;
    p.a = a;
    p.y = y;
    p.row_bytes = row_bytes;
    p.M = M;
    p.N = N;
    p.K = K;
    p.C = K / 32;
    p.log2cpb = log2cpb;
    p.nb = nb;
    p.zrb = zrb;
    p.tiles_m = s.tiles_m;
    p.tiles_n = s.tiles_n;
    int grid = 0, block = 0;
    mfma_launch_shape(N, M, &grid, &block);
    if (s.WM == 64 && s.BN == 128)
        hipLaunchKernelGGL((mfma_w4_kernel<64, 128>), dim3(grid), dim3(kMfmaThreads), 0, stream, p);
    else if (s.WM == 32 && s.BN == 128)
        hipLaunchKernelGGL((mfma_w4_kernel<32, 128>), dim3(grid), dim3(kMfmaThreads), 0, stream, p);
    else
        hipLaunchKernelGGL((mfma_w4_kernel<32, 64>), dim3(grid), dim3(kMfmaThreads), 0, stream, p);
    return hipPeekAtLastError() != hipSuccess;
}

}  // namespace msnb
