// mfma_w4.h — INT4 MatMulNBits GEMM on the CDNA4 matrix cores (M > 16), the general
// form: any power-of-two block size from 32 to 256, K a multiple of 32, any fp32 scales,
// no workspace. At fp32-level accuracy, like the small-M GEMV:
//   Y[m][n] = 2^e[m] * sum_b s[n][b] * sum_{k in b} (hi + lo)[m][k] * (q[n][k] - zp[n][b])
// with
//   * q - zp a small integer, exact in fp16 (packed-half dequant without the scale);
//   * A split per row into A = 2^e (hi + lo), hi = fp16(A 2^-e), lo = fp16(A 2^-e - hi),
//     e chosen so the row's max |A| 2^-e lies in [2^14, 2^15): every product
//     hi (q - zp), lo (q - zp) is exact in fp32, and hi + lo carries A to about 2^-22
//     of its row's max (no fp16 overflow for any finite A);
//   * the block sums (fp32, accumulated by the MFMAs) times s in fp32, added to the
//     running sum once per block; the row's 2^e at the end (exact).
// So no input range turns into inf or NaN that the fp32 reference would not produce:
// the library sends here the weights whose scales the fp16 kernels cannot carry, the
// block sizes and K they do not take, and calls that find no workspace.
//
// Work mapping:
//   * A workgroup owns a (4*WM) x BN tile of Y: 4 waves stacked along M, each wave
//     WM x BN as (WM/32) x (BN/32) v_mfma_f32_32x32x16_f16 fragments; K advances 32
//     codes (one 16-byte chunk per weight row) per step.
//   * Prologue: each wave reads its A rows once for their max |A| (lanes l and l + 32
//     share a row), and the exponents go to LDS for the epilogue.
//   * Producer: the 256 threads turn the step's BN x 32 codes into q - zp (fp16, exact)
//     in a double-buffered LDS tile, and the block's scales into an LDS row. The next
//     step's codes, scales and zero points are loaded before the current step's MFMAs.
//   * Consumer: each wave loads its A rows straight from global memory in the MFMA
//     operand layout (8 consecutive k per lane), one step ahead, and splits them into
//     hi / lo in registers; both operands carry the same permutation of each 8-k group
//     (k0,k4,k1,k5,k2,k6,k3,k7: the order in which one dword of codes dequantizes).
//   * Tile order is XCD-aware: workgroups are dealt round-robin to the 8 XCDs, so
//     tile t goes to XCD t % 8; tiles are numbered so that each XCD walks a contiguous
//     m-major range of tiles, and the CUs of one XCD share the same A row panel in L2.
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

// hi / lo halves of 8 activations times 2^-e, in the order k0,k4,k1,k5,k2,k6,k3,k7.
__device__ __forceinline__ void split8(const float4& x03, const float4& x47, int e, half8_t& hi, half8_t& lo)
{
    const float v[8] = {x03.x, x47.x, x03.y, x47.y, x03.z, x47.z, x03.w, x47.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float x = __builtin_amdgcn_ldexpf(v[i], -e);
        const _Float16 h = (_Float16)x;
        hi[i] = h;
        lo[i] = (_Float16)(x - (float)h);
    }
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
    __shared__ float Ss[2][BN];
    __shared__ int Es[BM];

    const int tile = xcd_tile(blockIdx.x, p.tiles_m * p.tiles_n);
    if (tile >= p.tiles_m * p.tiles_n) return;
    const int m0 = (tile / p.tiles_n) * BM;
    const int n0 = (tile % p.tiles_n) * BN;

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    const int cpb = 1 << p.log2cpb;           // steps per quantization block

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

    // ---- prologue: row exponents (lanes l and l + 32 read the two halves of each row) ---
    int ea[MF];
    {
        float mx[MF];
#pragma unroll
        for (int i = 0; i < MF; ++i) mx[i] = 0.0f;
        for (int t = 0; t < p.C; ++t) {
            float4 f[MF][4];
            load_a(t, f);
#pragma unroll
            for (int i = 0; i < MF; ++i) {
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    mx[i] = fmaxf(mx[i], fmaxf(fmaxf(fabsf(f[i][q].x), fabsf(f[i][q].y)),
                                               fmaxf(fabsf(f[i][q].z), fabsf(f[i][q].w))));
            }
        }
#pragma unroll
        for (int i = 0; i < MF; ++i) {
            const float m = fmaxf(mx[i], __shfl_xor(mx[i], 32));
            ea[i] = (m > 0.0f && m <= 3.402823466e38f) ? __builtin_amdgcn_frexp_expf(m) - 15 : 0;
            if (lane < 32) Es[wave * WM + 32 * i + lane] = ea[i];
        }
    }

    floatx16_t acc[MF][NF], blk[MF][NF];
#pragma unroll
    for (int i = 0; i < MF; ++i)
#pragma unroll
        for (int j = 0; j < NF; ++j) {
            acc[i][j] = floatx16_t{};
            blk[i][j] = floatx16_t{};
        }

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
        const int bk = t >> p.log2cpb;
        c.s = ps[bk];
        c.z = pz ? zp_nibble(pz, bk) : 8;
    };
    // q - zp for the producer's codes, exact in fp16, each dword in the order
    // (k0,k4),(k1,k5),(k2,k6),(k3,k7).
    auto store_b = [&](int buf, const Codes& c) {
        const h2_t zb = as_h2(kHalfMagic | ((uint32_t)c.z << 16) | (uint32_t)c.z);
#pragma unroll
        for (int w8 = 0; w8 < CPT / 8; ++w8) {
            const uint32_t x = c.q[w8];
            const u32x4_t d{as_u32(as_h2(and_or(x, 0x000F000Fu, kHalfMagic)) - zb),
                            as_u32(as_h2(and_or(x >> 4, 0x000F000Fu, kHalfMagic)) - zb),
                            as_u32(as_h2(and_or(x >> 8, 0x000F000Fu, kHalfMagic)) - zb),
                            as_u32(as_h2(and_or(x >> 12, 0x000F000Fu, kHalfMagic)) - zb)};
            *reinterpret_cast<u32x4_t*>(&Bs[buf][pn][ph * CPT + 8 * w8]) = d;
        }
        if (ph == 0) Ss[buf][pn] = c.s;
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

        half8_t ah[MF][2], al[MF][2];
#pragma unroll
        for (int i = 0; i < MF; ++i) {
#pragma unroll
            for (int s = 0; s < 2; ++s) split8(fa[i][2 * s], fa[i][2 * s + 1], ea[i], ah[i][s], al[i][s]);
        }
        if (more) load_a(t + 1, fa);

#pragma unroll
        for (int j = 0; j < NF; ++j) {
            const _Float16* brow = &Bs[buf][32 * j + (lane & 31)][8 * (lane >> 5)];
            const half8_t b0 = *reinterpret_cast<const half8_t*>(brow);
            const half8_t b1 = *reinterpret_cast<const half8_t*>(brow + 16);
#pragma unroll
            for (int i = 0; i < MF; ++i) {
                blk[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i][0], b0, blk[i][j], 0, 0, 0);
                blk[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[i][1], b1, blk[i][j], 0, 0, 0);
                blk[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[i][0], b0, blk[i][j], 0, 0, 0);
                blk[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[i][1], b1, blk[i][j], 0, 0, 0);
            }
        }
        // End of a quantization block (or of K, inside a partial last block): the block
        // sums times the scale of their column (lane % 32 of fragment j), into the
        // running sums.
        if (((t + 1) & (cpb - 1)) == 0 || !more) {
#pragma unroll
            for (int j = 0; j < NF; ++j) {
                const float sc = Ss[buf][32 * j + (lane & 31)];
#pragma unroll
                for (int i = 0; i < MF; ++i) {
#pragma unroll
                    for (int v = 0; v < 16; ++v) acc[i][j][v] = __builtin_fmaf(blk[i][j][v], sc, acc[i][j][v]);
                    blk[i][j] = floatx16_t{};
                }
            }
        }

        if (more) store_b(buf ^ 1, cn);
        __syncthreads();
    }

    // ---- epilogue: acc[i][j][v] is Y[row][col] / 2^Es[row], col = lane % 32 and
    //      row = 8*(v/4) + 4*(lane/32) + v%4 within fragment (i, j).
#pragma unroll
    for (int i = 0; i < MF; ++i) {
        const int r0 = wave * WM + 32 * i + 4 * (lane >> 5);
#pragma unroll
        for (int j = 0; j < NF; ++j) {
            const int col = n0 + 32 * j + (lane & 31);
            if (col < p.N) {
#pragma unroll
                for (int v = 0; v < 16; ++v) {
                    const int r = r0 + 8 * (v >> 2) + (v & 3);
                    const int row = m0 + r;
                    if (row < p.M) p.y[(int64_t)row * p.N + col] = __builtin_amdgcn_ldexpf(acc[i][j][v], Es[r]);
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
