// mfma_w4.h — INT4 MatMulNBits GEMM on the CDNA4 matrix cores (M > 16, the
// prefill path).
//
// Y[M,N] = A[M,K] * W[N,K]^T with W dequantized in-kernel:
//   * A workgroup owns a BM x BN tile of Y (4 waves stacked along M, each wave
//     WM x BN) and walks K in steps of 32 codes (one 16-byte chunk per row).
//   * Producer: every thread loads 8 bytes (16 codes) of one weight row, its
//     block scale and zero-point nibble, dequantizes them exactly in fp32
//     (W = (q - zp) * s, nbits_device.h) and rounds each weight to fp16 into a
//     double-buffered LDS tile Bs[BN][32 (+pad)] — one barrier per K step.
//   * Consumer: each wave reads its A rows straight from global memory in the
//     MFMA operand layout (8 consecutive k per lane), rounds them to fp16 in
//     registers, and issues v_mfma_f32_32x32x16_f16 against the LDS weight
//     fragments; accumulation is fp32 in the matrix-core accumulators.
// Numerics: A and W each carry one fp16 rounding (relative 2^-11); products
// and sums are fp32.
#pragma once
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
};

constexpr int kMfmaThreads = 256;
constexpr int kMfmaWM = 32;                 // rows of Y per wave
constexpr int kMfmaBM = 4 * kMfmaWM;        // rows of Y per workgroup
constexpr int kMfmaBN = 128;                // columns of Y per workgroup
constexpr int kMfmaNF = kMfmaBN / 32;       // 32-wide column fragments per wave
constexpr int kBsStride = 40;               // fp16 per LDS weight row (32 + 8 pad)

__global__ __launch_bounds__(kMfmaThreads, 2) void mfma_w4_kernel(MfmaParams p)
{
    __shared__ __attribute__((aligned(16))) _Float16 Bs[2][kMfmaBN][kBsStride];

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    const int n0 = blockIdx.x * kMfmaBN;
    const int m0 = blockIdx.y * kMfmaBM;

    // ---- producer mapping: 2 threads per weight row, 16 codes each ------------------
    const int pn = tid >> 1;
    const int ph = tid & 1;
    const int prow = min(n0 + pn, p.N - 1);
    const uint8_t* pb = p.b + (int64_t)prow * p.row_bytes + ph * 8;
    const float* ps = p.scales + (int64_t)prow * p.nb;
    const uint8_t* pz = p.zp ? p.zp + (int64_t)prow * p.zrb : nullptr;

    // ---- consumer mapping: lane -> A row, 8-k slot ----------------------------------
    const int am = m0 + wave * kMfmaWM + (lane & 31);
    const float* pa = p.a + (int64_t)min(am, p.M - 1) * p.K + 8 * (lane >> 5);

    floatx16_t acc[kMfmaNF];
#pragma unroll
    for (int j = 0; j < kMfmaNF; ++j) acc[j] = floatx16_t{};

    auto load_b = [&](int t, uint2& q, float& s, int& z) {
        q = *reinterpret_cast<const uint2*>(pb + (int64_t)t * 16);
        const int blk = t >> p.log2cpb;
        s = ps[blk];
        z = pz ? zp_nibble(pz, blk) : 8;
    };
    auto store_b = [&](int buf, const uint2& q, float s, int z) {
        const BlockDq dq = block_dq(z, s);
        float w0[8], w1[8];
        dequant8(q.x, dq, w0);
        dequant8(q.y, dq, w1);
        half8_t h0, h1;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            h0[e] = (_Float16)w0[e];
            h1[e] = (_Float16)w1[e];
        }
        *reinterpret_cast<half8_t*>(&Bs[buf][pn][ph * 16]) = h0;
        *reinterpret_cast<half8_t*>(&Bs[buf][pn][ph * 16 + 8]) = h1;
    };
    auto load_a = [&](int t, float4 (&f)[4]) {
        const float* src = pa + (int64_t)t * 32;
        f[0] = *reinterpret_cast<const float4*>(src);
        f[1] = *reinterpret_cast<const float4*>(src + 4);
        f[2] = *reinterpret_cast<const float4*>(src + 16);
        f[3] = *reinterpret_cast<const float4*>(src + 20);
    };

    uint2 qn;
    float sn;
    int zn;
    float4 fa[4];
    load_b(0, qn, sn, zn);
    load_a(0, fa);
    store_b(0, qn, sn, zn);
    __syncthreads();

    for (int t = 0; t < p.C; ++t) {
        const int buf = t & 1;
        const bool more = t + 1 < p.C;
        if (more) load_b(t + 1, qn, sn, zn);

        half8_t a0, a1;
        a0[0] = (_Float16)fa[0].x; a0[1] = (_Float16)fa[0].y; a0[2] = (_Float16)fa[0].z; a0[3] = (_Float16)fa[0].w;
        a0[4] = (_Float16)fa[1].x; a0[5] = (_Float16)fa[1].y; a0[6] = (_Float16)fa[1].z; a0[7] = (_Float16)fa[1].w;
        a1[0] = (_Float16)fa[2].x; a1[1] = (_Float16)fa[2].y; a1[2] = (_Float16)fa[2].z; a1[3] = (_Float16)fa[2].w;
        a1[4] = (_Float16)fa[3].x; a1[5] = (_Float16)fa[3].y; a1[6] = (_Float16)fa[3].z; a1[7] = (_Float16)fa[3].w;
        if (more) load_a(t + 1, fa);

#pragma unroll
        for (int j = 0; j < kMfmaNF; ++j) {
            const _Float16* brow = &Bs[buf][32 * j + (lane & 31)][8 * (lane >> 5)];
            const half8_t b0 = *reinterpret_cast<const half8_t*>(brow);
            const half8_t b1 = *reinterpret_cast<const half8_t*>(brow + 16);
            acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, b0, acc[j], 0, 0, 0);
            acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, b1, acc[j], 0, 0, 0);
        }

        if (more) store_b(buf ^ 1, qn, sn, zn);
        __syncthreads();
    }

    // ---- epilogue: acc[j][v] is Y[row][col] with col = lane % 32 and
    //      row = 8*(v/4) + 4*(lane/32) + v%4 within the wave's 32x32 fragment j.
    const int mrow0 = m0 + wave * kMfmaWM + 4 * (lane >> 5);
#pragma unroll
    for (int j = 0; j < kMfmaNF; ++j) {
        const int col = n0 + 32 * j + (lane & 31);
        if (col < p.N) {
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int row = mrow0 + 8 * (v >> 2) + (v & 3);
                if (row < p.M) p.y[(int64_t)row * p.N + col] = acc[j][v];
            }
        }
    }
}

inline void mfma_launch_shape(int N, int M, int* grid, int* block)
{
    const int gx = (N + kMfmaBN - 1) / kMfmaBN;
    const int gy = (M + kMfmaBM - 1) / kMfmaBM;
    *grid = gx * gy;
    *block = kMfmaThreads;
}

// Returns 0 on a successful launch, nonzero otherwise (hipGetLastError holds the cause).
inline int launch_mfma(const uint8_t* b, const float* scales, const uint8_t* zp, int64_t row_bytes, int N, int K,
                       int nb, int zrb, int log2cpb, const float* a, float* y, int M, hipStream_t stream)
{
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
    const dim3 grid((N + kMfmaBN - 1) / kMfmaBN, (M + kMfmaBM - 1) / kMfmaBM);
    hipLaunchKernelGGL(mfma_w4_kernel, grid, dim3(kMfmaThreads), 0, stream, p);
    return hipPeekAtLastError() != hipSuccess;
}

}  // namespace msnb
