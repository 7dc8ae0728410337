// generic_nbits.h — the operator's dequantization for every weight format, one weight
// at a time: the readback kernel, the per-output kernel the general paths fall back to
// (K or the block size not a multiple of 8), and the helpers of the general GEMV and
// GEMM kernels.
//
// All follow the reference's per-block loop directly (MatMulNBitsKernel.cs:236-258):
// block b of row n starts at byte n*nb*blob + b*blob, its zero point is the b-th float
// of row n's zero points (zpf, MatMulNBitsKernel.cs:239-240), the b-th packed code of
// row n (stride zrb bytes, :241) or 2^(bits-1) (:242), and the last block may be partial
// (len = min(bs, K - b*bs), :246). W = ((float)q - zp) * scale, each operation rounded
// in fp32 (MatMulNBitsSimd.cs:100-111): bit for bit the reference's weights.
#pragma once
#include "nbits_device.h"

namespace msnb {

struct RawLayout {
    const uint8_t* b;
    const float* scales;
    const uint8_t* zp;   // packed codes, or nullptr
    const float* zpf;    // float zero points [N * nb], or nullptr (then zp, else 2^(bits-1))
    int N, K, bits, bs, nb, blob, zrb;
};

__device__ __forceinline__ int unpack_code(const uint8_t* data, int64_t base, int index, int bits)
{
    if (bits == 8) return data[base + index];
    return (data[base + (index >> 1)] >> ((index & 1) * 4)) & 0x0F;
}

__device__ __forceinline__ float block_zp(const RawLayout& L, int n, int bk)
{
    if (L.zpf) return L.zpf[(int64_t)n * L.nb + bk];
    if (L.zp) return (float)unpack_code(L.zp, (int64_t)n * L.zrb, bk, L.bits);
    return (float)(1 << (L.bits - 1));
}

// One thread per output element (m, n); dot product in k order.
__global__ __launch_bounds__(256) void nbits_generic_kernel(RawLayout L, const float* __restrict__ a,
                                                            float* __restrict__ y, int M)
{
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)M * L.N) return;
    const int m = (int)(idx / L.N);
    const int n = (int)(idx - (int64_t)m * L.N);
    const float* arow = a + (int64_t)m * L.K;
    const int64_t row_base = (int64_t)n * L.nb * L.blob;
    float sum = 0.0f;
    for (int bk = 0; bk < L.nb; ++bk) {
        const float scale = L.scales[(int64_t)n * L.nb + bk];
        const float zp = block_zp(L, n, bk);
        const int k0 = bk * L.bs;
        const int len = min(L.bs, L.K - k0);
        const int64_t blob_base = row_base + (int64_t)bk * L.blob;
        for (int i = 0; i < len; ++i) {
            const float w = ((float)unpack_code(L.b, blob_base, i, L.bits) - zp) * scale;
            sum = __builtin_fmaf(arow[k0 + i], w, sum);
        }
    }
    y[idx] = sum;
}

// W[n,k] = ((float)q - zp) * scale for every (n, k).
__global__ __launch_bounds__(256) void nbits_dequant_kernel(RawLayout L, float* __restrict__ w)
{
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)L.N * L.K) return;
    const int n = (int)(idx / L.K);
    const int k = (int)(idx - (int64_t)n * L.K);
    const int bk = k / L.bs;
    const int i = k - bk * L.bs;
    const int64_t blob_base = (int64_t)n * L.nb * L.blob + (int64_t)bk * L.blob;
    const float scale = L.scales[(int64_t)n * L.nb + bk];
    w[idx] = ((float)unpack_code(L.b, blob_base, i, L.bits) - block_zp(L, n, bk)) * scale;
}

}  // namespace msnb
