// mfma_general.h — GEMM (M > 16) on the matrix cores for the weight formats the 4-bit
// kernels do not take: bits = 8, float zero points, block sizes other than 32/64/128/256,
// K not a multiple of 32 (K and the block size multiples of 8). At fp32-level accuracy:
//   * the producer dequantizes every weight exactly as the reference does
//     (W = fl(fl(q - zp) * s), generic_nbits.h) and splits it into fp16 halves,
//     W = 2^f[n] (Wh + Wl), with the row exponent f[n] (precomputed per weights handle)
//     bringing the row's largest possible |W| into [2^14, 2^15);
//   * each row of A is split the same way, A = 2^e[m] (Ah + Al), e[m] from the row's
//     max |A| (read once in the prologue);
//   * three MFMAs per operand pair, Ah Wh + Ah Wl + Al Wh: every product exact in fp32,
//     the terms dropped (Al Wl) below 2^-22 of the product, fp32 sums; the epilogue
//     multiplies by 2^(e[m] + f[n]) (exact).
//
// Mapping: a workgroup (4 waves stacked along M, 32 rows each) owns a 128 x 64 tile of Y,
// two v_mfma_f32_32x32x16_f16 fragments per wave; K advances 32 codes per step. The 256
// threads dequantize the step's 64 x 32 weights (4 threads per row, 8 codes each) into
// double-buffered LDS tiles of Wh and Wl; each wave loads its A rows straight from global
// memory in the MFMA operand layout, one step ahead, and splits them in registers.
#pragma once
#include "generic_nbits.h"
#include "mfma_w4.h"

namespace msnb {

constexpr int kGenBM = 128, kGenBN = 64;

struct GenParams {
    RawLayout L;
    const int* wexp;   // [N] row exponents f[n] of the weights
    const float* a;    // [M][K]
    float* y;          // [M][N]
    int M, tiles_m, tiles_n;
};

// Row exponent f[n]: the largest |W| a row can produce, max over its blocks of
// |s| * max(|zp|, |2^bits - 1 - zp|), brought into [2^14, 2^15) by 2^-f (rows that can
// only produce zeros, or non-finite ones, take 0).
__global__ __launch_bounds__(256) void weight_row_exponent_kernel(RawLayout L, int* __restrict__ wexp)
{
    const int n = blockIdx.x * blockDim.x + threadIdx.x;
    if (n >= L.N) return;
    const float qmax = (float)((1 << L.bits) - 1);
    float mx = 0.0f;
    for (int b = 0; b < L.nb; ++b) {
        const float zp = block_zp(L, n, b);
        mx = fmaxf(mx, fabsf(L.scales[(int64_t)n * L.nb + b]) * fmaxf(fabsf(zp), fabsf(qmax - zp)));
    }
    wexp[n] = (mx > 0.0f && mx <= 3.402823466e38f) ? __builtin_amdgcn_frexp_expf(mx) - 15 : 0;
}

// hi / lo fp16 halves of x * 2^-e.
__device__ __forceinline__ void split_hl(float x, int e, _Float16& h, _Float16& l)
{
    const float v = __builtin_amdgcn_ldexpf(x, -e);
    h = (_Float16)v;
    l = (_Float16)(v - (float)h);
}

__global__ __launch_bounds__(256) void mfma_general_kernel(GenParams p)
{
    constexpr int WM = 32, NF = kGenBN / 32;
    const RawLayout& L = p.L;
    __shared__ __attribute__((aligned(16))) _Float16 Bh[2][kGenBN][kBsStride];
    __shared__ __attribute__((aligned(16))) _Float16 Bl[2][kGenBN][kBsStride];
    __shared__ int Es[kGenBM], Fs[kGenBN];

    const int tile = xcd_tile(blockIdx.x, p.tiles_m * p.tiles_n);
    if (tile >= p.tiles_m * p.tiles_n) return;
    const int m0 = (tile / p.tiles_n) * kGenBM, n0 = (tile % p.tiles_n) * kGenBN;
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
    const int C = (L.K + 31) / 32;
    const int64_t row_bytes = (int64_t)L.nb * L.blob;

    // ---- producer: row pn of the tile, codes [8 ph, 8 ph + 8) of each 32-code step ----
    const int pn = tid >> 2, ph = tid & 3;
    const int prow = min(n0 + pn, L.N - 1);
    if (ph == 0) Fs[pn] = p.wexp[prow];
    const int fexp = p.wexp[prow];
    auto produce = [&](int t, int buf) {
        const int k0 = 32 * t + 8 * ph;
        _Float16 h[8], l[8];
        if (k0 < L.K) {   // K and the block size are multiples of 8: the group is whole, in one block
            const int bk = k0 / L.bs, i0 = k0 - bk * L.bs;
            const float s = L.scales[(int64_t)prow * L.nb + bk];
            const float zp = block_zp(L, prow, bk);
            const uint8_t* src = L.b + (int64_t)prow * row_bytes + (int64_t)bk * L.blob;
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
            for (int i = 0; i < 8; ++i) split_hl(w[i], fexp, h[i], l[i]);
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) h[i] = l[i] = (_Float16)0.0f;
        }
        half8_t hv, lv;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            hv[i] = h[i];
            lv[i] = l[i];
        }
        *reinterpret_cast<half8_t*>(&Bh[buf][pn][8 * ph]) = hv;
        *reinterpret_cast<half8_t*>(&Bl[buf][pn][8 * ph]) = lv;
    };

    // ---- consumer: lane -> A row (l % 32), 8-k slot (l / 32) of each 16-k half step ----
    const int am = min(m0 + wave * WM + (lane & 31), p.M - 1);
    const float* pa = p.a + (int64_t)am * L.K + 8 * (lane >> 5);
    auto load_a = [&](int t, float4 (&f)[4]) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int k = 32 * t + 8 * (lane >> 5) + 16 * (q >> 1) + 4 * (q & 1);
            f[q] = k < L.K ? *reinterpret_cast<const float4*>(pa + 32 * t + 16 * (q >> 1) + 4 * (q & 1))
                           : float4{0.0f, 0.0f, 0.0f, 0.0f};
        }
    };
    // Row exponent of A (lanes l and l + 32 hold the two halves of row l % 32).
    int ea;
    {
        float mx = 0.0f;
        for (int t = 0; t < C; ++t) {
            float4 f[4];
            load_a(t, f);
#pragma unroll
            for (int q = 0; q < 4; ++q)
                mx = fmaxf(mx, fmaxf(fmaxf(fabsf(f[q].x), fabsf(f[q].y)), fmaxf(fabsf(f[q].z), fabsf(f[q].w))));
        }
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        ea = (mx > 0.0f && mx <= 3.402823466e38f) ? __builtin_amdgcn_frexp_expf(mx) - 15 : 0;
        if (lane < 32) Es[wave * WM + lane] = ea;
    }

    floatx16_t acc[NF];
#pragma unroll
    for (int j = 0; j < NF; ++j) acc[j] = floatx16_t{};

    float4 fa[4];
    load_a(0, fa);
    produce(0, 0);
    __syncthreads();
    for (int t = 0; t < C; ++t) {
        const int buf = t & 1;
        half8_t ah[2], al[2];
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const float v[8] = {fa[2 * s].x, fa[2 * s].y, fa[2 * s].z, fa[2 * s].w,
                                fa[2 * s + 1].x, fa[2 * s + 1].y, fa[2 * s + 1].z, fa[2 * s + 1].w};
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                _Float16 h, l;
                split_hl(v[i], ea, h, l);
                ah[s][i] = h;
                al[s][i] = l;
            }
        }
        if (t + 1 < C) load_a(t + 1, fa);
#pragma unroll
        for (int j = 0; j < NF; ++j) {
            const int r = 32 * j + (lane & 31), c = 8 * (lane >> 5);
            const half8_t bh0 = *reinterpret_cast<const half8_t*>(&Bh[buf][r][c]);
            const half8_t bh1 = *reinterpret_cast<const half8_t*>(&Bh[buf][r][c + 16]);
            const half8_t bl0 = *reinterpret_cast<const half8_t*>(&Bl[buf][r][c]);
            const half8_t bl1 = *reinterpret_cast<const half8_t*>(&Bl[buf][r][c + 16]);
            acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[0], bh0, acc[j], 0, 0, 0);
            acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[1], bh1, acc[j], 0, 0, 0);
            acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[0], bl0, acc[j], 0, 0, 0);
            acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(ah[1], bl1, acc[j], 0, 0, 0);
            acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[0], bh0, acc[j], 0, 0, 0);
            acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(al[1], bh1, acc[j], 0, 0, 0);
        }
        if (t + 1 < C) produce(t + 1, buf ^ 1);
        __syncthreads();
    }

    // ---- epilogue: acc[j][v] is Y[row][col] / 2^(Es[row] + Fs[col]), col = lane % 32 of
    // fragment j, row = 8 (v / 4) + 4 (lane / 32) + v % 4 of the wave's 32 rows ----
    const int r0 = wave * WM + 4 * (lane >> 5);
#pragma unroll
    for (int j = 0; j < NF; ++j) {
        const int cl = 32 * j + (lane & 31), col = n0 + cl;
        if (col < L.N) {
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int r = r0 + 8 * (v >> 2) + (v & 3), row = m0 + r;
                if (row < p.M) p.y[(int64_t)row * L.N + col] = __builtin_amdgcn_ldexpf(acc[j][v], Es[r] + Fs[cl]);
            }
        }
    }
}

}  // namespace msnb
