// w4a8.h — the opt-in W4A8 product (MODELSHARP_W4A8): activations quantized to int8 per
// (row, K-block), integer block dots against signed weight codes, fp32 block terms added
// in block order. Bit for bit the reference's native ms_qgemm_w4a8 built without FP contraction
// (native/src/qgemm_w4a8.cpp:247-296 quantizer, :622-679 reduce, which its VNNI driver
// reproduces value for value):
//   s_a(m, b) = max|a[m, block b]| / 127,  aq = lrint(a * (1 / s_a)) clamped to [-127, 127];
//   wc = code - zp, clamped to [-127, 127];  d(m, n, b) = sum_k aq * wc  (int32, exact);
//   y[m, n] = (...((0 + t_0) + t_1) + ...) + t_{nb-1},  t_b = (s_a(m, b) * s_w(n, b)) * (float)d,
//   each operation rounded on its own in fp32 (the library is built with -ffp-contract=off).
//
// Activation codes are stored in "nibble order": within every aligned group of 8 k, the
// even k first, then the odd k — the order in which a packed 4-bit weight word splits into
// its low nibbles (x & 0x0F0F0F0F) and high nibbles (x >> 4 & 0x0F0F0F0F). Integer dots are
// independent of the order of their terms, so the weights need no byte permutation.
//
// Kernels:
//   w4a8_quantize_kernel   8 lanes per (row, block): aq [M][padK], s_a [M][nb] and its
//                          transpose [nb][Mp] (Mp = M rounded up to 4, zero rows past M)
//   gemv_w4a8_kernel<M>    M <= 16, 4-bit codes, block size a multiple of 32: 16 lanes per
//                          weight row, lane g takes blocks g, g + 16, ...; each round of 16
//                          blocks leaves its 16 terms per row of A in LDS and lane m of the
//                          row adds them, in block order, to row m's sum
//   mfma_w4a8_kernel       M > 16, same formats: a 128 x 64 tile of Y per workgroup,
//                          v_mfma_i32_32x32x32_i8 per 32 codes into an int32 block
//                          accumulator, rescaled into the fp32 sum at each block's end
//   w4a8_generic_kernel    every other format (8-bit codes, any block size): one thread
//                          per output, the definition above as written
#pragma once
#include "generic_nbits.h"
#include "mfma_w4.h"

namespace msnb {

typedef int v4i_t __attribute__((ext_vector_type(4)));
typedef int v16i_t __attribute__((ext_vector_type(16)));

// Position of k in the nibble-ordered code row.
__device__ __forceinline__ int w4a8_pos(int k)
{
    const int p = k & 7;
    return (k & ~7) + ((p & 1) ? 4 + (p >> 1) : (p >> 1));
}

struct W4a8Args {
    const int8_t* aq;   // [M][padK] nibble order, zero past K
    const float* sa;    // [M][nb]
    const float* sat;   // [nb][Mp]
    int M, Mp, padK;
};

// ---- activation quantizer (qgemm_w4a8.cpp:257-285) -----------------------------------------
__global__ __launch_bounds__(256) void w4a8_quantize_kernel(const float* __restrict__ a, int8_t* __restrict__ aq,
                                                            float* __restrict__ sa, float* __restrict__ sat, int M,
                                                            int Mp, int K, int bs, int nb, int padK)
{
    const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int j = (int)(gid & 7);
    const int64_t blk = gid >> 3;              // (row, block) id; rows M..Mp-1 only clear sat
    if (blk >= (int64_t)Mp * nb) return;       // whole groups of 8 lanes leave together
    const int m = (int)(blk / nb), bk = (int)(blk - (int64_t)m * nb);
    if (m >= M) {
        if (j == 0) sat[(int64_t)bk * Mp + m] = 0.0f;
        return;
    }
    const int k0 = bk * bs;
    const int len = min(bs, K - k0);
    const float* arow = a + (int64_t)m * K + k0;
    float amax = 0.0f;
    for (int i = j; i < len; i += 8) amax = fmaxf(amax, fabsf(arow[i]));
    amax = fmaxf(amax, __shfl_xor(amax, 1, 8));
    amax = fmaxf(amax, __shfl_xor(amax, 2, 8));
    amax = fmaxf(amax, __shfl_xor(amax, 4, 8));
    const float s = amax / 127.0f;
    const float inv = s > 0.0f ? 1.0f / s : 0.0f;
    int8_t* qrow = aq + (int64_t)m * padK;
    for (int i = j; i < bs; i += 8) {
        int q = 0;
        if (i < len) {
            q = (int)__builtin_rintf(arow[i] * inv);
            q = max(-127, min(127, q));
        }
        qrow[w4a8_pos(k0 + i)] = (int8_t)q;
    }
    if (j == 0) {
        sa[(int64_t)m * nb + bk] = s;
        sat[(int64_t)bk * Mp + m] = s;
    }
}

// Signed codes (code - zp, as int8 bytes) of 8 packed 4-bit codes: the even k, the odd k.
__device__ __forceinline__ void w4a8_codes(uint32_t x, uint32_t z4, uint32_t& ev, uint32_t& od)
{
    // 0x80 + code - zp stays within a byte (codes and zero points are 0..15): no borrow
    // crosses bytes, and the xor turns the biased byte into the two's-complement code.
    ev = (((x & 0x0F0F0F0Fu) | 0x80808080u) - z4) ^ 0x80808080u;
    od = ((((x >> 4) & 0x0F0F0F0Fu) | 0x80808080u) - z4) ^ 0x80808080u;
}

__device__ __forceinline__ int w4a8_zp4(const RawLayout& L, int n, int bk)
{
    return L.zp ? unpack_code(L.zp, (int64_t)n * L.zrb, bk, 4) : 8;
}

// ---- decode GEMV ----------------------------------------------------------------------------
constexpr int kW8RowsPerWg = 16;

template <int M>
__global__ __launch_bounds__(256) void gemv_w4a8_kernel(RawLayout L, W4a8Args A, float* __restrict__ y)
{
    __shared__ float T[4][4][M][16];   // [wave][row][m][block slot]
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int g = lane & 15, r = lane >> 4;
    const int n = blockIdx.x * kW8RowsPerWg + wave * 4 + r;
    const bool live = n < L.N;
    const int nr = live ? n : L.N - 1;
    const int64_t row_bytes = (int64_t)L.nb * L.blob;
    const uint8_t* brow = L.b + (int64_t)nr * row_bytes;
    const int spb = L.bs >> 5;   // 32-code steps per block
    float acc = 0.0f;            // lane g < M: row g of A
    for (int base = 0; base < L.nb; base += 16) {
        const int bk = base + g;
        float t[M];
        if (bk < L.nb) {
            const uint32_t z4 = (uint32_t)w4a8_zp4(L, nr, bk) * 0x01010101u;
            const float sw = L.scales[(int64_t)nr * L.nb + bk];
            int d[M];
#pragma unroll
            for (int m = 0; m < M; ++m) d[m] = 0;
            for (int s = 0; s < spb; ++s) {
                const uint4 x = *reinterpret_cast<const uint4*>(brow + (int64_t)bk * L.blob + 16 * s);
                uint32_t w[8];
                w4a8_codes(x.x, z4, w[0], w[1]);
                w4a8_codes(x.y, z4, w[2], w[3]);
                w4a8_codes(x.z, z4, w[4], w[5]);
                w4a8_codes(x.w, z4, w[6], w[7]);
#pragma unroll
                for (int m = 0; m < M; ++m) {
                    const int8_t* q = A.aq + (int64_t)m * A.padK + (int64_t)bk * L.bs + 32 * s;
                    const uint4 q0 = *reinterpret_cast<const uint4*>(q);
                    const uint4 q1 = *reinterpret_cast<const uint4*>(q + 16);
                    int v = d[m];
                    v = __builtin_amdgcn_sdot4((int)q0.x, (int)w[0], v, false);
                    v = __builtin_amdgcn_sdot4((int)q0.y, (int)w[1], v, false);
                    v = __builtin_amdgcn_sdot4((int)q0.z, (int)w[2], v, false);
                    v = __builtin_amdgcn_sdot4((int)q0.w, (int)w[3], v, false);
                    v = __builtin_amdgcn_sdot4((int)q1.x, (int)w[4], v, false);
                    v = __builtin_amdgcn_sdot4((int)q1.y, (int)w[5], v, false);
                    v = __builtin_amdgcn_sdot4((int)q1.z, (int)w[6], v, false);
                    v = __builtin_amdgcn_sdot4((int)q1.w, (int)w[7], v, false);
                    d[m] = v;
                }
            }
#pragma unroll
            for (int m = 0; m < M; ++m) {
                const float p = A.sa[(int64_t)m * L.nb + bk] * sw;
                t[m] = p * (float)d[m];
            }
        } else {
#pragma unroll
            for (int m = 0; m < M; ++m) t[m] = 0.0f;
        }
#pragma unroll
        for (int m = 0; m < M; ++m) T[wave][r][m][g] = t[m];
        __syncthreads();
        if (g < M) {
            const int cnt = min(16, L.nb - base);
            for (int j = 0; j < cnt; ++j) acc = acc + T[wave][r][g][j];
        }
        __syncthreads();
    }
    if (live && g < M) y[(int64_t)g * L.N + n] = acc;
}

// ---- prefill on the int8 matrix cores ---------------------------------------------------------
constexpr int kW8BM = 128, kW8BN = 64;

struct W4a8MfmaParams {
    RawLayout L;
    W4a8Args A;
    float* y;
    int tiles_m, tiles_n;
};

__global__ __launch_bounds__(256) void mfma_w4a8_kernel(W4a8MfmaParams p)
{
    constexpr int NF = kW8BN / 32;
    const RawLayout& L = p.L;
    __shared__ __attribute__((aligned(16))) uint32_t Bw[2][kW8BN][8];   // 32 signed codes per row
    __shared__ float Sw[2][kW8BN];

    const int tile = xcd_tile(blockIdx.x, p.tiles_m * p.tiles_n);
    if (tile >= p.tiles_m * p.tiles_n) return;
    const int m0 = (tile / p.tiles_n) * kW8BM, n0 = (tile % p.tiles_n) * kW8BN;
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wave = tid / kWave;
    const int spb = L.bs >> 5;
    const int C = L.nb * spb;   // 32-code steps over padK
    const int64_t row_bytes = (int64_t)L.nb * L.blob;

    // producer: row pn of the tile, codes [8 ph, 8 ph + 8) of each step
    const int pn = tid >> 2, ph = tid & 3;
    const int prow = min(n0 + pn, L.N - 1);
    const uint8_t* brow = L.b + (int64_t)prow * row_bytes + 4 * ph;
    auto produce = [&](int bk, int s, int buf) {
        const uint32_t x = *reinterpret_cast<const uint32_t*>(brow + (int64_t)bk * L.blob + 16 * s);
        const uint32_t z4 = (uint32_t)w4a8_zp4(L, prow, bk) * 0x01010101u;
        uint32_t ev, od;
        w4a8_codes(x, z4, ev, od);
        Bw[buf][pn][2 * ph] = ev;
        Bw[buf][pn][2 * ph + 1] = od;
        if (ph == 0) Sw[buf][pn] = L.scales[(int64_t)prow * L.nb + bk];
    };

    // consumer: lane -> A row (l % 32), 16-byte k slot (l / 32) of each step
    const int am = min(m0 + wave * 32 + (lane & 31), p.A.M - 1);
    const int8_t* pa = p.A.aq + (int64_t)am * p.A.padK + 16 * (lane >> 5);
    // rows of the lane's 16 outputs: rbase + 8 (v / 4) + v % 4; groups of 4 rows read as one
    // float4 of the transposed activation scales (clamped into the array past M)
    const int rbase = m0 + wave * 32 + 4 * (lane >> 5);
    int sa_off[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) sa_off[q] = min(rbase + 8 * q, p.A.Mp - 4);

    float facc[NF][16];
#pragma unroll
    for (int j = 0; j < NF; ++j)
#pragma unroll
        for (int v = 0; v < 16; ++v) facc[j][v] = 0.0f;
    v16i_t iacc[NF];
#pragma unroll
    for (int j = 0; j < NF; ++j) iacc[j] = v16i_t{};

    v4i_t a_next = *reinterpret_cast<const v4i_t*>(pa);
    produce(0, 0, 0);
    __syncthreads();
    int t = 0;   // 32-code step; buffer t & 1
    for (int bk = 0; bk < L.nb; ++bk) {
        float4 sa4[4];   // the block's activation scales, read while its steps run
#pragma unroll
        for (int q = 0; q < 4; ++q)
            sa4[q] = *reinterpret_cast<const float4*>(p.A.sat + (int64_t)bk * p.A.Mp + sa_off[q]);
        for (int s = 0; s < spb; ++s, ++t) {
            const int buf = t & 1;
            const v4i_t a_cur = a_next;
            if (t + 1 < C) a_next = *reinterpret_cast<const v4i_t*>(pa + 32 * (t + 1));
#pragma unroll
            for (int j = 0; j < NF; ++j) {
                const v4i_t b = *reinterpret_cast<const v4i_t*>(&Bw[buf][32 * j + (lane & 31)][4 * (lane >> 5)]);
                iacc[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a_cur, b, iacc[j], 0, 0, 0);
            }
            if (s == spb - 1) {   // the block's end: its terms join the fp32 sums, in block order
#pragma unroll
                for (int j = 0; j < NF; ++j) {
                    const float sw = Sw[buf][32 * j + (lane & 31)];
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const float sq[4] = {sa4[q].x, sa4[q].y, sa4[q].z, sa4[q].w};
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const int v = 4 * q + i;
                            const float pr = sq[i] * sw;
                            facc[j][v] = facc[j][v] + pr * (float)iacc[j][v];
                        }
                    }
                    iacc[j] = v16i_t{};
                }
            }
            if (t + 1 < C) {
                if (s + 1 < spb) produce(bk, s + 1, buf ^ 1);
                else produce(bk + 1, 0, buf ^ 1);
            }
            __syncthreads();
        }
    }

#pragma unroll
    for (int j = 0; j < NF; ++j) {
        const int col = n0 + 32 * j + (lane & 31);
        if (col < L.N) {
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const int row = rbase + 8 * (v >> 2) + (v & 3);
                if (row < p.A.M) p.y[(int64_t)row * L.N + col] = facc[j][v];
            }
        }
    }
}

// ---- every other format ---------------------------------------------------------------------
__global__ __launch_bounds__(256) void w4a8_generic_kernel(RawLayout L, W4a8Args A, float* __restrict__ y)
{
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= (int64_t)A.M * L.N) return;
    const int m = (int)(idx / L.N);
    const int n = (int)(idx - (int64_t)m * L.N);
    const int64_t row_base = (int64_t)n * L.nb * L.blob;
    const int8_t* q = A.aq + (int64_t)m * A.padK;
    float acc = 0.0f;
    for (int bk = 0; bk < L.nb; ++bk) {
        const int zp = L.zp ? unpack_code(L.zp, (int64_t)n * L.zrb, bk, L.bits) : (1 << (L.bits - 1));
        const int k0 = bk * L.bs;
        const int len = min(L.bs, L.K - k0);
        const int64_t blob_base = row_base + (int64_t)bk * L.blob;
        int d = 0;
        for (int i = 0; i < len; ++i) {
            const int v = max(-127, min(127, unpack_code(L.b, blob_base, i, L.bits) - zp));
            d += (int)q[w4a8_pos(k0 + i)] * v;
        }
        const float pr = A.sa[(int64_t)m * L.nb + bk] * L.scales[(int64_t)n * L.nb + bk];
        acc = acc + pr * (float)d;
    }
    y[idx] = acc;
}

}  // namespace msnb
