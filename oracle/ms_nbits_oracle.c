/*
 * ms_nbits_oracle.c — CPU restatement of ModelSharp's managed MatMulNBits.
 *
 * TEST INFRASTRUCTURE: the oracle the HIP path is checked against, and the
 * CPU baseline bench.py times beside the GPU. Nothing in the product loads it.
 *
 * Built with -ffp-contract=off so that every multiply-add is fused exactly
 * where the reference fuses it (explicit fmaf, standing for the
 * Avx512F/Fma.FusedMultiplyAdd calls) and nowhere else.
 *
 * Pinning (tests/test_oracle.py):
 *   msor_unpack_nbit        exhaustive over all 256 bytes vs the packing rule,
 *                           reference KATs (MatMulNBitsTests.cs:57-267).
 *   msor_dequant_block4/8   closed form fl32((q-zp)*s) element-wise; bit-exact
 *                           against the reference's own ms_qgemm_nbits
 *                           (native/src/qgemm.cpp, built from source) through
 *                           one-hot activations.
 *   msor_fma_accumulate     exact sums of small integers (every partial sum
 *                           representable), double-precision brute force on
 *                           random data, all lengths 0..200 (every branch).
 *   msor_matmul_nbits       the 8 hand-derived KATs, the reference native
 *                           kernel on its own parity grid, f64 brute force.
 *   msor_matmul_f64         exact small-integer products.
 * The horizontal-sum order of Vector512.Sum / Vector256.Sum lives in the .NET
 * runtime (not in the checkout); it is restated as a pairwise fold of halves,
 * which fixes the oracle's own bits but not the managed kernel's (parity to
 * tolerance only, as the reference's own tests do).
 */
#include "ms_nbits_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

int msor_unpack_nbit(const uint8_t* data, int64_t base_byte, int index, int bits)
{
    /* MatMulNBitsKernel.cs:351-355 */
    if (bits == 8) return data[base_byte + index];
    const int64_t byte_off = base_byte + (index >> 1);
    const int shift = (index & 1) * 4;
    return (data[byte_off] >> shift) & 0x0F;
}

void msor_dequant_block4(const uint8_t* src, int64_t blob_base, int count,
                         float zp, float scale, float* dst)
{
    /* MatMulNBitsSimd.cs:50-95. The AVX2 path (UnpackLow/High of the low and
     * high nibbles, widen, convert, (q - zp) * scale) and the scalar tail
     * compute the same two fp32 operations per code, so one loop states all. */
    for (int i = 0; i < count; ++i) {
        const int b = src[blob_base + (i >> 1)];
        const int q = ((i & 1) == 0) ? (b & 0x0F) : ((b >> 4) & 0x0F);
        dst[i] = ((float)q - zp) * scale;
    }
}

void msor_dequant_block8(const uint8_t* src, int64_t blob_base, int count,
                         float zp, float scale, float* dst)
{
    /* MatMulNBitsSimd.cs:125-131 */
    for (int i = 0; i < count; ++i) dst[i] = ((float)src[blob_base + i] - zp) * scale;
}

/* Horizontal sums standing for Vector512.Sum / Vector256.Sum (runtime code,
 * not in the checkout): fold the upper half onto the lower half until one
 * lane remains. */
static float hsum16(const float* v)
{
    float t[8], u[4];
    for (int j = 0; j < 8; ++j) t[j] = v[j] + v[j + 8];
    for (int j = 0; j < 4; ++j) u[j] = t[j] + t[j + 4];
    return (u[0] + u[2]) + (u[1] + u[3]);
}

static float hsum8(const float* v)
{
    float u[4];
    for (int j = 0; j < 4; ++j) u[j] = v[j] + v[j + 4];
    return (u[0] + u[2]) + (u[1] + u[3]);
}

float msor_fma_accumulate(float acc, const float* a, const float* w, int n)
{
    int i = 0;
    if (n >= 16) {
        /* MatMulNBitsSimd.cs:145-162 (Avx512F branch) */
        float s0[16], s1[16], s2[16], s3[16], s[16];
        for (int j = 0; j < 16; ++j) s0[j] = s1[j] = s2[j] = s3[j] = 0.0f;
        const int last4 = n - 64;
        for (; i <= last4; i += 64) {
            for (int j = 0; j < 16; ++j) s0[j] = fmaf(a[i + j], w[i + j], s0[j]);
            for (int j = 0; j < 16; ++j) s1[j] = fmaf(a[i + 16 + j], w[i + 16 + j], s1[j]);
            for (int j = 0; j < 16; ++j) s2[j] = fmaf(a[i + 32 + j], w[i + 32 + j], s2[j]);
            for (int j = 0; j < 16; ++j) s3[j] = fmaf(a[i + 48 + j], w[i + 48 + j], s3[j]);
        }
        for (int j = 0; j < 16; ++j) s[j] = (s0[j] + s1[j]) + (s2[j] + s3[j]);
        const int last = n - 16;
        for (; i <= last; i += 16)
            for (int j = 0; j < 16; ++j) s[j] = fmaf(a[i + j], w[i + j], s[j]);
        acc += hsum16(s);
    } else if (n >= 8) {
        /* MatMulNBitsSimd.cs:163-180 (Fma branch; AVX-512 hosts take it for 8 <= n < 16) */
        float s0[8], s1[8], s2[8], s3[8], s[8];
        for (int j = 0; j < 8; ++j) s0[j] = s1[j] = s2[j] = s3[j] = 0.0f;
        const int last4 = n - 32;
        for (; i <= last4; i += 32) {
            for (int j = 0; j < 8; ++j) s0[j] = fmaf(a[i + j], w[i + j], s0[j]);
            for (int j = 0; j < 8; ++j) s1[j] = fmaf(a[i + 8 + j], w[i + 8 + j], s1[j]);
            for (int j = 0; j < 8; ++j) s2[j] = fmaf(a[i + 16 + j], w[i + 16 + j], s2[j]);
            for (int j = 0; j < 8; ++j) s3[j] = fmaf(a[i + 24 + j], w[i + 24 + j], s3[j]);
        }
        for (int j = 0; j < 8; ++j) s[j] = (s0[j] + s1[j]) + (s2[j] + s3[j]);
        const int last = n - 8;
        for (; i <= last; i += 8)
            for (int j = 0; j < 8; ++j) s[j] = fmaf(a[i + j], w[i + j], s[j]);
        acc += hsum8(s);
    } else {
        /* MatMulNBitsSimd.cs:181-199 (portable Vector<T>, 8 lanes): for n < 8
         * no full vector is formed, and Vector.Dot of the zero vector adds 0. */
        acc += 0.0f;
    }
    /* MatMulNBitsSimd.cs:201 — scalar tail, multiply then add */
    for (; i < n; ++i) {
        const float p = a[i] * w[i];
        acc += p;
    }
    return acc;
}

int msor_should_parallelize(int64_t rows, int64_t inner_cost, int dop)
{
    /* MatMulParallel.cs:32 (threshold 1<<16) and :38-39 */
    return rows > 1 && dop > 1 && rows * inner_cost >= (1LL << 16);
}

static float zero_point_of(const uint8_t* zp_packed, const float* zp_float, int64_t scale_row_base,
                           int64_t zp_row_base, int bk, int bits)
{
    /* MatMulNBitsKernel.cs:239-242 and the default at :115 */
    if (zp_float) return zp_float[scale_row_base + bk];
    if (zp_packed) return (float)msor_unpack_nbit(zp_packed, zp_row_base, bk, bits);
    return (float)(1 << (bits - 1));
}

void msor_matmul_nbits(const float* a, const uint8_t* b, const float* scales,
                       const uint8_t* zp_packed, const float* zp_float, float* y,
                       int M, int N, int K, int bits, int block_size, int nthreads)
{
    /* MatMulNBitsKernel.cs:95-96, :118, :193 */
    const int nb = (K + block_size - 1) / block_size;
    const int blob = (block_size * bits + 7) / 8;
    const int zrb = (nb * bits + 7) / 8;
    const int64_t row_bytes = (int64_t)nb * blob;
    if (nthreads < 1) nthreads = 1;
    const int par = msor_should_parallelize(N, (int64_t)K * (M + 1), nthreads);

#pragma omp parallel num_threads(nthreads) if (par)
    {
        /* MatMulNBitsKernel.cs:233-234 (block scratch and per-row accumulators) */
        float* wblock = (float*)malloc(sizeof(float) * (size_t)block_size);
        float* acc = (float*)malloc(sizeof(float) * (size_t)(M > 0 ? M : 1));
#pragma omp for schedule(static)
        for (int n = 0; n < N; ++n) {
            const int64_t b_row_base = (int64_t)n * row_bytes;
            const int64_t scale_row_base = (int64_t)n * nb;
            const int64_t zp_row_base = (int64_t)n * zrb;
            for (int m = 0; m < M; ++m) acc[m] = 0.0f;
            for (int bk = 0; bk < nb; ++bk) {              /* :236-258 */
                const float scale = scales[scale_row_base + bk];
                const float zp = zero_point_of(zp_packed, zp_float, scale_row_base, zp_row_base, bk, bits);
                const int64_t blob_base = b_row_base + (int64_t)bk * blob;
                const int k_start = bk * block_size;
                const int len = (block_size < K - k_start) ? block_size : K - k_start;
                if (len <= 0) break;
                if (bits == 4) msor_dequant_block4(b, blob_base, len, zp, scale, wblock);
                else msor_dequant_block8(b, blob_base, len, zp, scale, wblock);
                for (int m = 0; m < M; ++m)
                    acc[m] = msor_fma_accumulate(acc[m], a + (int64_t)m * K + k_start, wblock, len);
            }
            for (int m = 0; m < M; ++m) y[(int64_t)m * N + n] = acc[m];   /* :260-261 */
        }
        free(wblock);
        free(acc);
    }
}

void msor_dequant_weights(const uint8_t* b, const float* scales,
                          const uint8_t* zp_packed, const float* zp_float, float* w,
                          int N, int K, int bits, int block_size, int nthreads)
{
    const int nb = (K + block_size - 1) / block_size;
    const int blob = (block_size * bits + 7) / 8;
    const int zrb = (nb * bits + 7) / 8;
    const int64_t row_bytes = (int64_t)nb * blob;
    if (nthreads < 1) nthreads = 1;
#pragma omp parallel for schedule(static) num_threads(nthreads)
    for (int n = 0; n < N; ++n) {
        for (int bk = 0; bk < nb; ++bk) {
            const float scale = scales[(int64_t)n * nb + bk];
            const float zp = zero_point_of(zp_packed, zp_float, (int64_t)n * nb, (int64_t)n * zrb, bk, bits);
            const int k_start = bk * block_size;
            const int len = (block_size < K - k_start) ? block_size : K - k_start;
            if (len <= 0) break;
            float* dst = w + (int64_t)n * K + k_start;
            const int64_t blob_base = (int64_t)n * row_bytes + (int64_t)bk * blob;
            if (bits == 4) msor_dequant_block4(b, blob_base, len, zp, scale, dst);
            else msor_dequant_block8(b, blob_base, len, zp, scale, dst);
        }
    }
}

void msor_matmul_f64(const float* a, const float* w, double* y, int M, int N, int K, int nthreads)
{
    if (nthreads < 1) nthreads = 1;
#pragma omp parallel for schedule(static) num_threads(nthreads)
    for (int n = 0; n < N; ++n) {
        const float* wr = w + (int64_t)n * K;
        for (int m = 0; m < M; ++m) {
            const float* ar = a + (int64_t)m * K;
            double s = 0.0;
            for (int k = 0; k < K; ++k) s += (double)ar[k] * (double)wr[k];
            y[(int64_t)m * N + n] = s;
        }
    }
}

/* ---- W4A8: the opt-in approximate path (MODELSHARP_W4A8) ---------------------------------
 * Restates the reference's native ms_qgemm_w4a8 (native/src/qgemm_w4a8.cpp), the kernel
 * NativeQuant.TryMatMulNBits runs when MODELSHARP_W4A8 is on (NativeQuant.cs:78-115).
 *
 * Pinning (tests/test_oracle.py): bit-exact against the reference's own qgemm_w4a8.cpp
 * built from source (both its VNNI driver and, under MODELSHARP_FORCE_NOAVX512, its
 * scalar driver); exact on activations that quantize without error (integer rows whose
 * block max is 127: sa = 1, aq = a) against the integer dot; the reference test's
 * accuracy bar (rel-L2 < 0.03, cosine > 0.999 against the f64 dequantized product,
 * qgemm_w4a8_test.cpp:49-85) on its case grid; the quantizer against its closed form. */

void msor_w4a8_quantize(const float* a, int8_t* aq, float* sa, int M, int K, int block_size)
{
    /* qgemm_w4a8.cpp:257-285: per (row, K-block) symmetric int8, s = max|a| / 127,
     * q = lrintf(a * (1 / s)) clamped to [-127, 127]; the padding past K stays 0. */
    const int nb = (K + block_size - 1) / block_size;
    const int64_t padK = (int64_t)nb * block_size;
    for (int m = 0; m < M; ++m) {
        const float* arow = a + (int64_t)m * K;
        int8_t* qrow = aq + (int64_t)m * padK;
        for (int bk = 0; bk < nb; ++bk) {
            const int k0 = bk * block_size;
            const int k1 = (k0 + block_size < K) ? k0 + block_size : K;
            float amax = 0.0f;
            for (int k = k0; k < k1; ++k) {
                const float v = fabsf(arow[k]);
                if (v > amax) amax = v;
            }
            const float s = amax / 127.0f;
            sa[(int64_t)m * nb + bk] = s;
            const float inv = (s > 0.0f) ? (1.0f / s) : 0.0f;
            for (int k = k0; k < k1; ++k) {
                int q = (int)lrintf(arow[k] * inv);
                if (q > 127) q = 127;
                else if (q < -127) q = -127;
                qrow[k] = (int8_t)q;
            }
            for (int k = k1; k < k0 + block_size; ++k) qrow[k] = 0;
        }
    }
}

void msor_qgemm_w4a8(const float* a, const uint8_t* b, const float* scales, const uint8_t* zp_packed,
                     float* y, int M, int N, int K, int bits, int block_size, int nthreads)
{
    const int nb = (K + block_size - 1) / block_size;
    const int blob = (block_size * bits + 7) / 8;
    const int zrb = (nb * bits + 7) / 8;
    const int64_t row_bytes = (int64_t)nb * blob;
    const int64_t padK = (int64_t)nb * block_size;
    if (nthreads < 1) nthreads = 1;
    int8_t* aq = (int8_t*)malloc((size_t)(M > 0 ? M : 1) * (size_t)padK);
    float* sa = (float*)malloc(sizeof(float) * (size_t)(M > 0 ? M : 1) * (size_t)nb);
    msor_w4a8_quantize(a, aq, sa, M, K, block_size);
#pragma omp parallel num_threads(nthreads)
    {
        int* wc = (int*)malloc(sizeof(int) * (size_t)block_size);
#pragma omp for schedule(static)
        for (int n = 0; n < N; ++n) {
            for (int m = 0; m < M; ++m) {
                float acc = 0.0f;
                for (int bk = 0; bk < nb; ++bk) {
                    /* qgemm_w4a8.cpp:640-652: signed codes wc = code - zp, clamped to
                     * [-127, 127] (only 8-bit codes can reach the clamp) */
                    const int zp = zp_packed ? msor_unpack_nbit(zp_packed, (int64_t)n * zrb, bk, bits)
                                             : (1 << (bits - 1));
                    const int k0 = bk * block_size;
                    const int len = (block_size < K - k0) ? block_size : K - k0;
                    const int64_t blob_base = (int64_t)n * row_bytes + (int64_t)bk * blob;
                    int32_t dot = 0;
                    for (int i = 0; i < len; ++i) {
                        int v = msor_unpack_nbit(b, blob_base, i, bits) - zp;
                        if (v > 127) v = 127;
                        else if (v < -127) v = -127;
                        wc[i] = v;
                        dot += (int32_t)aq[(int64_t)m * padK + k0 + i] * v;
                    }
                    /* :676-689: the block's term, sa * s_w * (float)dot, added in block order */
                    acc += sa[(int64_t)m * nb + bk] * scales[(int64_t)n * nb + bk] * (float)dot;
                }
                y[(int64_t)m * N + n] = acc;
            }
        }
        free(wc);
    }
    free(aq);
    free(sa);
}

/* ---- W4A8, the managed variant ----------------------------------------------------------
 * Restates MatMulNBitsKernel.ExecuteColumnW4A8 (MatMulNBitsKernel.cs:275-331) with
 * MatMulNBitsSimd.QuantizeActivationInt8 (MatMulNBitsSimd.cs:225-255) and DotU8xU8
 * (:268-298, an exact integer dot): what the reference runs under MODELSHARP_W4A8 for 4-bit
 * codes when its native library does not take the call (library absent, or float zero
 * points, MatMulNBitsKernel.cs:174, :209).
 *
 * Against the native kernel above it differs in the quantizer's reciprocal
 * (inv = 127 / absmax instead of 1 / (absmax / 127), so a code can move by one where
 * a * inv lies next to a rounding tie), in the clamp (-128 instead of -127, unreachable
 * since |a * inv| <= 127 up to rounding), in skipping all-zero activation blocks (the
 * native kernel adds a zero term) and in taking float zero points: the block term is
 * s_w * s_a * (float)(dot(aq, q) - zp * sum(aq)), with q the raw code.
 *
 * Pinning (tests/test_oracle.py): equal bit for bit to msor_qgemm_w4a8 when every
 * activation block quantizes exactly (integer rows whose block maximum is 127: both
 * reciprocals are 1), codes within one step of the native quantizer's, and the reference
 * test's accuracy bar against the exact product. */
void msor_w4a8_managed(const float* a, const uint8_t* b, const float* scales, const uint8_t* zp_packed,
                       const float* zp_float, float* y, int M, int N, int K, int block_size, int nthreads)
{
    const int bits = 4;
    const int nb = (K + block_size - 1) / block_size;
    const int blob = (block_size * bits + 7) / 8;
    const int zrb = (nb * bits + 7) / 8;
    const int64_t row_bytes = (int64_t)nb * blob;
    if (nthreads < 1) nthreads = 1;
    /* the activation codes do not depend on the column: quantize every (row, block) once */
    int8_t* aq = (int8_t*)malloc((size_t)(M > 0 ? M : 1) * (size_t)nb * (size_t)block_size);
    float* sa = (float*)malloc(sizeof(float) * (size_t)(M > 0 ? M : 1) * (size_t)nb);
    int* sum_aq = (int*)malloc(sizeof(int) * (size_t)(M > 0 ? M : 1) * (size_t)nb);
    for (int m = 0; m < M; ++m) {
        for (int bk = 0; bk < nb; ++bk) {
            const int k0 = bk * block_size;
            const int len = (block_size < K - k0) ? block_size : K - k0;
            const float* src = a + (int64_t)m * K + k0;
            int8_t* dst = aq + ((int64_t)m * nb + bk) * block_size;
            /* MatMulNBitsSimd.cs:228-254 */
            float absmax = 0.0f;
            for (int i = 0; i < len; ++i) {
                const float v = fabsf(src[i]);
                if (v > absmax) absmax = v;
            }
            int sum = 0;
            if (absmax == 0.0f) {
                memset(dst, 0, (size_t)block_size);
                sa[(int64_t)m * nb + bk] = 0.0f;
            } else {
                const float inv = 127.0f / absmax;
                sa[(int64_t)m * nb + bk] = absmax / 127.0f;
                for (int i = 0; i < len; ++i) {
                    /* MathF.Round: to nearest, ties to even (rintf in the default mode) */
                    int q = (int)rintf(src[i] * inv);
                    if (q > 127) q = 127;
                    else if (q < -128) q = -128;
                    dst[i] = (int8_t)q;
                    sum += q;
                }
            }
            sum_aq[(int64_t)m * nb + bk] = sum;
        }
    }
#pragma omp parallel for num_threads(nthreads) schedule(static)
    for (int n = 0; n < N; ++n) {
        for (int m = 0; m < M; ++m) {
            float total = 0.0f;
            for (int bk = 0; bk < nb; ++bk) {
                const float sw = scales[(int64_t)n * nb + bk];
                float zp;
                if (zp_float) zp = zp_float[(int64_t)n * nb + bk];
                else if (zp_packed) zp = (float)msor_unpack_nbit(zp_packed, (int64_t)n * zrb, bk, bits);
                else zp = 8.0f;
                const int k0 = bk * block_size;
                const int len = (block_size < K - k0) ? block_size : K - k0;
                if (len <= 0) break;
                const float s_a = sa[(int64_t)m * nb + bk];
                if (s_a == 0.0f) continue;   /* MatMulNBitsKernel.cs:310 */
                const int8_t* q8 = aq + ((int64_t)m * nb + bk) * block_size;
                const int64_t blob_base = (int64_t)n * row_bytes + (int64_t)bk * blob;
                /* :314-322: sum over (aq + 128) * q, less 128 * sum(q): exactly sum(aq * q) */
                int32_t dot = 0;
                for (int i = 0; i < len; ++i) dot += (int32_t)q8[i] * msor_unpack_nbit(b, blob_base, i, bits);
                /* :325: scaleW * scaleA * (dotAqQ - zp * sumAq), float arithmetic throughout */
                const float comp = zp * (float)sum_aq[(int64_t)m * nb + bk];
                total += sw * s_a * ((float)dot - comp);
            }
            y[(int64_t)m * N + n] = total;
        }
    }
    free(aq);
    free(sa);
    free(sum_aq);
}
