/*
 * ms_nbits_oracle.h — CPU oracle for the MatMulNBits operator.
 *
 * TEST INFRASTRUCTURE. Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg load this library, and only to check the device's results or
 * as the timed CPU baseline. The product library (modelsharp_amd/csrc) never links it.
 *
 * Every function restates one piece of the reference's managed kernel; the
 * file:line citation is on each declaration (paths are relative to the
 * ModelSharp checkout).
 */
#ifndef MS_NBITS_ORACLE_H
#define MS_NBITS_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* UnpackNBit — src/ModelSharp/Cpu/Kernels/Quantize/MatMulNBitsKernel.cs:349-356.
 * index-th `bits`-wide code of the packed region at base_byte; bits=4 keeps the
 * even index in the low nibble. */
int msor_unpack_nbit(const uint8_t* data, int64_t base_byte, int index, int bits);

/* DequantBlock4 — MatMulNBitsSimd.cs:40-96 (AVX2 unpack :50-69, vector tail
 * :72-88, scalar tail :90-95; all three produce the same fp32 values).
 * dst[i] = ((float)q_i - zp) * scale, one rounding for integer zp. */
void msor_dequant_block4(const uint8_t* src, int64_t blob_base, int count,
                         float zp, float scale, float* dst);

/* DequantBlock8 — MatMulNBitsSimd.cs:117-132. */
void msor_dequant_block8(const uint8_t* src, int64_t blob_base, int count,
                         float zp, float scale, float* dst);

/* FmaAccumulate — MatMulNBitsSimd.cs:141-203, the branch an AVX-512 host takes:
 * n>=16: four 16-lane FMA accumulators over 64-element steps, fold, 16-lane
 * steps, horizontal sum added to acc; 8<=n<16: the 8-lane FMA branch;
 * n<8: the portable branch (no full vector); then the scalar tail
 * acc += a*w (separate multiply and add, no fusion). */
float msor_fma_accumulate(float acc, const float* a, const float* w, int n);

/* MatMulParallel.ShouldParallelize — Cpu/Kernels/Linear/MatMulParallel.cs:32-39. */
int msor_should_parallelize(int64_t rows, int64_t inner_cost, int dop);

/* MatMulNBitsKernel.Execute default path — MatMulNBitsKernel.cs:193-262:
 * column-parallel over N (MatMulParallel.For, :216), per column the fused
 * block loop (:236-258) and the store (:260-261).
 * zp_packed / zp_float: at most one non-NULL (NULL/NULL = default 2^(bits-1)).
 * nthreads is the degree of parallelism (Environment.ProcessorCount). */
void msor_matmul_nbits(const float* a, const uint8_t* b, const float* scales,
                       const uint8_t* zp_packed, const float* zp_float, float* y,
                       int M, int N, int K, int bits, int block_size, int nthreads);

/* The dequantized weight matrix W[N,K] the kernel above multiplies by, built
 * from the same per-block dequant (MatMulNBitsKernel.cs:236-253). */
void msor_dequant_weights(const uint8_t* b, const float* scales,
                          const uint8_t* zp_packed, const float* zp_float, float* w,
                          int N, int K, int bits, int block_size, int nthreads);

/* Double-accumulated brute force y[m,n] = sum_k (double)a[m,k]*(double)w[n,k]
 * over the fp32 dequantized weights, as native/test/qgemm_test.cpp:60-89
 * does for its reference. */
void msor_matmul_f64(const float* a, const float* w, double* y,
                     int M, int N, int K, int nthreads);

/* W4A8 (native/src/qgemm_w4a8.cpp): per (row, block) int8 activations aq [M][nb*bs]
 * (zero past K) and their scales sa [M][nb]; the approximate product. */
void msor_w4a8_quantize(const float* a, int8_t* aq, float* sa, int M, int K, int block_size);
void msor_qgemm_w4a8(const float* a, const uint8_t* b, const float* scales, const uint8_t* zp_packed,
                     float* y, int M, int N, int K, int bits, int block_size, int nthreads);
/* The managed W4A8 variant (MatMulNBitsKernel.ExecuteColumnW4A8, 4-bit codes): packed,
 * float (zp_float, [N][nb]) or no zero points. */
void msor_w4a8_managed(const float* a, const uint8_t* b, const float* scales, const uint8_t* zp_packed,
                       const float* zp_float, float* y, int M, int N, int K, int block_size, int nthreads);

/* Decoder-layer neighbours (ms_decoder_oracle.c). */
void msor_rmsnorm(const float* x, const float* scale, float* y, float* inv_std, int64_t rows, int norm, float eps);
void msor_skip_rmsnorm(const float* input, const float* skip, const float* gamma, const float* beta,
                       const float* bias, float* out, float* sum, float* inv_std, int64_t rows, int norm, float eps);
void msor_silu_mul(const float* g, const float* u, float* y, int64_t n);

typedef struct msor_gqa_desc {
    int batch, q_seq, kv_seq;
    int num_heads, kv_num_heads, head_dim;
    int packed_qkv;
    int past_seq, past_in_present, present_capacity;
    int do_rotary, rotary_interleaved, cos_rows, cos_cols;
    int local_window_size;
    float scale;
    int seqlens_len;
} msor_gqa_desc;
/* present K/V are [B, kv_heads, past + kv_seq, head_dim] (the reference's layout) */
void msor_gqa(const msor_gqa_desc* d, const float* q, const float* k, const float* v, const float* past_k,
              const float* past_v, const int32_t* seqlens, const float* cos_c, const float* sin_c, float* out,
              float* present_k, float* present_v);

#ifdef __cplusplus
}
#endif
#endif
