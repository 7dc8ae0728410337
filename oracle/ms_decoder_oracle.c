/*
 * ms_decoder_oracle.c — CPU restatement of the decoder-layer operators next to
 * MatMulNBits in the reference's managed engine.
 *
 * TEST INFRASTRUCTURE: the oracle the device neighbours are checked against.
 * Nothing in the product loads it.
 *
 * Built with -ffp-contract=off: every multiply and add is rounded on its own
 * unless an fmaf() stands for the reference's SimdFma.MulAdd.
 *
 * Vector<float> reductions (KernelSimd.cs) are restated with 8 lanes and the
 * lane sum taken in lane order; the .NET runtime's horizontal order is not in
 * the checkout, so these functions fix the oracle's bits but the reference's
 * only to summation-order tolerance.
 *
 * Pinning (tests/test_oracle.py):
 *   msor_rmsnorm / msor_skip_rmsnorm   the float64 closed form, rows of constant
 *                                      magnitude (inv exact), the residual-sum output
 *   msor_silu_mul                      float64 closed form; sigmoid(0) = 1/2, odd
 *                                      symmetry sigmoid(-x) = 1 - sigmoid(x)
 *   msor_gqa                           float64 brute-force attention (causal,
 *                                      window, seqlens_k, past, packed QKV, group
 *                                      sharing), rotary as the closed-form rotation
 *                                      (pair norms kept, identity at cos 1 / sin 0),
 *                                      one visible key gives its value row, equal
 *                                      scores give the mean of the value rows
 */
#include "ms_nbits_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#define LANES 8

static float sum_squares(const float* a, int n)
{
    /* KernelSimd.cs:66-78 */
    float acc[LANES] = {0};
    int i = 0;
    for (; i + LANES <= n; i += LANES)
        for (int l = 0; l < LANES; ++l) acc[l] = acc[l] + a[i + l] * a[i + l];
    float s = 0.0f;
    for (int l = 0; l < LANES; ++l) s = s + acc[l];
    for (; i < n; ++i) s = s + a[i] * a[i];
    return s;
}

void msor_rmsnorm(const float* x, const float* scale, float* y, float* inv_std, int64_t rows, int norm, float eps)
{
    /* SimplifiedLayerNormalizationKernel.cs:46-53 and NormApply (KernelSimd.cs:112-135) */
    for (int64_t o = 0; o < rows; ++o) {
        const float* xr = x + o * norm;
        const float inv = 1.0f / sqrtf(sum_squares(xr, norm) / (float)norm + eps);
        if (inv_std) inv_std[o] = inv;
        for (int i = 0; i < norm; ++i) y[o * norm + i] = (xr[i] * inv) * scale[i];
    }
}

void msor_skip_rmsnorm(const float* input, const float* skip, const float* gamma, const float* beta,
                       const float* bias, float* out, float* sum, float* inv_std, int64_t rows, int norm, float eps)
{
    /* SkipSimplifiedLayerNormalizationKernel.cs:65-75, Add3 (KernelSimd.cs:160-177) */
    float* t = (float*)malloc(sizeof(float) * (size_t)(norm > 0 ? norm : 1));
    for (int64_t o = 0; o < rows; ++o) {
        const int64_t off = o * norm;
        for (int i = 0; i < norm; ++i) {
            float v = input[off + i] + skip[off + i];
            if (bias) v = v + bias[i];
            t[i] = v;
            if (sum) sum[off + i] = v;
        }
        const float inv = 1.0f / sqrtf(sum_squares(t, norm) / (float)norm + eps);
        if (inv_std) inv_std[o] = inv;
        for (int i = 0; i < norm; ++i) {
            float v = (t[i] * inv) * gamma[i];
            if (beta) v = v + beta[i];
            out[off + i] = v;
        }
    }
    free(t);
}

void msor_silu_mul(const float* g, const float* u, float* y, int64_t n)
{
    /* SigmoidKernel.cs:19-20, then Mul(g, sigmoid(g)) and Mul(., u) */
    for (int64_t i = 0; i < n; ++i) {
        const float s = 1.0f / (1.0f + expf(-g[i]));
        y[i] = (g[i] * s) * u[i];
    }
}

static float dot4(const float* a, const float* b, int n)
{
    /* KernelSimd.cs:43-61: four 8-lane fused accumulators, then one, then the tail */
    float a0[LANES] = {0}, a1[LANES] = {0}, a2[LANES] = {0}, a3[LANES] = {0};
    int i = 0;
    for (; i + 4 * LANES <= n; i += 4 * LANES)
        for (int l = 0; l < LANES; ++l) {
            a0[l] = fmaf(a[i + l], b[i + l], a0[l]);
            a1[l] = fmaf(a[i + LANES + l], b[i + LANES + l], a1[l]);
            a2[l] = fmaf(a[i + 2 * LANES + l], b[i + 2 * LANES + l], a2[l]);
            a3[l] = fmaf(a[i + 3 * LANES + l], b[i + 3 * LANES + l], a3[l]);
        }
    float acc[LANES];
    for (int l = 0; l < LANES; ++l) acc[l] = (a0[l] + a1[l]) + (a2[l] + a3[l]);
    for (; i + LANES <= n; i += LANES)
        for (int l = 0; l < LANES; ++l) acc[l] = fmaf(a[i + l], b[i + l], acc[l]);
    float d = 0.0f;
    for (int l = 0; l < LANES; ++l) d = d + acc[l];
    for (; i < n; ++i) d = d + a[i] * b[i];
    return d;
}

static void rotate(float* row, int pos, const float* cos_c, const float* sin_c, int half, int rot_half,
                   int interleaved)
{
    /* GroupQueryAttentionKernel.cs:330-370 */
    for (int j = 0; j < rot_half; ++j) {
        const float c = cos_c[(int64_t)pos * half + j], s = sin_c[(int64_t)pos * half + j];
        const int i0 = interleaved ? 2 * j : j;
        const int i1 = interleaved ? 2 * j + 1 : j + rot_half;
        const float a = row[i0], b = row[i1];
        row[i0] = a * c - b * s;
        row[i1] = b * c + a * s;
    }
}

void msor_gqa(const msor_gqa_desc* d, const float* q, const float* k, const float* v, const float* past_k,
              const float* past_v, const int32_t* seqlens, const float* cos_c, const float* sin_c, float* out,
              float* present_k, float* present_v)
{
    const int B = d->batch, Sq = d->q_seq, Skv = d->kv_seq, H = d->num_heads, KH = d->kv_num_heads;
    const int D = d->head_dim, past = d->past_seq, total = past + Skv, group = H / KH;
    const int qh = H * D, kvh = KH * D;
    const int q_stride = d->packed_qkv ? qh + 2 * kvh : qh;
    const int kv_stride = d->packed_qkv ? q_stride : kvh;
    const float* kk = d->packed_qkv ? q + qh : k;
    const float* vv = d->packed_qkv ? q + qh + kvh : v;
    const int rot_half = d->do_rotary ? ((2 * d->cos_cols < D ? 2 * d->cos_cols : D) / 2) : 0;
    const float scale = d->scale != 0.0f ? d->scale : 1.0f / sqrtf((float)D);

    /* present = past rows, then the new rows (:239-264), K rotated (:200-210) */
    for (int bg = 0; bg < B * KH; ++bg)
        for (int j = 0; j < past; ++j)
            for (int e = 0; e < D; ++e) {
                present_k[((int64_t)bg * total + j) * D + e] = past_k[((int64_t)bg * past + j) * D + e];
                present_v[((int64_t)bg * total + j) * D + e] = past_v[((int64_t)bg * past + j) * D + e];
            }
    float* row = (float*)malloc(sizeof(float) * (size_t)D);
    for (int b = 0; b < B; ++b)
        for (int s = 0; s < Skv; ++s)
            for (int g = 0; g < KH; ++g) {
                const float* src = kk + (int64_t)(b * Skv + s) * kv_stride + g * D;
                memcpy(row, src, sizeof(float) * (size_t)D);
                if (d->do_rotary) {
                    int pos = past + s;
                    if (pos >= d->cos_rows) pos = d->cos_rows - 1;
                    rotate(row, pos, cos_c, sin_c, d->cos_cols, rot_half, d->rotary_interleaved);
                }
                const int64_t dst = ((int64_t)(b * KH + g) * total + past + s) * D;
                memcpy(present_k + dst, row, sizeof(float) * (size_t)D);
                memcpy(present_v + dst, vv + (int64_t)(b * Skv + s) * kv_stride + g * D, sizeof(float) * (size_t)D);
            }

    /* attention per (b, h, qi) unit (:283-312) */
    float* scores = (float*)malloc(sizeof(float) * (size_t)(total > 0 ? total : 1));
    for (int unit = 0; unit < B * H * Sq; ++unit) {
        const int qi = unit % Sq, hb = unit / Sq, h = hb % H, b = hb / H;
        int bound = total - 1;
        if (d->seqlens_len > 0) {
            const int sb = seqlens[b < d->seqlens_len - 1 ? b : d->seqlens_len - 1];
            if (sb < bound) bound = sb;
        }
        const int g = h / group;
        const int q_abs = past + qi;
        const int k_limit = q_abs < bound ? q_abs : bound;
        const int k_start = d->local_window_size >= 0 ? (q_abs - d->local_window_size + 1 > 0
                                                             ? q_abs - d->local_window_size + 1 : 0)
                                                      : 0;
        memcpy(row, q + (int64_t)(b * Sq + qi) * q_stride + h * D, sizeof(float) * (size_t)D);
        if (d->do_rotary) {
            int pos = q_abs;
            if (pos >= d->cos_rows) pos = d->cos_rows - 1;
            rotate(row, pos, cos_c, sin_c, d->cos_cols, rot_half, d->rotary_interleaved);
        }
        const int64_t kv_base = (int64_t)(b * KH + g) * total * D;
        float mx = -INFINITY;
        for (int j = k_start; j <= k_limit; ++j) {
            const float sc = dot4(row, present_k + kv_base + (int64_t)j * D, D) * scale;
            scores[j] = sc;
            if (sc > mx) mx = sc;
        }
        float sum = 0.0f;
        for (int j = k_start; j <= k_limit; ++j) {
            const float e = expf(scores[j] - mx);
            scores[j] = e;
            sum = sum + e;
        }
        const float inv = sum > 0.0f ? 1.0f / sum : 0.0f;
        float* o = out + (int64_t)(b * Sq + qi) * qh + h * D;
        for (int e = 0; e < D; ++e) o[e] = 0.0f;
        for (int j = k_start; j <= k_limit; ++j) {   /* AxpyInto, KernelSimd.cs:180-193 */
            const float w = scores[j] * inv;
            const float* vr = present_v + kv_base + (int64_t)j * D;
            const int vec = D - D % LANES;   /* fused vector body, unfused scalar tail */
            for (int e = 0; e < vec; ++e) o[e] = fmaf(w, vr[e], o[e]);
            for (int e = vec; e < D; ++e) o[e] = o[e] + w * vr[e];
        }
    }
    free(scores);
    free(row);
}
