/*
 * ms_hip_kernels.h — C ABI of the MI355X (gfx950) MatMulNBits library,
 * libms_hip_nbits.so.
 *
 * The operator: Y[M,N] = A[M,K] * dequant(B)^T with
 *   B       uint8 [N, ceil(K/block_size), block_size*bits/8], codes packed
 *           least-significant first (bits=4: even k in the low nibble);
 *   scales  fp32 [N * ceil(K/block_size)], scales[n*nb + b];
 *   zp      optional uint8 packed like B, row stride ceil(nb*bits/8) bytes,
 *           or NULL for the symmetric default 2^(bits-1);
 *   W[n,k]  = ((float)q - zp) * scale (one fp32 rounding).
 * Semantics follow src/ModelSharp/Cpu/Kernels/Quantize/MatMulNBitsKernel.cs
 * (paths relative to the ModelSharp checkout).
 *
 * Conventions (those of native/ms_kernels.h:7-13, plus a status code):
 *   - fp32 buffers are IEEE binary32, row-major, contiguous;
 *   - pointers are caller-owned; outputs are fully overwritten;
 *   - every entry returns int status, MS_HIP_OK (0) on success; on failure
 *     ms_hip_last_error() (thread-local) holds the message and outputs are
 *     untouched;
 *   - add functions rather than change signatures.
 * Threading: every entry may be called from any host thread. A weights handle's
 * weights are immutable after creation; the synchronous host-pointer entries
 * serialise per handle. Device-pointer entries enqueue on the caller's stream.
 * A handle stays valid until ms_hip_nbits_weights_destroy; entries given any
 * other pointer (a destroyed handle included) return MS_HIP_ERR_INVALID. Destroying
 * a handle while another thread is calling with it is not allowed.
 */
#ifndef MS_HIP_KERNELS_H
#define MS_HIP_KERNELS_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MS_HIP_OK               0
#define MS_HIP_ERR_INVALID      1  /* argument / layout validation failed    */
#define MS_HIP_ERR_NO_DEVICE    2  /* no usable gfx950 device                */
#define MS_HIP_ERR_HIP          3  /* a HIP runtime call failed              */
#define MS_HIP_ERR_UNSUPPORTED  4  /* valid operator input this ABI cannot take */
#define MS_HIP_ERR_DISABLED     5  /* MODELSHARP_HIP=0 (off, false) turned the library off */
#define MS_HIP_ERR_FORCED       6  /* forced failure: MS_HIP_FORCE_FAIL=1 or ms_hip_debug_force_failure */

/* Element types of ms_hip_nbits_weights_create_ex's scales and zero points. */
#define MS_HIP_DTYPE_NONE       0  /* no zero-point tensor (default zero point) */
#define MS_HIP_DTYPE_F32        1
#define MS_HIP_DTYPE_F16        2
#define MS_HIP_DTYPE_U8         3  /* packed codes, as B */

/* ms_hip_nbits_set_tuning value: the handle follows the process default again. */
#define MS_HIP_TUNING_INHERIT   (-2147483647 - 1)

/* ---- capability / diagnostics ---------------------------------------------
 * Replace ms_build_info / ms_has_avx512 / ms_has_vnni
 * (native/ms_kernels.h:23-25, native/src/info.cpp:10-26) for the GPU library:
 * the C# guard probes these before routing (NativeQuant.cs:41-56). */
int         ms_hip_available(void);     /* 1 if a gfx950 device is usable, else 0
                                           (0 also under MODELSHARP_HIP=0)          */
const char* ms_hip_device_name(void);   /* "" when unavailable                    */
const char* ms_hip_build_info(void);
const char* ms_hip_last_error(void);    /* thread-local, "" when none              */

/* Switches (the reference's MODELSHARP_NATIVE / MODELSHARP_NATIVE_QUANT convention,
 * NativeGemm.cs:42-57, NativeQuant.cs:33-56), read once on first use:
 *   MODELSHARP_HIP in {0, off, false}: the library is off — ms_hip_available() returns 0
 *     and every entry that creates weights or computes returns MS_HIP_ERR_DISABLED
 *     without a HIP call;
 *   MS_HIP_FORCE_FAIL in {1, on, true}: those entries return MS_HIP_ERR_FORCED, so a
 *     caller's managed fallback can be exercised on any host.
 * ms_hip_debug_force_failure(on) sets the forced failure at run time (the reference's
 * enable flags are likewise settable for tests, NativeQuant.cs:33-39). Validation
 * (ms_hip_nbits_check), queries and ms_hip_last_error keep working. */
int ms_hip_debug_force_failure(int on);

/* ---- validation ------------------------------------------------------------
 * The operator's input rules, MatMulNBitsKernel.cs:87-145 and :158-161, with
 * the reference's exception messages (returned through ms_hip_last_error).
 * zp_kind: 0 absent, 1 uint8 packed, 2 float32, 3 any other dtype.
 * a_last_dim: A's innermost dimension, or -1 to skip that check. */
int ms_hip_nbits_check(int N, int K, int bits, int block_size,
                       int64_t b_len, int64_t scales_len,
                       int zp_kind, int64_t zp_len, int64_t a_last_dim);

/* ---- load-time weight upload (once per initializer) ------------------------
 * Replaces the per-run widening + upload of IlgpuEngine.RunMatMulNBits
 * (src/ModelSharp.Gpu/IlgpuEngine.cs:2222-2229, ResidentOrTempInt/Float
 * :3392-3429): B, scales and packed zero points are copied once into HBM.
 * Lengths are element counts of the host arrays and are validated as
 * MatMulNBitsKernel.cs:100-139 does. zp may be NULL (zp_len ignored). */
int ms_hip_nbits_weights_create(const uint8_t* bq, int64_t bq_len,
                                const float* scales, int64_t scales_len,
                                const uint8_t* zero_points, int64_t zp_len,
                                int N, int K, int bits, int block_size,
                                void** out_handle);
/* The same with the element types the operator accepts (MatMulNBitsKernel.cs:119-145):
 * scales Float32 or Float16 (q4f16 exports; widened exactly on the device, as
 * GraphContext.Get widens them on the host, GraphContext.cs:106), zero points packed
 * UInt8 (MS_HIP_DTYPE_U8), Float32 or Float16 (zpMode 1 of GpuKernels.cs:578-638, float
 * zero points of MatMulNBitsKernel.cs:239-240; these run the general kernels), or
 * MS_HIP_DTYPE_NONE. Lengths are element counts. */
int ms_hip_nbits_weights_create_ex(const uint8_t* bq, int64_t bq_len,
                                   const void* scales, int64_t scales_len, int scales_type,
                                   const void* zero_points, int64_t zp_len, int zp_type,
                                   int N, int K, int bits, int block_size,
                                   void** out_handle);
/* The load-time path from the model file (OnnxModelLoader.cs:236-431 reads these
 * initializers; :468-511 maps external data): each tensor given as a slice of a file
 * (the .onnx itself for inline raw_data, or an external-data file), streamed from disk
 * into the handle's device buffers through pinned double buffers — no host copy of the
 * weights. dtype: B MS_HIP_DTYPE_U8; scales F32 or F16; zero points U8, F32 or F16
 * (zero_points or its path NULL: none). length is in bytes. */
typedef struct ms_hip_file_slice {
    const char* path;
    int64_t offset;
    int64_t length;
    int dtype;
} ms_hip_file_slice;
int ms_hip_nbits_weights_create_from_files(const ms_hip_file_slice* b, const ms_hip_file_slice* scales,
                                           const ms_hip_file_slice* zero_points,
                                           int N, int K, int bits, int block_size,
                                           void** out_handle);
/* Same, from buffers already resident on the device (copied device-to-device). */
int ms_hip_nbits_weights_create_dev(const uint8_t* d_bq, const float* d_scales,
                                    const uint8_t* d_zero_points,
                                    int N, int K, int bits, int block_size,
                                    void** out_handle);
/* Frees the device copy (IlgpuEngine.Dispose, IlgpuEngine.cs:3926-3942). */
int ms_hip_nbits_weights_destroy(void* handle);
/* N, K, bits, block_size and has-zero-points of a handle (any pointer may be NULL). */
int ms_hip_nbits_weights_info(void* handle, int* N, int* K, int* bits, int* block_size,
                              int* has_zp);

/* ---- the operator ----------------------------------------------------------
 * Host-pointer drop-in: y[M,N] = a[M,K] * dequant(B)^T, synchronous.
 * Replaces ms_qgemm_nbits (native/ms_kernels.h:42-44, qgemm.cpp:77-118) on the
 * path NativeQuant.TryMatMulNBits (NativeQuant.cs:78-115) takes from
 * MatMulNBitsKernel.Execute (MatMulNBitsKernel.cs:174-191), with the weights
 * already resident. M<=16 runs the dequant-fused GEMV (block size 128 and
 * 3 <= M <= 16: its matrix-core form at the same accuracy), larger M the MFMA GEMM.
 * A and Y go through pinned staging buffers owned by the handle: A as a DMA copy;
 * Y stored by the kernel straight into the pinned buffer when A and Y each fit in
 * 1 MiB, else a DMA copy back. */
int ms_hip_nbits_gemm(void* handle, const float* a_host, float* y_host, int M);

/* Device-pointer form: enqueues on `stream` (a hipStream_t, NULL = the null
 * stream) and returns without synchronising. dA: [M,K] fp32, dY: [M,N] fp32,
 * both 16-byte aligned device memory. Prefill calls (M > 16) stage A as fp16 in
 * a workspace owned by the handle (each row scaled by an exact power of two), and
 * launches with few output tiles split K over two workgroups per tile that meet
 * through the handle's per-tile counters and partial-sum slots; the small-M
 * matrix-core kernel splits K over several workgroups per 128-row tile the same
 * way. These buffers grow on demand, never while `stream` is being captured (a
 * call under capture that would need larger ones takes a workspace-free kernel
 * instead), so such calls on one handle from different streams must not overlap.
 * If they do, or a hand-off between the two halves of a split tile does not
 * complete within its bound, the kernel records it in the handle's error word and
 * the output of that call is not valid: the next call on the handle (or
 * ms_hip_nbits_device_error) returns MS_HIP_ERR_HIP and clears the record. */
int ms_hip_nbits_gemm_dev(void* handle, const float* dA, float* dY, int M, void* stream);

/* ms_hip_nbits_gemm_dev with fp16 activations (q4f16 exports): dA16 is [M,K] fp16,
 * widened exactly into the handle's workspace, then the fp32 path runs (the reference
 * widens fp16 inputs, GraphContext.cs:106). Y stays fp32. Needs the workspace to have
 * grown outside stream capture (else MS_HIP_ERR_UNSUPPORTED). */
int ms_hip_nbits_gemm_dev_f16(void* handle, const void* dA16, float* dY, int M, void* stream);

/* Allocation-free form of ms_hip_nbits_gemm_dev, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). No counterpart in the reference. Same arguments, kernels and
 * results as ms_hip_nbits_gemm_dev, with one exception: a call that
 * ms_hip_nbits_gemm_dev would run on mfma_w4_rb (M > 16 prefill) needs the handle's
 * chunk-major scale copy, which the first such eager call builds (an allocation); until
 * one has, this entry runs the call on mfma_w4 (the exact-scale prefill kernel: the same
 * 2e-3 relative Frobenius bar, not bit-identical). The workspace comes from a fixed scratch array
 * that the library holds on each GPU it runs on until the process ends (96 MiB of
 * data and 64 Ki counters; enough for M = 2048 on the Llama-2-7B MLP shapes). A call
 * that needs more returns MS_HIP_ERR_INVALID without launching anything. Every call
 * on one GPU shares that GPU's scratch: calls that overlap on one GPU (other streams,
 * other threads) race, and must not be made. The calling thread's current device must
 * be the handle's. */
int ms_hip_nbits_gemm_dev_noalloc(void* handle, const float* dA, float* dY, int M, void* stream);

/* The device-side failure recorded for this handle since the last check (see
 * ms_hip_nbits_gemm_dev): MS_HIP_ERR_HIP with its message, or MS_HIP_OK. Clears
 * the record. Synchronise the streams of earlier calls first. No counterpart in
 * the reference (its native calls are synchronous). */
int ms_hip_nbits_device_error(void* handle);

/* Enqueues `count` device-pointer calls back to back on `stream`, call i on
 * handles[i] with dA[i], dY[i] (all with the same M). For callers that chain
 * several projections without a host round trip per call. Consecutive decode
 * calls (M <= 4) on the same dA pointer whose weights share K and block size (the
 * projections of one input: q/k/v, gate/up) run as one grouped launch of up to
 * four matrices; results are those of the same calls made one by one, to the
 * decode tolerance. Prefill calls (M > 16) on the same dA pointer, M and K share
 * one fp16 copy of A (made by the first of them; bit-identical results). */
int ms_hip_nbits_gemm_dev_batch(void* const* handles, const float* const* dA,
                                float* const* dY, int count, int M, void* stream);

/* The MLP's gate and up projections of one input and their SiLU-gated product in one
 * call: H = (G * (1 / (1 + exp(-G)))) * U with G = A W_gate^T, U = A W_up^T, the
 * product the reference computes with two MatMulNBits nodes and Sigmoid -> Mul -> Mul
 * (MatMulNBitsKernel.cs:77-265, Activations/SigmoidKernel.cs:13-22, the elementwise Mul),
 * with the same roundings as ms_hip_silu_mul. No single counterpart in the reference:
 * for a decode step (M = 1, both 4-bit with the fast layouts, K and N equal) it is one
 * launch whose workgroups compute the same rows of both projections and store only H,
 * bit-identical to the grouped gate+up launch of ms_hip_nbits_gemm_dev_batch followed
 * by ms_hip_silu_mul; otherwise it runs those steps, with U in the gate handle's
 * workspace (which may grow: not under stream capture before a first eager call). The
 * handles must share K, N and the device (MS_HIP_ERR_INVALID otherwise). */
int ms_hip_nbits_gemm_dev_swiglu(void* gate_handle, void* up_handle, const float* dA, float* dH,
                                 int M, void* stream);
/* Whether ms_hip_nbits_gemm_dev_swiglu with these arguments is the single fused launch
 * (*fused = 1, with its grid and block) or the three-step form (*fused = 0). */
int ms_hip_nbits_swiglu_launch_info(void* gate_handle, void* up_handle, const float* dA, int M,
                                    int* fused, int* grid, int* block);

/* SkipSimplifiedLayerNormalization without beta or bias followed by the projections that
 * read its output, in one call (SkipSimplifiedLayerNormalizationKernel.cs:29-86, then
 * MatMulNBitsKernel.cs:77-265): T = X + Skip (M rows of K, K the handles' common K),
 * Norm = (T * inv) * gamma with inv = 1 / sqrt(mean(T^2) + eps) per row, Y_i = Norm W_i^T.
 * dSum (may be null) receives T, dNorm the normed rows; neither may overlap dX or dSkip,
 * nor may an output dY[i] overlap any of the four (MS_HIP_ERR_INVALID). No single
 * counterpart in the reference. For a decode step (M = 1,
 * up to four 4-bit projections that ms_hip_nbits_gemm_dev_batch would group, 16-byte
 * aligned norm buffers) it is one launch: every workgroup computes the norm in its staging
 * and scales its sums by inv (Y = inv * (T gamma) W^T, the decode tolerance of the batch
 * call); otherwise ms_hip_skip_rmsnorm, then ms_hip_nbits_gemm_dev_batch on dNorm. */
int ms_hip_nbits_gemm_dev_skipnorm(void* const* handles, int count, const float* dX,
                                   const float* dSkip, const float* dGamma, float eps,
                                   float* dNorm, float* dSum, float* const* dY, int M,
                                   void* stream);
/* The same norm followed by ms_hip_nbits_gemm_dev_swiglu on its output: one launch where
 * the SwiGLU call's fused form applies, else the norm and that call. */
int ms_hip_nbits_gemm_dev_skipnorm_swiglu(void* gate_handle, void* up_handle, const float* dX,
                                          const float* dSkip, const float* dGamma, float eps,
                                          float* dNorm, float* dSum, float* dH, int M,
                                          void* stream);
/* Whether the call above (swiglu = 0: ms_hip_nbits_gemm_dev_skipnorm with `count`
 * handles; 1: the SwiGLU form, handles = {gate, up}) with these buffers is the fused
 * launch (*fused = 1, with its grid and block) or the norm and the projections apart. */
int ms_hip_nbits_skipnorm_launch_info(void* const* handles, int count, int swiglu, const float* dX,
                                      const float* dSkip, const float* dGamma, const float* dNorm,
                                      const float* dSum, int M, int* fused, int* grid, int* block);

/* One-shot form with the exact signature semantics of ms_qgemm_nbits
 * (native/ms_kernels.h:42-44): uploads, computes, downloads, frees. */
int ms_hip_qgemm_nbits(const float* a, const uint8_t* bq, const float* scales,
                       const uint8_t* zero_points, float* y,
                       int M, int N, int K, int bits, int block_size);

/* ---- W4A8: the opt-in approximate product (MODELSHARP_W4A8) ------------------
 * Replace ms_qgemm_w4a8 (native/ms_kernels.h:47-53, native/src/qgemm_w4a8.cpp), the
 * kernel NativeQuant.TryMatMulNBits runs when W4A8Enabled (NativeQuant.cs:78-115):
 * activations quantized to int8 per (row, K-block), s_a = max|a| / 127, codes
 * lrint(a / s_a) clamped to [-127, 127]; weight codes code - zp clamped to [-127, 127];
 * int32 block dots; y = sum over blocks, in block order, of (s_a * s_w) * (float)dot.
 * Bit for bit the reference's result (built without floating-point contraction).
 * bits 4 or 8, packed or default zero points (a handle with float zero points returns
 * MS_HIP_ERR_UNSUPPORTED, as the native seam declines them, NativeQuant.cs:87-89).
 * The workspace (M*ceil32(nb*bs) + 4*M*nb + 4*nb*ceil4(M) bytes, each 256-aligned)
 * is the handle's; it cannot grow under stream capture (MS_HIP_ERR_UNSUPPORTED). */
int ms_hip_nbits_gemm_dev_w4a8(void* handle, const float* dA, float* dY, int M, void* stream);
int ms_hip_nbits_gemm_w4a8(void* handle, const float* a_host, float* y_host, int M);
int ms_hip_qgemm_w4a8(const float* a, const uint8_t* bq, const float* scales,
                      const uint8_t* zero_points, float* y,
                      int M, int N, int K, int bits, int block_size);
/* Which W4A8 kernel a call with M rows takes: 9 gemv_w4a8, 10 mfma_w4a8,
 * 11 w4a8_generic; and its grid. */
int ms_hip_nbits_launch_info_w4a8(void* handle, int M, int* kernel_id, int* grid);

/* ---- dequantized weights ---------------------------------------------------
 * W[N,K] fp32 as the device stores it, W[n,k] = ((float)q - zp) * scale
 * (MatMulNBitsSimd.cs:40-111); for the bit-exact dequant check. */
int ms_hip_nbits_dequant(void* handle, float* w_host);
int ms_hip_nbits_dequant_dev(void* handle, float* dW, void* stream);

/* ---- device memory helpers (NativeCuda.Alloc/Upload/Download/Free,
 * src/ModelSharp.Gpu/NativeCuda.cs:92-128) ---------------------------------- */
int ms_hip_alloc(void** dptr, int64_t bytes);
int ms_hip_free(void* dptr);
int ms_hip_upload(void* dptr, const void* host, int64_t bytes);
int ms_hip_download(void* host, const void* dptr, int64_t bytes);
int ms_hip_sync(void);

/* ---- measurement support ---------------------------------------------------
 * No counterpart in the reference; for launch-shape sweeps and tests.
 * ms_hip_set_tuning sets a process-wide default, ms_hip_nbits_set_tuning one
 * handle's own value (MS_HIP_TUNING_INHERIT: follow the default again); a call
 * reads its handle's knobs once, so a sweep on one handle cannot change the kernel
 * another handle's calls take.
 * ms_hip_set_gemv_lanes: lanes per weight row of the gemv_w4_panel kernel
 *   (16, 32 or 64; 0 restores the shape heuristic) — the same as knob 0 below.
 * Knobs (value 0 restores the heuristic):
 *   0 gemv_w4_panel lanes per row;
 *   1 gemv_w4 launch configuration: c+1 forces configuration c of the library's
 *     table (used only where it fits the shape), -1 forces gemv_w4_panel;
 *   2 1 routes every M > 16 call to mfma_w4 (the pipelined prefill off);
 *   3 the pipelined prefill's K split: 1 no tile split, 2 every tile split in two,
 *     3 the second half of the tiles split (needs K >= 256);
 *   4 1 keeps M <= 16 off the small-M matrix-core kernel, 2 sends every eligible
 *     M (1 and 2 included) to it;
 *   5 workgroups per row tile of the small-M matrix-core kernel (1..64, clamped to
 *     [ceil(K / 512), K / 128]);
 *   6 1 keeps M > 16 off the register-operand prefill kernel, 2 sends every eligible
 *     M > 16 to it;
 *   7 its K split (workgroups per 128 x 256 tile, 1..64, clamped to K / 128);
 *   8 polls of the pipelined prefill's split-K flag before the second half of a
 *     tile gives up (0: about 4 million);
 *   9 the register-operand prefill's weight fragments per wave (1, 2 or 4: tiles of
 *     128 x 64, 128 x 128 or 128 x 256 outputs);
 *  10 the host-pointer entries' staging, value - 1 as bits: bit 0 copies A to the
 *     device with a kernel reading the pinned host buffer (else a DMA copy), bit 1
 *     has the GEMM store Y straight into pinned host memory (else a DMA copy back);
 *     0 = the default (Y straight for calls of up to 1 MiB of A and Y, else DMA);
 *  11 the 8-bit GEMV's launch configuration: c+1 forces configuration c (0..8) of the
 *     library's table, -1 sends the 8-bit calls of M <= 4 to gemv_general.
 * ms_hip_nbits_debug_set_counters sets the arrival tag of every split tile of the
 *   handle's pipelined-prefill counters to `value` (or to the tag the next split-K
 *   launch will carry, when next_epoch_tag != 0) and clears their ready flags: it
 *   makes the overlap and time-out reports of ms_hip_nbits_gemm_dev testable with
 *   every kernel still exiting normally.
 * ms_hip_nbits_launch_info reports what a call with M rows would launch:
 *   kernel_id 0 generic, 1 gemv_w4, 2 mfma_w4, 3 gemv_w4_panel, 4 mfma_w4_pipe,
 *   5 skinny_w4, 6 mfma_w4_rb, 7 gemv_general, 8 mfma_general, 12 gemv_w8 (9-11 are
 *   the W4A8 kernels of ms_hip_nbits_launch_info_w4a8); lanes_per_row is the
 *   lanes per weight row of the
 *   GEMV kernels, the output tile width of mfma_w4_rb, 0 otherwise. */
/* ms_hip_nbits_batch_launch_info: what the first launch of a batch call with these
 * handles and activations would be: `calls` = how many of the leading calls it
 * serves, then as ms_hip_nbits_launch_info. */
int ms_hip_nbits_batch_launch_info(void* const* handles, const float* const* dA, int count, int M,
                                   int* calls, int* kernel_id, int* lanes_per_row, int* grid, int* block);
int ms_hip_set_gemv_lanes(int lanes_per_row);
int ms_hip_set_tuning(int knob, int value);
int ms_hip_nbits_set_tuning(void* handle, int knob, int value);
int ms_hip_nbits_debug_set_counters(void* handle, int value, int next_epoch_tag);
int ms_hip_nbits_launch_info(void* handle, int M, int* kernel_id, int* lanes_per_row,
                             int* grid, int* block);

/* ---- decoder-layer neighbours of MatMulNBits ---------------------------------
 * The operators either side of the projections of a Llama-family decoder layer, on
 * device pointers and a stream, so activations stay in HBM from one MatMulNBits to
 * the next (no host copies, nothing allocated). fp32, row-major, 4-byte aligned.
 *
 * SimplifiedLayerNormalization (Cpu/Kernels/Llm/SimplifiedLayerNormalizationKernel.cs:
 * 24-64): rows x norm; inv = 1 / sqrt(sum(x^2) / norm + eps), y = (x * inv) * scale;
 * dInvStd [rows] optional. dY may equal dX. */
int ms_hip_rmsnorm(const float* dX, const float* dScale, float* dY, float* dInvStd,
                   int64_t rows, int norm, float eps, void* stream);
/* SkipSimplifiedLayerNormalization (SkipSimplifiedLayerNormalizationKernel.cs:29-86):
 * t = (input + skip) + bias, out = (t * inv) * gamma + beta; dBeta, dBias, dSum
 * (input_skip_bias_sum, output 3) and dInvStd (output 2) optional. dOut and dSum may
 * equal dInput or dSkip (a residual stream updated in place). */
int ms_hip_skip_rmsnorm(const float* dInput, const float* dSkip, const float* dGamma,
                        const float* dBeta, const float* dBias, float* dOut, float* dSum,
                        float* dInvStd, int64_t rows, int norm, float eps, void* stream);
/* The MLP gate of Llama-family exports, Sigmoid -> Mul -> Mul fused
 * (Activations/SigmoidKernel.cs:13-22 and the elementwise Mul):
 * y = (g * (1 / (1 + exp(-g)))) * u over n elements; dY may equal an input. */
int ms_hip_silu_mul(const float* dGate, const float* dUp, float* dY, int64_t n, void* stream);
/* Elementwise Add of equal shapes (the residual stream), y = a + b; and the unfused
 * Sigmoid (SigmoidKernel.cs:13-22, 1 / (1 + exp(-x))) and Mul of equal shapes. */
int ms_hip_add(const float* dA, const float* dB, float* dY, int64_t n, void* stream);
int ms_hip_sigmoid(const float* dX, float* dY, int64_t n, void* stream);
int ms_hip_mul(const float* dA, const float* dB, float* dY, int64_t n, void* stream);

/* GroupQueryAttention (com.microsoft; Cpu/Kernels/Llm/GroupQueryAttentionKernel.cs).
 * query [batch, q_seq, num_heads*head_dim] (packed_qkv: [batch, q_seq,
 * (num_heads + 2*kv_num_heads)*head_dim] with K and V the row tails, dK/dV unused);
 * key/value [batch, kv_seq, kv_num_heads*head_dim]; past K/V [batch, kv_num_heads,
 * past_seq, head_dim]; present K/V [batch, kv_num_heads, present_capacity, head_dim],
 * rows [0, past_seq + kv_seq) written (past_in_present: the past rows are already
 * there and only the new rows are appended — the cache stays resident); seqlens_k
 * int32 [seqlens_len] on the device (0: none); cos/sin caches [cos_rows, cos_cols]
 * (do_rotary); output [batch, q_seq, num_heads*head_dim]. Causal with the reference's
 * key range min(past + qi, seqlens_k[b]) and local_window_size lower bound; scale 0
 * means 1/sqrt(head_dim). The softmax keeps a unit's (or a key split's) scores in
 * LDS. */
typedef struct ms_hip_gqa_desc {
    int batch, q_seq, kv_seq;
    int num_heads, kv_num_heads, head_dim;
    int packed_qkv;
    int past_seq, past_in_present, present_capacity;
    int do_rotary, rotary_interleaved, cos_rows, cos_cols;
    int local_window_size;
    float scale;
    int seqlens_len;
} ms_hip_gqa_desc;
int ms_hip_gqa_check(const ms_hip_gqa_desc* desc);
/* Bytes of the optional workspace that lets few (batch, head, query) units over a long
 * history split their keys over several workgroups (0: no split for this shape). With
 * a smaller or NULL workspace ms_hip_gqa runs unsplit, or returns MS_HIP_ERR_UNSUPPORTED
 * when one workgroup cannot hold the history's scores. */
int64_t ms_hip_gqa_workspace_size(const ms_hip_gqa_desc* desc);
int ms_hip_gqa(const ms_hip_gqa_desc* desc, const float* dQ, const float* dK, const float* dV,
               const float* dPastK, const float* dPastV, const int32_t* dSeqlensK,
               const float* dCos, const float* dSin, float* dOut,
               float* dPresentK, float* dPresentV, void* dWorkspace, int64_t workspace_bytes,
               void* stream);

#ifdef __cplusplus
}
#endif
#endif
