// ms_hip_nbits.hip — host runtime and C ABI of libms_hip_nbits.so (gfx950).
//
// Weights handles hold B, scales and packed zero points resident in HBM in the
// operator's own layout (uploaded once per initializer); each call dispatches
//   bits=4, block_size in {32,64,128,256}, K % 32 == 0 ("fast" layouts):
//     M <= 16, block_size 128, K % 128 == 0, M >= 3          -> skinny_w4
//     M <= 4, block_size 32 or 128, A panel fits one LDS pass -> gemv_w4
//     M <= 16 otherwise                                       -> gemv_w4_panel
//     M >  16, fp16-safe scales, K % 128 == 0:
//       few output tiles or block_size != 32                  -> a_rows_f16 + mfma_w4_rb
//       otherwise (block_size 32)                             -> a_rows_f16 + mfma_w4_pipe
//     M >  16 otherwise                                       -> mfma_w4 (exact, no workspace)
//   bits=8, packed or no zero points, power-of-two block size >= 16, K % 16 == 0:
//     M <= 4, A panel fits LDS                                -> gemv_w8
//   other formats (bits 8, float zero points, other block sizes or K), K and the block
//   size multiples of 8:
//     M <= 16                                                 -> gemv_general
//     M >  16                                                 -> mfma_general (exact)
//   anything else                                             -> generic
// Declarations and reference citations: include/ms_hip_kernels.h.
#include "../../include/ms_hip_kernels.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <array>
#include <atomic>
#include <climits>
#include <cerrno>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <initializer_list>
#include <mutex>
#include <string>
#include <unordered_set>
#include <utility>
#include <vector>

#include <fcntl.h>
#include <strings.h>
#include <unistd.h>

#include "gemv_general.h"
#include "gemv_w8.h"
#include "gemv_w4.h"
#include "gemv_w4_panel.h"
#include "generic_nbits.h"
#include "mfma_general.h"
#include "w4a8.h"
#include "gqa.h"
#include "mfma_w4.h"
#include "mfma_w4_pipe.h"
#include "mfma_w4_rb.h"
#include "skinny_w4.h"

using namespace msnb;

namespace {

thread_local std::string g_last_error;

int fail(int status, const char* fmt, ...)
{
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return status;
}

#define MS_HIP_CHECK(expr)                                                                  \
    do {                                                                                    \
        hipError_t e_ = (expr);                                                             \
        if (e_ != hipSuccess)                                                               \
            return fail(MS_HIP_ERR_HIP, "[ms_hip] %s failed: %s", #expr, hipGetErrorString(e_)); \
    } while (0)

// ---- device probe ---------------------------------------------------------------------
struct DeviceInfo {
    int ok = 0;
    int device = -1;
    std::string name;
};

const DeviceInfo& device_info()
{
    static DeviceInfo info = [] {
        DeviceInfo d;
        int count = 0;
        if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) {
            (void)hipGetLastError();
            return d;
        }
        hipDeviceProp_t prop;
        for (int i = 0; i < count; ++i) {
            if (hipGetDeviceProperties(&prop, i) != hipSuccess) continue;
            if (std::strncmp(prop.gcnArchName, "gfx950", 6) == 0) {
                d.ok = 1;
                d.device = i;
                d.name = std::string(prop.name) + " (" + prop.gcnArchName + ")";
                break;
            }
        }
        (void)hipGetLastError();
        return d;
    }();
    return info;
}

// ---- switches ---------------------------------------------------------------------------
// MODELSHARP_HIP in {0, off, false} turns the library off for the process (read once, on
// first use, before any HIP call): ms_hip_available() answers 0 and every entry that
// creates weights or computes returns MS_HIP_ERR_DISABLED, as MODELSHARP_NATIVE=0 keeps
// the reference's native library out (NativeGemm.cs:42-57). MS_HIP_FORCE_FAIL in
// {1, on, true}, or ms_hip_debug_force_failure(1), makes those entries fail with
// MS_HIP_ERR_FORCED before touching anything, so a caller's fallback can be tested on any
// host (the reference's switches are settable for tests, NativeQuant.cs:33-39).
bool env_is(const char* name, std::initializer_list<const char*> values)
{
    const char* v = std::getenv(name);
    if (!v) return false;
    for (const char* x : values)
        if (strcasecmp(v, x) == 0) return true;
    return false;
}

bool disabled()
{
    static const bool off = env_is("MODELSHARP_HIP", {"0", "off", "false"});
    return off;
}

std::atomic<int>& forced_failure()
{
    static std::atomic<int> on{env_is("MS_HIP_FORCE_FAIL", {"1", "on", "true"}) ? 1 : 0};
    return on;
}

int gate()
{
    if (disabled()) return fail(MS_HIP_ERR_DISABLED, "[ms_hip] disabled by MODELSHARP_HIP=%s", std::getenv("MODELSHARP_HIP"));
    if (forced_failure().load(std::memory_order_relaxed))
        return fail(MS_HIP_ERR_FORCED, "[ms_hip] forced failure (MS_HIP_FORCE_FAIL / ms_hip_debug_force_failure)");
    return MS_HIP_OK;
}

int require_device()
{
    if (int st = gate()) return st;
    const DeviceInfo& d = device_info();
    if (!d.ok) return fail(MS_HIP_ERR_NO_DEVICE, "[ms_hip] no gfx950 device is available");
    return MS_HIP_OK;
}

// ---- tuning knobs ----------------------------------------------------------------------
// Launch-shape knobs for sweeps and tests (ms_hip_set_tuning: process defaults;
// ms_hip_nbits_set_tuning: one handle). 0 = the shape heuristics below.
//   0 gemv_w4_panel lanes per row          5 skinny_w4 workgroups per row tile
//   1 gemv_w4 configuration (c+1; -1 panel) 6 mfma_w4_rb: 1 off, 2 every eligible M
//   2 1: every M > 16 call to mfma_w4       7 mfma_w4_rb K split
//   3 pipelined prefill K split              8 split-K hand-off poll bound (pipelined)
//   4 skinny_w4: 1 off, 2 every eligible M   9 mfma_w4_rb fragments per wave (1, 2, 4)
//  10 host-pointer staging: bit 0 A by kernel, bit 1 Y straight to pinned host memory
//     (value + 1; 0 = the default for the call's size)
//  11 gemv_w8 configuration (c+1; -1 keeps 8-bit calls on gemv_general)
constexpr int kNumKnobs = 12;
constexpr int kDefaultSpinLimit = 1 << 22;
std::atomic<int> g_knob[kNumKnobs];   // zero-initialised (static storage)

struct Knobs {
    int v[kNumKnobs];
    int panel_lanes() const { return v[0]; }
    int gemv_config() const { return v[1]; }
    int pipe_off() const { return v[2]; }
    int pipe_ksplit() const { return v[3]; }
    int skinny() const { return v[4]; }
    int skinny_ksw() const { return v[5]; }
    int rb() const { return v[6]; }
    int rb_ksw() const { return v[7]; }
    int spin_limit() const { return v[8] > 0 ? v[8] : kDefaultSpinLimit; }
    int rb_nf() const { return v[9]; }
    int host_staging() const { return v[10]; }
    int gemv8_config() const { return v[11]; }
};

int validate_knob(int knob, int value)
{
    bool ok = false;
    switch (knob) {
        case 0: ok = value == 0 || value == 16 || value == 32 || value == 64; break;
        case 1: ok = value >= -1 && value <= kNumGemvConfigs; break;
        case 2: ok = value == 0 || value == 1; break;
        case 3: ok = value >= 0 && value <= 3; break;
        case 4: ok = value >= 0 && value <= 2; break;
        case 5: ok = value >= 0 && value <= 64; break;
        case 6: ok = value >= 0 && value <= 2; break;
        case 7: ok = value >= 0 && value <= 64; break;
        case 8: ok = value >= 0; break;
        case 9: ok = value == 0 || value == 1 || value == 2 || value == 4; break;
        case 10: ok = value >= 0 && value <= 4; break;
        case 11: ok = value >= -1 && value <= kNumGemv8Configs; break;
        default: break;
    }
    return ok ? MS_HIP_OK : fail(MS_HIP_ERR_INVALID, "[ms_hip] invalid tuning knob %d = %d", knob, value);
}

// ---- weights handle --------------------------------------------------------------------
// A workspace: data (fp16 activations, row exponents, split-K partial sums) and
// counters (split-K arrival counters, zero between launches).
struct Ws {
    uint8_t* data = nullptr;
    size_t data_bytes = 0;
    int* cnt = nullptr;
    size_t cnt_ints = 0;
};

struct Weights {
    int N = 0, K = 0, bits = 0, bs = 0, nb = 0, blob = 0, zrb = 0;
    int has_zp = 0;     // packed uint8 zero points in d_zp
    int zp_float = 0;   // float zero points in d_zpf
    int64_t row_bytes = 0;
    int fast = 0;       // gemv_w4 / mfma_w4 eligible
    int log2cpb = 0;    // log2(bs / 32) when fast
    int device = 0;
    uint8_t* d_b = nullptr;
    float* d_scales = nullptr;
    uint8_t* d_zp = nullptr;
    float* d_zpf = nullptr;     // float zero points [N * nb]
    int* d_wexp = nullptr;      // general formats: row exponents of the weights [N]
    // mfma_w4_rb's chunk-major scales / zero points [K / 128][N][4], built by the first
    // eager call that takes it (rb_ready then 1; guarded by ws_mu)
    uint32_t* d_sz4 = nullptr;
    std::atomic<int> rb_ready{0};
    std::atomic<int> knob[kNumKnobs];   // MS_HIP_TUNING_INHERIT: the process default
    // Device-side failure report: a split-K hand-off that gives up writes a nonzero code
    // here (pinned host memory the kernels write through d_err); calls check and clear it.
    int* h_err = nullptr;
    int* d_err = nullptr;
    // synchronous host-pointer path: device and pinned host staging + stream, guarded by mu
    std::mutex mu;
    hipStream_t stream = nullptr;
    float* d_stage = nullptr;
    size_t stage_bytes = 0;
    uint8_t* h_stage = nullptr;
    size_t h_stage_bytes = 0;
    // prefill kernels: scales fp16-safe (checked at load)
    int pipe_scales_ok = 0;
    // workspace, grown on demand under ws_mu (never while the launch stream is captured)
    std::mutex ws_mu;
    Ws ws;
};

Knobs knobs_of(const Weights& w)
{
    Knobs k;
    for (int i = 0; i < kNumKnobs; ++i) {
        const int h = w.knob[i].load(std::memory_order_relaxed);
        k.v[i] = h != MS_HIP_TUNING_INHERIT ? h : g_knob[i].load(std::memory_order_relaxed);
    }
    return k;
}

// Live handles: a handle is valid from create until destroy; calls with any other
// pointer fail instead of reading freed memory.
std::mutex g_live_mu;
std::unordered_set<const void*> g_live;

Weights* from_handle(void* h)
{
    std::lock_guard<std::mutex> lock(g_live_mu);
    return h && g_live.count(h) ? static_cast<Weights*>(h) : nullptr;
}

// Split-K launch tags: nonzero, distinct for launches that could overlap.
std::atomic<uint32_t> g_epoch{0};
int next_epoch() { return (int)(g_epoch.fetch_add(1, std::memory_order_relaxed) % 0x7FFFFFFEu) + 1; }

void derive_layout(Weights& w, int N, int K, int bits, int bs)
{
    w.N = N;
    w.K = K;
    w.bits = bits;
    w.bs = bs;
    w.nb = (K + bs - 1) / bs;
    w.blob = (bs * bits + 7) / 8;
    w.zrb = (w.nb * bits + 7) / 8;
    w.row_bytes = (int64_t)w.nb * w.blob;
    w.fast = 0;
    // The fast kernels address B, scales and zero points with 32-bit buffer offsets.
    const bool fits = (int64_t)N * w.row_bytes <= INT32_MAX && (int64_t)N * w.nb * 4 <= INT32_MAX;
    if (bits == 4 && fits && (K % 32) == 0 && (bs == 32 || bs == 64 || bs == 128 || bs == 256)) {
        w.fast = 1;
        w.log2cpb = bs == 32 ? 0 : bs == 64 ? 1 : bs == 128 ? 2 : 3;
    }
}

RawLayout raw_layout(const Weights& w)
{
    RawLayout L;
    L.b = w.d_b;
    L.scales = w.d_scales;
    L.zp = w.has_zp ? w.d_zp : nullptr;
    L.zpf = w.zp_float ? w.d_zpf : nullptr;
    L.N = w.N;
    L.K = w.K;
    L.bits = w.bits;
    L.bs = w.bs;
    L.nb = w.nb;
    L.blob = w.blob;
    L.zrb = w.zrb;
    return L;
}

void free_weights(Weights& w)
{
    if (w.d_b) (void)hipFree(w.d_b);
    if (w.d_scales) (void)hipFree(w.d_scales);
    if (w.d_sz4) (void)hipFree(w.d_sz4);
    if (w.d_zp) (void)hipFree(w.d_zp);
    if (w.d_zpf) (void)hipFree(w.d_zpf);
    if (w.d_wexp) (void)hipFree(w.d_wexp);
    if (w.d_stage) (void)hipFree(w.d_stage);
    if (w.h_stage) (void)hipHostFree(w.h_stage);
    if (w.h_err) (void)hipHostFree(w.h_err);
    if (w.ws.data) (void)hipFree(w.ws.data);
    if (w.ws.cnt) (void)hipFree(w.ws.cnt);
    if (w.stream) (void)hipStreamDestroy(w.stream);
    w.d_b = nullptr;
    w.d_scales = nullptr;
    w.d_zp = nullptr;
    w.d_zpf = nullptr;
    w.d_wexp = nullptr;
    w.d_stage = nullptr;
    w.stage_bytes = 0;
    w.h_stage = nullptr;
    w.h_stage_bytes = 0;
    w.h_err = nullptr;
    w.d_err = nullptr;
    w.ws = Ws{};
    w.stream = nullptr;
}

// Smallest nonzero and largest |scale| bit patterns (positive floats order as integers):
// a reduction per workgroup, then one atomic pair per workgroup.
__global__ __launch_bounds__(256) void scale_range_kernel(const float* __restrict__ s, int64_t n, unsigned* out)
{
    __shared__ unsigned red[2][4];
    unsigned lo = 0xFFFFFFFFu, hi = 0u;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const unsigned b = __builtin_bit_cast(unsigned, s[i]) & 0x7FFFFFFFu;
        if (b) {
            lo = min(lo, b);
            hi = max(hi, b);
        }
    }
    for (int o = 32; o > 0; o >>= 1) {
        lo = min(lo, (unsigned)__shfl_xor((int)lo, o));
        hi = max(hi, (unsigned)__shfl_xor((int)hi, o));
    }
    const int wave = threadIdx.x / kWave;
    if ((threadIdx.x & (kWave - 1)) == 0) {
        red[0][wave] = lo;
        red[1][wave] = hi;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; ++w) {
            lo = min(lo, red[0][w]);
            hi = max(hi, red[1][w]);
        }
        atomicMin(&out[0], lo);
        atomicMax(&out[1], hi);
    }
}

// Zero fill of n ints (counters), a kernel rather than a memset so that it can sit in
// a captured graph.
__global__ __launch_bounds__(256) void zero_ints_kernel(int* __restrict__ p, int64_t n)
{
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        p[i] = 0;
}

int zero_ints(int* p, int64_t n, hipStream_t stream)
{
    if (n <= 0) return MS_HIP_OK;
    hipLaunchKernelGGL(zero_ints_kernel, dim3((unsigned)std::min<int64_t>((n + 255) / 256, 256)), dim3(256), 0,
                       stream, p, n);
    MS_HIP_CHECK(hipGetLastError());
    return MS_HIP_OK;
}

// The fp16 prefill kernels round scales to fp16 and form (q - zp) * s in fp16: every
// nonzero |s| must be an fp16 normal (>= 2^-14) and max|q - zp| |s| (15, or 255 for 8-bit
// codes) must stay below 65504.
int check_pipe_scales(Weights& w)
{
    w.pipe_scales_ok = 0;
    if (!w.fast && !(w.bits == 8 && !w.zp_float)) return MS_HIP_OK;
    unsigned* d = nullptr;
    MS_HIP_CHECK(hipMalloc(&d, 2 * sizeof(unsigned)));
    const unsigned init[2] = {0xFFFFFFFFu, 0u};
    hipError_t e = hipMemcpy(d, init, sizeof init, hipMemcpyHostToDevice);
    const int64_t n = (int64_t)w.N * w.nb;
    if (e == hipSuccess) {
        hipLaunchKernelGGL(scale_range_kernel, dim3((unsigned)std::min<int64_t>((n + 255) / 256, 1024)), dim3(256), 0,
                           nullptr, w.d_scales, n, d);
        e = hipGetLastError();
    }
    unsigned r[2] = {0u, 0u};
    if (e == hipSuccess) e = hipMemcpy(r, d, sizeof r, hipMemcpyDeviceToHost);
    (void)hipFree(d);
    if (e != hipSuccess) return fail(MS_HIP_ERR_HIP, "[ms_hip] scale range check failed: %s", hipGetErrorString(e));
    const unsigned kMinNormal16 = 0x38800000u;   // 2^-14
    const unsigned kMaxScale = w.bits == 8 ? 0x43800000u    // 256.0: 255 * s < 65504
                                           : 0x45886000u;   // 4364.0: 15 * s < 65504
    w.pipe_scales_ok = (r[0] == 0xFFFFFFFFu) || (r[0] >= kMinNormal16 && r[1] <= kMaxScale);
    return MS_HIP_OK;
}

// A device-side failure recorded in the handle's error word since the last check (the
// split-K hand-off of a pipelined prefill launch that gave up): clears it, zeroes the
// workspace counters on `stream` and returns MS_HIP_ERR_HIP; MS_HIP_OK otherwise.
int take_device_error(Weights& w, hipStream_t stream)
{
    if (!w.h_err) return MS_HIP_OK;
    const int code = __atomic_exchange_n(w.h_err, 0, __ATOMIC_ACQ_REL);
    if (!code) return MS_HIP_OK;
    {
        std::lock_guard<std::mutex> lock(w.ws_mu);
        if (w.ws.cnt) (void)zero_ints(w.ws.cnt, (int64_t)w.ws.cnt_ints, stream);
    }
    return fail(MS_HIP_ERR_HIP,
                code == kPipeErrOverlap
                    ? "[ms_hip] split-K prefill: another launch was using this workspace (overlapping calls on one "
                      "handle); the output of that call is not valid"
                    : "[ms_hip] split-K prefill: a partial-sum hand-off timed out; the output of that call is not valid");
}

// Grows the handle's workspace to at least (data_bytes, cnt_ints) — new counters are
// zeroed on `stream`. Returns 1 with *out set, 0 when it would have to grow while `stream`
// is being captured (the caller takes a workspace-free kernel), -1 on a HIP error.
int ensure_ws(Weights& w, size_t data_bytes, size_t cnt_ints, hipStream_t stream, Ws* out)
{
    std::lock_guard<std::mutex> lock(w.ws_mu);
    const bool grow_d = w.ws.data_bytes < data_bytes, grow_c = w.ws.cnt_ints < cnt_ints;
    if (grow_d || grow_c) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(stream, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) {
            (void)hipGetLastError();
            return 0;
        }
        // Earlier launches on this stream may still use the old buffers.
        if (hipStreamSynchronize(stream) != hipSuccess) return -1;
    }
    if (grow_d) {
        if (w.ws.data && hipFree(w.ws.data) != hipSuccess) return -1;
        w.ws.data = nullptr;
        w.ws.data_bytes = 0;
        if (hipMalloc(&w.ws.data, data_bytes) != hipSuccess) return -1;
        w.ws.data_bytes = data_bytes;
    }
    if (grow_c) {
        if (w.ws.cnt && hipFree(w.ws.cnt) != hipSuccess) return -1;
        w.ws.cnt = nullptr;
        w.ws.cnt_ints = 0;
        if (hipMalloc(&w.ws.cnt, cnt_ints * sizeof(int)) != hipSuccess) return -1;
        w.ws.cnt_ints = cnt_ints;
        // Every launch leaves its counters zero again; they start zero here.
        if (zero_ints(w.ws.cnt, (int64_t)cnt_ints, stream) != MS_HIP_OK) return -1;
    }
    *out = w.ws;
    return 1;
}

constexpr size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

// ---- GEMV launch shape --------------------------------------------------------------------
// gemv_w4 instantiations: [M-1][L slot][config], L slot 0 = block size 32, 1 = block size 128.
typedef void (*GemvFn)(GemvParams);
template <int M, int L, size_t I>
constexpr GemvFn gemv_fn_at()
{
    constexpr GemvConfig c = kGemvConfigs[I];
    return gemv_w4_kernel<M, c.G, c.KW, c.U, L, c.waves, c.RL, c.NB>;
}
template <int M, int L, size_t... I>
constexpr std::array<GemvFn, sizeof...(I)> gemv_row(std::index_sequence<I...>)
{
    return {gemv_fn_at<M, L, I>()...};
}
template <int M, int L>
constexpr std::array<GemvFn, kNumGemvConfigs> gemv_row()
{
    return gemv_row<M, L>(std::make_index_sequence<kNumGemvConfigs>{});
}
const std::array<GemvFn, kNumGemvConfigs> kGemvTable[kGemvMaxM][2] = {
    {gemv_row<1, 0>(), gemv_row<1, 2>()},
    {gemv_row<2, 0>(), gemv_row<2, 2>()},
    {gemv_row<3, 0>(), gemv_row<3, 2>()},
    {gemv_row<4, 0>(), gemv_row<4, 2>()},
};
std::atomic<bool> g_gemv_lds_raised[kGemvMaxM][2][kNumGemvConfigs];

// The SwiGLU form of gemv_w4 (gate and up of one input, their SiLU-Mul stored), M = 1:
// [L slot][config], null for configs whose row-waves do not split in two.
template <int L, size_t I>
constexpr GemvFn gemv_sw_fn_at()
{
    constexpr GemvConfig c = kGemvConfigs[I];
    if constexpr ((c.waves / c.KW) % 2 == 0)
        return gemv_w4_kernel<1, c.G, c.KW, c.U, L, c.waves, c.RL, c.NB, true>;
    else
        return nullptr;
}
template <int L, size_t... I>
constexpr std::array<GemvFn, sizeof...(I)> gemv_sw_row(std::index_sequence<I...>)
{
    return {gemv_sw_fn_at<L, I>()...};
}
const std::array<GemvFn, kNumGemvConfigs> kGemvSwTable[2] = {
    gemv_sw_row<0>(std::make_index_sequence<kNumGemvConfigs>{}),
    gemv_sw_row<2>(std::make_index_sequence<kNumGemvConfigs>{}),
};
std::atomic<bool> g_gemv_sw_lds_raised[2][kNumGemvConfigs];

// The same two forms with the SkipRMSNorm prologue (NORM, M = 1): [L slot][config].
template <int L, size_t I, bool SW>
constexpr GemvFn gemv_norm_fn_at()
{
    constexpr GemvConfig c = kGemvConfigs[I];
    if constexpr (SW && (c.waves / c.KW) % 2 != 0)
        return nullptr;
    else
        return gemv_w4_kernel<1, c.G, c.KW, c.U, L, c.waves, c.RL, c.NB, SW, true>;
}
template <int L, bool SW, size_t... I>
constexpr std::array<GemvFn, sizeof...(I)> gemv_norm_row(std::index_sequence<I...>)
{
    return {gemv_norm_fn_at<L, I, SW>()...};
}
const std::array<GemvFn, kNumGemvConfigs> kGemvNormTable[2][2] = {   // [SW][L slot]
    {gemv_norm_row<0, false>(std::make_index_sequence<kNumGemvConfigs>{}),
     gemv_norm_row<2, false>(std::make_index_sequence<kNumGemvConfigs>{})},
    {gemv_norm_row<0, true>(std::make_index_sequence<kNumGemvConfigs>{}),
     gemv_norm_row<2, true>(std::make_index_sequence<kNumGemvConfigs>{})},
};
std::atomic<bool> g_gemv_norm_lds_raised[2][2][kNumGemvConfigs];

// The SkipRMSNorm that a NORM launch computes in its staging.
struct NormArgs {
    const float* x;
    const float* skip;
    const float* gamma;
    float* sum;   // x + skip, or nullptr
    float* out;   // the normed activations
    float eps;
};

// Output rows of one gemv_w4 workgroup.
constexpr int gemv_rows(const GemvConfig& c) { return (kWave / c.G) * (c.waves / c.KW) * c.RL; }

int l_slot(const Weights& w) { return w.log2cpb == 0 ? 0 : w.log2cpb == 2 ? 1 : -1; }

// gemv_w4 takes M <= 4, block size 32 or 128, and A panels that one thread per
// chunk stages in LDS (M * C <= 64 * waves).
bool gemv_config_fits(const Weights& w, int M, const GemvConfig& c)
{
    return M <= kGemvMaxM && l_slot(w) >= 0 && M * (w.K / 32) <= 64 * c.waves;
}

// Config choice: the first config of a preference list that fits the shape and gives
// every lane at least 2 steps. The lists come from sweeping every config over the
// 7B and Qwen2.5-0.5B decode launches on MI355X (M = 1, 2, 4; single matrices and
// groups of one input's projections): for M <= 2, two rows per lane at 16 lanes per
// row win from 16K rows up, 64 lanes per row with two rows per lane from 2K to 16K rows
// (re-swept with the non-temporal code loads: 7B o at M = 1 / 2 5.41 -> 5.26 /
// 6.83 -> 6.54 us against the 32-lane pick), 32 lanes per row below; for M = 3-4 the
// 8-wave configs. From 2K to 4K rows at M <= 2, 8 waves of 64 lanes per row with two rows
// per lane (7B q / o, 3584 x 3584: M = 1 / 2 5.27 -> 5.14 / 6.62 -> 6.12 us), and the
// same 8-wave config from 8K to 16K rows (Llama-2-7B up, K = 4096, N = 11008, bs 128,
// no zero points: M = 1 / 2 9.61 -> 8.89 / 12.87 -> 11.03 us). N is the launch's total
// rows (summed over a group). Indices are into kGemvConfigs.
int pick_gemv_config(const Weights& w, const Knobs& kn, int M, int N)
{
    if (kn.gemv_config() < 0) return -1;
    if (kn.gemv_config() > 0) {
        const int ci = kn.gemv_config() - 1;
        return gemv_config_fits(w, M, kGemvConfigs[ci]) ? ci : -1;
    }
    static constexpr int kLargeM2[] = {16, 11, 0, 6};   // M <= 2, N >= 16384
    static constexpr int kUpperM2[] = {17, 14, 11, 2};  // M <= 2, N >= 8192
    static constexpr int kMidM2[] = {14, 11, 2};        // M <= 2, N >= 4096
    static constexpr int kSmallM2[] = {17, 14, 13, 6};  // M <= 2, N >= 2048
    static constexpr int kTinyM2[] = {3, 14, 8};        // M <= 2
    static constexpr int kLargeM4[] = {7, 6, 0};        // M <= 4, N >= 16384
    static constexpr int kMidM4[] = {15, 7, 8};         // M <= 4, N >= 4096
    static constexpr int kSmallM4[] = {6, 8, 0};        // M <= 4
    static constexpr int kWide[] = {18, 9, 10};         // panels that need 16 waves to stage
    const int C = w.K / 32;
    auto usable = [&](int ci) {
        const GemvConfig& c = kGemvConfigs[ci];
        return gemv_config_fits(w, M, c) && C > c.G * c.KW;   // >= 2 steps per lane
    };
    auto first_of = [&](const int* list, int len) {
        for (int i = 0; i < len; ++i)
            if (usable(list[i])) return list[i];
        return -1;
    };
    int ci;
    if (M <= 2)
        ci = N >= 16384 ? first_of(kLargeM2, 4) : N >= 8192 ? first_of(kUpperM2, 4)
           : N >= 4096  ? first_of(kMidM2, 3)
           : N >= 2048  ? first_of(kSmallM2, 4) : first_of(kTinyM2, 3);
    else
        ci = N >= 16384 ? first_of(kLargeM4, 3) : N >= 4096 ? first_of(kMidM4, 3) : first_of(kSmallM4, 3);
    if (ci < 0) ci = first_of(kWide, 3);
    if (ci < 0) {   // short rows (a lane gets a single step): any config that fits
        for (int i = 0; i < kNumGemvConfigs && ci < 0; ++i)
            if (gemv_config_fits(w, M, kGemvConfigs[i])) ci = i;
    }
    return ci;
}

// One gemv_w4 launch over `n` weight matrices (1 <= n <= kGemvMaxOps) that share A,
// K and the block size: member i's rows take workgroups after member i-1's.
struct GemvMember {
    const Weights* w;
    float* dY;
};

void set_norm(GemvParams& p, const NormArgs* na)
{
    p.nx = na ? na->x : nullptr;
    p.nskip = na ? na->skip : nullptr;
    p.ngamma = na ? na->gamma : nullptr;
    p.nsum = na ? na->sum : nullptr;
    p.nout = na ? na->out : nullptr;
    p.neps = na ? na->eps : 0.0f;
}

// A NORM launch stages two half chunks per thread: 2 C <= threads.
bool norm_fits(const GemvConfig& c, int K) { return 2 * (K / 32) <= c.waves * kWave; }

int launch_gemv_group(const GemvMember* mem, int n, const float* dA, int M, int ci, hipStream_t stream,
                      const NormArgs* na = nullptr)
{
    const Weights& w0 = *mem[0].w;
    const GemvConfig& c = kGemvConfigs[ci];
    const int ls = l_slot(w0);
    GemvFn fn = na ? kGemvNormTable[0][ls][ci] : kGemvTable[M - 1][ls][ci];
    const int rows = gemv_rows(c);
    const size_t lds = (size_t)M * (w0.K / 32) * kChunkStride4 * 16;
    std::atomic<bool>& raised = na ? g_gemv_norm_lds_raised[0][ls][ci] : g_gemv_lds_raised[M - 1][ls][ci];
    if (lds > 64 * 1024 && !raised.load()) {
        MS_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        raised.store(true);
    }
    GemvParams p;
    set_norm(p, na);
    int first = 0;
    for (int i = 0; i < kGemvMaxOps; ++i) {
        const GemvMember& m = mem[std::min(i, n - 1)];   // unused entries repeat the last member
        p.op[i].b = m.w->d_b;
        p.op[i].scales = m.w->d_scales;
        p.op[i].zp = m.w->has_zp ? m.w->d_zp : nullptr;
        p.op[i].y = m.dY;
        p.op[i].N = m.w->N;
        p.op[i].first = first;
        if (i < n) first += (m.w->N + rows - 1) / rows;
    }
    p.nops = n;
    p.a = dA;
    p.row_bytes = (int)w0.row_bytes;
    p.K = w0.K;
    p.C = w0.K / 32;
    p.nb = w0.nb;
    p.zrb = w0.zrb;
    hipLaunchKernelGGL(fn, dim3(first), dim3(c.waves * kWave), lds, stream, p);
    MS_HIP_CHECK(hipGetLastError());
    return MS_HIP_OK;
}

bool gemv_groupable(const Weights& a, const Weights& b);

// The fused SwiGLU launch: M = 1, gate and up groupable on gemv_w4 with the same N, and the
// config the grouped launch of the two would take splits its row-waves in two. *ci
// receives that config.
bool swiglu_fused_config(const Weights& wg, const Weights& wu, const float* dA, int M, int* ci)
{
    if (M != 1 || !dA || (reinterpret_cast<uintptr_t>(dA) & 15) || !gemv_groupable(wg, wu) || wg.N != wu.N)
        return false;
    const int c = pick_gemv_config(wg, knobs_of(wg), 1, 2 * wg.N);
    if (c < 0 || !kGemvSwTable[l_slot(wg)][c]) return false;
    *ci = c;
    return true;
}

int launch_gemv_swiglu(const Weights& wg, const Weights& wu, const float* dA, float* dH, int ci, hipStream_t stream,
                       const NormArgs* na = nullptr)
{
    const GemvConfig& c = kGemvConfigs[ci];
    const int ls = l_slot(wg);
    GemvFn fn = na ? kGemvNormTable[1][ls][ci] : kGemvSwTable[ls][ci];
    const int rows = gemv_rows(c) / 2;   // of each projection per workgroup
    const size_t lds = (size_t)(wg.K / 32) * kChunkStride4 * 16;
    std::atomic<bool>& raised = na ? g_gemv_norm_lds_raised[1][ls][ci] : g_gemv_sw_lds_raised[ls][ci];
    if (lds > 64 * 1024 && !raised.load()) {
        MS_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        raised.store(true);
    }
    const int grid = (wg.N + rows - 1) / rows;
    GemvParams p;
    set_norm(p, na);
    const Weights* mem[2] = {&wg, &wu};
    for (int i = 0; i < kGemvMaxOps; ++i) {
        const Weights& m = *mem[std::min(i, 1)];
        p.op[i].b = m.d_b;
        p.op[i].scales = m.d_scales;
        p.op[i].zp = m.has_zp ? m.d_zp : nullptr;
        p.op[i].y = dH;
        p.op[i].N = m.N;
        p.op[i].first = 0;
    }
    p.nops = 2;
    p.a = dA;
    p.row_bytes = (int)wg.row_bytes;
    p.K = wg.K;
    p.C = wg.K / 32;
    p.nb = wg.nb;
    p.zrb = wg.zrb;
    hipLaunchKernelGGL(fn, dim3(grid), dim3(c.waves * kWave), lds, stream, p);
    MS_HIP_CHECK(hipGetLastError());
    return MS_HIP_OK;
}

// Members that one gemv_w4 launch can serve together: same device, 4-bit fast layout,
// K and block size (hence row_bytes, nb and zrb).
bool gemv_groupable(const Weights& a, const Weights& b)
{
    return a.device == b.device && a.fast && b.fast && a.bits == 4 && b.bits == 4 && a.K == b.K &&
           a.log2cpb == b.log2cpb && l_slot(a) >= 0;
}

bool skinny_eligible(const Weights& w, const Knobs& kn, int M);

// How many of the calls starting at handles[0] one launch serves: consecutive calls on
// the same activations (the projections of one input) that gemv_w4 can group, up to
// kGemvMaxOps; 1 when the first call launches alone. *ci receives the group's config
// (the first handle's knobs decide it).
int batch_group(Weights* const* ws, const float* const* dA, int count, int M, int* ci)
{
    const Weights* w = ws[0];
    const Knobs kn = knobs_of(*w);
    if (M <= 0 || M > kGemvMaxM || !dA[0] || (reinterpret_cast<uintptr_t>(dA[0]) & 15)) return 1;
    // Block size 128 takes the matrix-core small-M path per matrix from M = 3, and so do the
    // large matrices of other block sizes from M = 4 (7B gate and up, bs 32, M = 4: two
    // launches of 19.3 us against 41.8 us grouped on gemv_w4; at M = 3 the grouped launch
    // is faster, 35.1 against 2 x 19.0 us). Otherwise the projections of one input group on
    // gemv_w4 where its panel fits (7B q+k+v, bs 32, M = 3 / 4: 10.5 / 12.0 us grouped
    // against 27.9 / 28.4 us as three matrix-core launches; the small k and v leave that
    // kernel's row tiles too few).
    if (skinny_eligible(*w, kn, M) && (w->log2cpb == 2 || (M >= 4 && w->N >= 8192))) return 1;
    int n = 1, ntot = w->N;
    while (n < count && n < kGemvMaxOps && dA[n] == dA[0] && gemv_groupable(*w, *ws[n])) {
        ntot += ws[n]->N;
        ++n;
    }
    if (n == 1) return 1;
    *ci = pick_gemv_config(*w, kn, M, ntot);
    return *ci >= 0 ? n : 1;
}

// ---- gemv_w4_panel: M <= 16, any fast block size, A staged in LDS panels ---------------
constexpr int kPanelMaxM = 16;
constexpr int kPanelLanes[3] = {16, 32, 64};

// Lanes per row G: lane efficiency on the row's C chunks x wave fill (>= 1024
// waves) x a penalty when a lane owns fewer than 3 chunks; ties go to the larger G.
int pick_panel_lanes(const Knobs& kn, int N, int C)
{
    if (kn.panel_lanes()) return kn.panel_lanes();
    double best = -1.0;
    int best_g = 16;
    for (int G : kPanelLanes) {
        const int R = kWave / G;
        const double waves = (double)((N + R - 1) / R);
        const int steps = (C + G - 1) / G;
        const double eff = (double)C / (double)(steps * G);
        const double fill = std::min(1.0, waves / 1024.0);
        const double per_lane = (double)C / G < 3.0 ? 0.85 : 1.0;
        const double score = eff * fill * per_lane;
        if (score >= best - 1e-9) {
            best = score;
            best_g = G;
        }
    }
    return best_g;
}

typedef void (*PanelFn)(GemvPanelParams);
template <int M>
PanelFn panel_for_lanes(int G)
{
    switch (G) {
        case 16: return gemv_w4_panel_kernel<M, 16>;
        case 32: return gemv_w4_panel_kernel<M, 32>;
        default: return gemv_w4_panel_kernel<M, 64>;
    }
}

template <size_t... I>
constexpr std::array<PanelFn (*)(int), sizeof...(I)> panel_table(std::index_sequence<I...>)
{
    return {panel_for_lanes<(int)I + 1>...};
}
constexpr auto kPanelTable = panel_table(std::make_index_sequence<kPanelMaxM>{});

struct PanelShape {
    int G, grid, panel_chunks;
    size_t lds_bytes;
};

PanelShape panel_shape(const Weights& w, const Knobs& kn, int M)
{
    PanelShape s;
    const int C = w.K / 32;
    s.G = pick_panel_lanes(kn, w.N, C);
    const int rows_per_wg = (kPanelThreads / kWave) * (kWave / s.G);
    s.grid = (w.N + rows_per_wg - 1) / rows_per_wg;
    // LDS panel: <= 40 KiB for M <= 4 (4 workgroups per CU), <= 64 KiB beyond.
    const size_t budget = M <= 4 ? 40 * 1024 : 64 * 1024;
    const int bytes_per_chunk = M * kChunkStride4 * 16;
    int pmax = (int)(budget / bytes_per_chunk);
    if (pmax < 1) pmax = 1;
    const int npanels = (C + pmax - 1) / pmax;
    int P = (C + npanels - 1) / npanels;
    if (P % s.G) {
        const int up = ((P + s.G - 1) / s.G) * s.G;
        if (up <= pmax) P = up;
    }
    s.panel_chunks = P;
    s.lds_bytes = (size_t)M * P * kChunkStride4 * 16;
    return s;
}

int launch_panel(const Weights& w, const Knobs& kn, const float* dA, float* dY, int M, hipStream_t stream)
{
    const PanelShape s = panel_shape(w, kn, M);
    GemvPanelParams p;
    p.b = w.d_b;
    p.scales = w.d_scales;
    p.zp = w.has_zp ? w.d_zp : nullptr;
    p.a = dA;
    p.y = dY;
    p.row_bytes = (int)w.row_bytes;
    p.N = w.N;
    p.K = w.K;
    p.C = w.K / 32;
    p.log2cpb = w.log2cpb;
    p.nb = w.nb;
    p.zrb = w.zrb;
    p.panel_chunks = s.panel_chunks;
    hipLaunchKernelGGL(kPanelTable[M - 1](s.G), dim3(s.grid), dim3(kPanelThreads), s.lds_bytes, stream, p);
    MS_HIP_CHECK(hipGetLastError());
    return MS_HIP_OK;
}

int launch_gemv(const Weights& w, const Knobs& kn, const float* dA, float* dY, int M, hipStream_t stream)
{
    const int ci = pick_gemv_config(w, kn, M, w.N);
    if (ci >= 0) {
        const GemvMember m{&w, dY};
        return launch_gemv_group(&m, 1, dA, M, ci, stream);
    }
    return launch_panel(w, kn, dA, dY, M, stream);
}

// The general kernels take K and the block size multiples of 8 (8-code groups lie in one
// block and start at 4-byte aligned codes).
bool general_eligible(const Weights& w)
{
    return (w.K % 8) == 0 && (w.bs % 8) == 0 && (int64_t)w.N * w.nb * w.blob < ((int64_t)1 << 40);
}

typedef void (*GenGemvFn)(RawLayout, const float*, float*);
template <size_t... I>
constexpr std::array<GenGemvFn, sizeof...(I)> gen_gemv_table(std::index_sequence<I...>)
{
    return {gemv_general_kernel<(int)I + 1>...};
}
constexpr auto kGenGemvTable = gen_gemv_table(std::make_index_sequence<16>{});

int launch_gemv_general(const Weights& w, const float* dA, float* dY, int M, hipStream_t stream)
{
    hipLaunchKernelGGL(kGenGemvTable[M - 1], dim3((w.N + kGenRowsPerWg - 1) / kGenRowsPerWg), dim3(256), 0, stream,
                       raw_layout(w), dA, dY);
    MS_HIP_CHECK(hipGetLastError());
    return MS_HIP_OK;
}

// ---- gemv_w8: 8-bit decode GEMV ------------------------------------------------------------
// Instantiations [M-1][config][panel slot]: slot 0 stages the activations through
// registers (up to kGemv8Av float4 per thread), slot 1 in a loop.
typedef void (*Gemv8Fn)(Gemv8Params);
template <int M, size_t I>
constexpr std::array<Gemv8Fn, 2> gemv8_pair()
{
    constexpr Gemv8Config c = kGemv8Configs[I];
    constexpr int av = kGemv8Av * 4 / c.waves;   // the same panel bytes per workgroup
    return {gemv_w8_kernel<M, c.waves, c.G, c.KW, c.U, c.RL, av>, gemv_w8_kernel<M, c.waves, c.G, c.KW, c.U, c.RL, 0>};
}
template <int M, size_t... I>
constexpr std::array<std::array<Gemv8Fn, 2>, sizeof...(I)> gemv8_row(std::index_sequence<I...>)
{
    return {gemv8_pair<M, I>()...};
}
template <int M>
constexpr std::array<std::array<Gemv8Fn, 2>, kNumGemv8Configs> gemv8_row()
{
    return gemv8_row<M>(std::make_index_sequence<kNumGemv8Configs>{});
}
const std::array<std::array<Gemv8Fn, 2>, kNumGemv8Configs> kGemv8Table[kGemvMaxM] = {
    gemv8_row<1>(), gemv8_row<2>(), gemv8_row<3>(), gemv8_row<4>(),
};
std::atomic<bool> g_gemv8_lds_raised[kGemvMaxM][kNumGemv8Configs][2];

int log2_exact(int v)
{
    int l = 0;
    while ((1 << l) < v) ++l;
    return (1 << l) == v ? l : -1;
}

// gemv_w8 takes 8-bit codes with packed or default zero points, M <= 4, a power-of-two
// block size >= 16, K a multiple of 16, an activation panel that fits LDS, and buffers
// within 32-bit offsets.
bool gemv8_eligible(const Weights& w, int M)
{
    return w.bits == 8 && !w.zp_float && M >= 1 && M <= kGemvMaxM && (w.K % 16) == 0 && w.bs >= 16 &&
           log2_exact(w.bs) >= 0 && (int64_t)M * w.K * 4 <= kGemv8MaxLds &&
           (int64_t)w.N * w.row_bytes <= INT32_MAX && (int64_t)w.N * w.nb * 4 <= INT32_MAX;
}

// Config choice (knob 11: c + 1 forces configuration c, -1 keeps 8-bit calls on
// gemv_general). From sweeping every config over 7B-shaped launches (K x N = 4096 x
// 4096, 4096 x 11008, 11008 x 4096, 4096 x 12288, 4096 x 32000, block sizes 32 and 128)
// and 896 x 896 at M = 1, 2, 4 on MI355X: 8 waves at 64 lanes per row for M <= 2 (gate
// 4096 x 11008 at M = 1: 12.4 us against 13.2-18.1 for the others), 16 waves for M >= 3
// and for K >= 8192 (gate at M = 4: 20.9 us against 21.0-39.2; 11008 x 4096 at M = 2:
// 16.4 us against 21.3 with 8 waves), 4 waves below 2048 rows (fewer, fuller
// workgroups; 3.4 us for 896 x 896 at M = 1).
int pick_gemv8_config(const Weights& w, const Knobs& kn, int M)
{
    if (!gemv8_eligible(w, M) || kn.gemv8_config() < 0) return -1;
    if (kn.gemv8_config() > 0) return kn.gemv8_config() - 1;
    if (w.N < 2048) return 7;
    return M >= 3 || w.K >= 8192 ? 3 : 0;
}

int gemv8_grid(const Weights& w, int ci) { return (w.N + gemv8_rows(kGemv8Configs[ci]) - 1) / gemv8_rows(kGemv8Configs[ci]); }

int launch_gemv_w8(const Weights& w, const Knobs& kn, const float* dA, float* dY, int M, hipStream_t stream)
{
    const int ci = pick_gemv8_config(w, kn, M);
    const int slot = (int64_t)M * w.K / 4 <= 256 * kGemv8Av ? 0 : 1;
    Gemv8Fn fn = kGemv8Table[M - 1][ci][slot];
    const size_t lds = (size_t)M * w.K * 4;
    if (lds > 64 * 1024 && !g_gemv8_lds_raised[M - 1][ci][slot].load()) {
        MS_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        g_gemv8_lds_raised[M - 1][ci][slot].store(true);
    }
    Gemv8Params p;
    p.b = w.d_b;
    p.scales = w.d_scales;
    p.zp = w.has_zp ? w.d_zp : nullptr;
    p.a = dA;
    p.y = dY;
    p.N = w.N;
    p.K = w.K;
    p.C = w.K / 16;
    p.row_bytes = (int)w.row_bytes;
    p.nb = w.nb;
    p.zrb = w.zrb;
    p.lcpb = log2_exact(w.bs / 16);
    hipLaunchKernelGGL(fn, dim3(gemv8_grid(w, ci)), dim3(kGemv8Configs[ci].waves * kWave), lds, stream, p);
    MS_HIP_CHECK(hipGetLastError());
    return MS_HIP_OK;
}

int launch_mfma_general(const Weights& w, const float* dA, float* dY, int M, hipStream_t stream)
{
    GenParams p;
    p.L = raw_layout(w);
    p.wexp = w.d_wexp;
    p.a = dA;
    p.y = dY;
    p.M = M;
    p.tiles_m = (M + kGenBM - 1) / kGenBM;
    p.tiles_n = (w.N + kGenBN - 1) / kGenBN;
    const int tiles = p.tiles_m * p.tiles_n;
    hipLaunchKernelGGL(mfma_general_kernel, dim3(((tiles + kXcds - 1) / kXcds) * kXcds), dim3(256), 0, stream, p);
    MS_HIP_CHECK(hipGetLastError());
    return MS_HIP_OK;
}

int launch_generic(const Weights& w, const float* dA, float* dY, int M, hipStream_t stream)
{
    const int64_t total = (int64_t)M * w.N;
    const int64_t grid = (total + 255) / 256;
    hipLaunchKernelGGL(nbits_generic_kernel, dim3((unsigned)grid), dim3(256), 0, stream, raw_layout(w), dA,
                       dY, M);
    MS_HIP_CHECK(hipGetLastError());
    return MS_HIP_OK;
}

// ---- workspace layouts -------------------------------------------------------------------
// fp16 activations [M][K] then row exponents [M], each 256-byte aligned.
size_t a16_bytes(int M, int K) { return align256((size_t)M * K * 2) + align256((size_t)M * 4); }

// The pipelined prefill takes M > 16, 4-bit codes (a fast layout) or 8-bit codes with
// packed or no zero points, block size 32, K a multiple of 128, fp16-safe scales, and
// buffers (Y included) below kPipeFar (its out-of-range offset).
bool pipe_eligible(const Weights& w, const Knobs& kn, int M)
{
    const bool fmt = (w.fast && w.log2cpb == 0) || (w.bits == 8 && !w.zp_float && w.bs == 32);
    return !kn.pipe_off() && fmt && M > kPanelMaxM && (w.K % 128) == 0 && w.pipe_scales_ok &&
           (int64_t)w.N * w.row_bytes < kPipeFar && (int64_t)M * w.K * 2 < kPipeFar &&
           (int64_t)w.N * w.nb * 4 < kPipeFar && (int64_t)M * w.N * 4 < kPipeFar;
}

// Compute units of the current device (the launch heuristics' notion of "filled").
int device_cus()
{
    static std::atomic<int> cached[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int v = cached[dev].load();
    if (v == 0) {
        if (hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || v <= 0) v = 256;
        cached[dev].store(v);
    }
    return v;
}

// K split of the pipelined prefill. Which tiles have their K range split over two
// workgroups (they need two groups of 4 steps, K >= 256):
//   * all of them when the tiles fill at most half of the CUs (measured: at 128 tiles on
//     256 CUs the split takes K=11008 from 297 to 227 us);
//   * else the tiles of a last round that would fill at most half of the CUs (344 tiles
//     on 256: the 88 of the second round run as 176 halves, so the launch takes about
//     1.5 rounds instead of 2; splitting all 344 into 688 items is slower);
//   * none otherwise.
// Knob 3: 1 none, 2 all, 3 the second half of the tiles (a test hook for the mixed form).
struct PipeSplit {
    int tiles, full, xu, xv;   // whole tiles [0, full); per-XCD whole and split work items
};
PipeSplit pipe_split(const Weights& w, const Knobs& kn, int M)
{
    const int tiles = ((M + kPipeBM - 1) / kPipeBM) * ((w.N + kPipeBN - 1) / kPipeBN);
    int full = tiles;
    if (w.K / 128 >= 2) {
        if (kn.pipe_ksplit() == 2) {
            full = 0;
        } else if (kn.pipe_ksplit() == 3) {
            full = tiles / 2;
        } else if (kn.pipe_ksplit() == 0) {
            const int cus = device_cus();
            if (2 * tiles <= cus) {
                full = 0;
            } else {
                const int rem = tiles % cus;
                if (rem > 0 && 2 * rem <= cus) full = tiles - rem;
            }
        }
    }
    PipeSplit sp;
    sp.tiles = tiles;
    sp.full = full;
    sp.xu = (full + kXcds - 1) / kXcds;
    sp.xv = 2 * ((tiles - full + kXcds - 1) / kXcds);
    return sp;
}

// The fp16 copy of A (and its row exponents) that the prefill kernels read, made by
// a_rows_f16_kernel in the call's workspace. Consecutive calls of one batch on the same
// activations (gate and up) share it: the first call records where it wrote the copy,
// and a later call with the same A, M and K reads that copy instead of converting again
// (the copy lives in the first call's handle workspace, untouched until the batch ends).
struct AConv {
    const float* dA = nullptr;   // the activations the copy was made from (nullptr: none)
    int M = 0, K = 0;
    const uint32_t* a16 = nullptr;
    const int* rexp = nullptr;
};
struct AConvView {
    const uint32_t* a16;
    const int* rexp;
};
AConvView a_conv_for(AConv* conv, const Ws& ws, const float* dA, int M, int K, hipStream_t stream)
{
    if (conv && conv->dA == dA && conv->M == M && conv->K == K && conv->a16) return {conv->a16, conv->rexp};
    uint32_t* a16 = reinterpret_cast<uint32_t*>(ws.data);
    int* rexp = reinterpret_cast<int*>(ws.data + align256((size_t)M * K * 2));
    launch_a_rows_f16(dA, a16, rexp, M, K, stream);
    if (conv) *conv = AConv{dA, M, K, a16, rexp};
    return {a16, rexp};
}

// Workspace of a pipelined launch: fp16 A and row exponents, then one partial-sum slot
// per split tile; two counters per split tile.
struct PipeWs {
    size_t data, cnt, part_off;
};
PipeWs pipe_ws(const Weights& w, int M, const PipeSplit& sp)
{
    PipeWs r;
    const int nsplit = sp.tiles - sp.full;
    r.part_off = a16_bytes(M, w.K);
    r.data = r.part_off + (size_t)nsplit * kPipeBM * kPipeBN * sizeof(float);
    r.cnt = (size_t)2 * nsplit;
    return r;
}

int launch_pipe(Weights& w, const Knobs& kn, const Ws& ws, const float* dA, float* dY, int M, hipStream_t stream,
                AConv* conv)
{
    const int tiles_m = (M + kPipeBM - 1) / kPipeBM, tiles_n = (w.N + kPipeBN - 1) / kPipeBN;
    const PipeSplit sp = pipe_split(w, kn, M);
    const PipeWs L = pipe_ws(w, M, sp);
    const bool b8 = w.bits == 8;
    static std::atomic<bool> lds_raised[2] = {false, false};
    if (!lds_raised[b8].load()) {
        if (b8)
            MS_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(mfma_w4_pipe_kernel<true>),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, PipeLds<true>::BYTES));
        else
            MS_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(mfma_w4_pipe_kernel<false>),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, PipeLds<false>::BYTES));
        lds_raised[b8].store(true);
    }
    const AConvView av = a_conv_for(conv, ws, dA, M, w.K, stream);
    const uint32_t* a16 = av.a16;
    const int* rexp = av.rexp;
    PipeParams p;
    p.b = w.d_b;
    p.scales = w.d_scales;
    p.zp = w.has_zp ? w.d_zp : nullptr;
    p.a16 = reinterpret_cast<const _Float16*>(a16);
    p.rexp = rexp;
    p.y = dY;
    p.row_bytes = (int)w.row_bytes;
    p.M = M;
    p.N = w.N;
    p.K = w.K;
    p.C = w.K / 32;
    p.nb = w.nb;
    p.zrb = w.zrb;
    p.tiles_m = tiles_m;
    p.tiles_n = tiles_n;
    p.full = sp.full;
    p.xu = sp.xu;
    p.xv = sp.xv;
    p.sync = ws.cnt;
    p.part = reinterpret_cast<float*>(ws.data + L.part_off);
    p.epoch = next_epoch();
    p.spin_limit = kn.spin_limit();
    p.err = w.d_err;
    const dim3 grid(kXcds * (sp.xu + sp.xv)), block(256);
    if (b8)
        hipLaunchKernelGGL(mfma_w4_pipe_kernel<true>, grid, block, PipeLds<true>::BYTES, stream, p);
    else
        hipLaunchKernelGGL(mfma_w4_pipe_kernel<false>, grid, block, PipeLds<false>::BYTES, stream, p);
    MS_HIP_CHECK(hipGetLastError());
    return MS_HIP_OK;
}

// ---- skinny_w4: M <= 16 on the matrix cores at fp32-level accuracy (block sizes 32-128) ----

// The small-M matrix-core path takes block sizes 32, 64 and 128 (a 128-k block is one group
// of four MFMA steps; with 32 and 64 the code dwords are transposed so that each step is
// one quantization block), K a multiple of 128, and M <= 16 by the rules below: at M <= 2
// gemv_w4 is faster where its panel fits (measured on the Llama-2-7B MLP shapes, bs 128:
// M=2 13.2 / 12.5 us against 15.4 / 16.7 us; M=3 20.4 / 24.2 us against 15.8 / 17.3 us),
// unless knob 4 says otherwise.
constexpr int kSkinnyMinM = 3;
// Quantization blocks per 128-k block of a layout the small-M matrix-core kernel takes
// (4-bit or 8-bit codes with packed or no zero points, block size 32, 64 or 128), else 0.
int skinny_qpb(const Weights& w)
{
    const bool fmt = w.fast || (w.bits == 8 && !w.zp_float);
    if (!fmt) return 0;
    return w.bs == 128 ? 1 : w.bs == 64 ? 2 : w.bs == 32 ? 4 : 0;
}
bool skinny_eligible(const Weights& w, const Knobs& kn, int M)
{
    if (kn.skinny() == 1 || skinny_qpb(w) == 0 || (w.K % 128) != 0 || M < 1 || M > kSkinnyMT) return false;
    if ((int64_t)kSkinnyMT * w.K * 4 >= INT32_MAX || (int64_t)w.N * w.row_bytes >= kOOB) return false;
    // the partial-sum slices stay within the reduce's 32-bit buffer offsets
    if ((int64_t)(w.K / 128) * ((int64_t)kSkinnyMT * w.N + 3) / 4 * 16 >= kOOB) return false;
    if (kn.skinny() == 2) return true;
    // 8-bit codes: from M = 5, where gemv_w8 stops; below that by default where it measured
    // faster than gemv_w8 (K=4096/N=11008: bs 128 from M = 3, 15.9 against 17.8 us; bs 32
    // from M = 4, 19.1 against 20.9 us, while at M = 3 gemv_w8 leads, 18.5 against 19.2) and
    // wherever gemv_w8's panel does not fit (K=11008, M = 4: 22.1 us against 202 us on
    // gemv_general). A forced gemv_w8 configuration or knob 11 = -1 keeps M <= 4 where that
    // knob sends it.
    if (w.bits == 8) {
        if (M >= 5) return true;
        if (M < kSkinnyMinM || kn.gemv8_config() != 0) return false;
        return pick_gemv8_config(w, kn, M) < 0 || M >= (w.bs == 128 ? 3 : 4);
    }
    const bool gemv_fits = pick_gemv_config(w, kn, M, w.N) >= 0;
    // Block size 128: from M = 3. Block sizes 32 and 64 (a scale per 32-k step): from M = 5,
    // and from M = 3 for large matrices (N >= 8192); measured on the 7B decode launches
    // (bs 32, zero points), gate 3584 x 18944 at M = 3 / 4: 19.0 / 19.3 us against 21.2 /
    // 24.5 with gemv_w4, but o 3584 x 3584: 12.5 / 12.7 against 7.6 / 9.0 (few row tiles
    // force a wide K split). At M = 5 the panel kernel is a little faster on the short-K
    // q+k+v and o (27.8 / 12.4 against 28.8 / 12.8 us) and far slower on down (K=18944:
    // 54.1 against 24.1 us); from M = 6 this kernel leads on all four. Either way at M = 2
    // where the VALU GEMV's panel does not fit one workgroup (the panel kernel would take
    // it: 7B down, K=18944, bs 32: 26.9 us against 23.2 us here).
    if (M == 2) return !gemv_fits;
    if (w.log2cpb == 2) return M >= kSkinnyMinM;
    return M >= 5 || !gemv_fits || (M >= kSkinnyMinM && w.N >= 8192);
}

// Workgroups per row tile: each takes at most kSkinnyNB blocks and at least one; beyond
// that minimum, more only while the grid has fewer than two workgroups per CU (every
// extra split adds a slot to write and to sum).
int skinny_ksw(const Weights& w, const Knobs& kn)
{
    const int tiles = (w.N + kSkinnyRows - 1) / kSkinnyRows;
    const int G = w.K / 128;
    const int kmin = (G + kSkinnyNB - 1) / kSkinnyNB;
    int ksw = kmin;
    if (kn.skinny_ksw() > 0) {
        ksw = kn.skinny_ksw();
    } else {
        while (ksw < G && (int64_t)tiles * ksw < 2 * device_cus()) ++ksw;
    }
    return std::max(kmin, std::min(ksw, G));
}

// Workspace of a skinny_w4 launch: one slot per workgroup, one counter per row tile.
// Workspace of a K-split call: up to kSkinnyHandoffMax workgroups per tile, a slot per
// workgroup and an arrival counter per row tile (the in-kernel hand-off); wider splits,
// ksw slices of M * N floats, each rounded up to a multiple of 4 (16-byte aligned), for
// skinny_reduce_kernel.
int skinny_slice4(const Weights& w, int M) { return (int)(((int64_t)M * w.N + 3) / 4); }
void skinny_ws(const Weights& w, int ksw, int M, size_t* data, size_t* cnt)
{
    const int tiles = (w.N + kSkinnyRows - 1) / kSkinnyRows;
    *data = ksw <= 1 ? 0
          : ksw <= kSkinnyHandoffMax ? (size_t)tiles * ksw * kSkinnySlot * sizeof(float)
                                      : (size_t)ksw * skinny_slice4(w, M) * 16;
    *cnt = ksw > 1 && ksw <= kSkinnyHandoffMax ? (size_t)tiles : 0;
}

int launch_skinny(Weights& w, const Knobs& kn, const Ws& ws, const float* dA, float* dY, int M, hipStream_t stream)
{
    const int tiles = (w.N + kSkinnyRows - 1) / kSkinnyRows;
    const int ksw = skinny_ksw(w, kn);
    SkinnyParams p;
    p.b = w.d_b;
    p.scales = w.d_scales;
    p.zp = w.has_zp ? w.d_zp : nullptr;
    p.a = dA;
    p.y = dY;
    const bool handoff = ksw > 1 && ksw <= kSkinnyHandoffMax;
    p.part = ksw > 1 && !handoff ? reinterpret_cast<float*>(ws.data) : nullptr;
    p.slice4 = skinny_slice4(w, M);
    p.slots = handoff ? reinterpret_cast<float*>(ws.data) : nullptr;
    p.sync = handoff ? ws.cnt : nullptr;
    p.row_bytes = (int)w.row_bytes;
    p.M = M;
    p.N = w.N;
    p.K = w.K;
    p.nb = w.nb;
    p.zrb = w.zrb;
    p.ksw = ksw;
    // quantization blocks per 128-k block: 1 (bs 128), 2 (bs 64), 4 (bs 32); 4- or 8-bit codes
    const int qpb = skinny_qpb(w);
    const dim3 grid(tiles * ksw), block(256);
    if (w.bits == 8) {
        if (qpb == 1)
            hipLaunchKernelGGL((skinny_w4_kernel<1, true>), grid, block, 0, stream, p);
        else if (qpb == 2)
            hipLaunchKernelGGL((skinny_w4_kernel<2, true>), grid, block, 0, stream, p);
        else
            hipLaunchKernelGGL((skinny_w4_kernel<4, true>), grid, block, 0, stream, p);
    } else if (qpb == 1) {
        hipLaunchKernelGGL((skinny_w4_kernel<1, false>), grid, block, 0, stream, p);
    } else if (qpb == 2) {
        hipLaunchKernelGGL((skinny_w4_kernel<2, false>), grid, block, 0, stream, p);
    } else {
        hipLaunchKernelGGL((skinny_w4_kernel<4, false>), grid, block, 0, stream, p);
    }
    MS_HIP_CHECK(hipGetLastError());
    if (p.part) {
        hipLaunchKernelGGL(skinny_reduce_kernel, dim3((p.slice4 + 255) / 256), dim3(256), 0, stream, p.part, dY,
                           M * w.N, p.slice4, ksw);
        MS_HIP_CHECK(hipGetLastError());
    }
    return MS_HIP_OK;
}

// ---- mfma_w4_rb: prefill with the weights dequantized into MFMA operand registers ----
// Any power-of-two block size >= 32, K a multiple of 128, fp16-safe scales (as the
// pipelined kernel: W = fl16((q - zp) * fl16(s))), every buffer below the out-of-range
// offset the kernel uses for padding rows.
bool rb_eligible(const Weights& w, const Knobs& kn, int M)
{
    // 4-bit fast layouts, or 8-bit codes with packed or no zero points and a power-of-two
    // block size >= 32 (one scale per 32-code chunk)
    const bool fmt = w.fast || (w.bits == 8 && !w.zp_float && w.bs >= 32 && log2_exact(w.bs) >= 0);
    return kn.rb() != 1 && fmt && M > kPanelMaxM && (w.K % 128) == 0 && w.pipe_scales_ok &&
           (int64_t)w.N * w.row_bytes < kOOB && (int64_t)M * w.K * 2 < kOOB && (int64_t)w.N * w.K / 8 < kOOB &&
           (int64_t)M * w.N * 4 < kOOB;
}

// Tile width and K split of an mfma_w4_rb launch: tiles of 128 x 64 NF outputs, ksw
// workgroups per tile (each a contiguous range of 128-k blocks), the partial sums summed
// (and scaled by the row exponents) by rb_reduce_kernel. The pick minimises
//   rounds x ceil(G / ksw) x t_block(NF) + (2 ksw + 1) x 4 M N / 4 TB/s + t_launch
// over NF in {1, 2, 4} and ksw <= min(G, 32): rounds of one workgroup per CU, t_block the
// time a workgroup spends on one 128-k block (about 3.5 us at NF = 4 with the chip busy,
// measured: K = 11008 unsplit at M = 2048 took 301 us for 86 blocks; the model charges the
// A block every workgroup stages whatever its width), and the partial sums written and
// read back once each, plus Y, charged at 2 TB/s: the slices leave in one burst at the end
// of the GEMM with no MFMA work beside it (a sweep of NF x K split on the 7B shapes put
// K=11008, N=4096, M=64 at NF 2 / split 8, 29.6 us, where the 4 TB/s charge picked NF 4 /
// split 15, 32.1 us; the other few-tile shapes keep their picks). Knob 9 forces NF, knob 7
// ksw.
struct RbShape {
    int nf, ksw, tiles_m, tiles_n;
};
RbShape rb_shape(const Weights& w, const Knobs& kn, int M)
{
    const int G = w.K / 128;
    const int cus = device_cus();
    const int tiles_m = (M + kRbBM - 1) / kRbBM;
    const double hbm = 2.0e12, t_launch = 2e-6;
    const double ybytes = (double)M * w.N * 4;
    // The 8-bit form is instantiated for NF 1 and 2 only (twice the code registers per
    // fragment); a forced NF of 4 falls back to the pick there.
    const bool b8 = w.bits == 8;
    const int force_nf = b8 && kn.rb_nf() == 4 ? 0 : kn.rb_nf();
    RbShape best = b8 ? RbShape{2, 1, tiles_m, (w.N + 127) / 128} : RbShape{4, 1, tiles_m, (w.N + 255) / 256};
    double best_t = 1e30;
    for (int nf : {4, 2, 1}) {
        if (force_nf > 0 && nf != force_nf) continue;
        if (b8 && nf == 4) continue;
        const int tiles_n = (w.N + 64 * nf - 1) / (64 * nf);
        const int64_t tiles = (int64_t)tiles_m * tiles_n;
        const double t_block = 1.4e-6 + 0.525e-6 * nf;
        for (int k = 1; k <= std::min(G, 32); ++k) {
            // the slices stay within the reduce's 32-bit buffer offsets
            if (k > 1 && (int64_t)k * (((int64_t)M * w.N + 3) / 4) * 16 >= kOOB) break;
            if (kn.rb_ksw() > 0 && k != std::max(1, std::min(kn.rb_ksw(), G))) continue;
            const double rounds = (double)((tiles * k + cus - 1) / cus);
            const double t = rounds * std::ceil((double)G / k) * t_block + (2.0 * k + 1) * ybytes / hbm + t_launch;
            if (t < best_t * 0.97) {
                best_t = t;
                best = RbShape{nf, k, tiles_m, tiles_n};
            }
        }
    }
    return best;
}

// Which prefill kernel: mfma_w4_rb where the pipelined kernel does not apply (block
// sizes other than 32), and where the pipelined launch would fill less than half of the
// CUs: measured on the 7B MLP shapes, 128 x 256 tiles with a wide K split beat it there
// (M=128: 49 / 45 us against 78 / 143 us; M=512, K=11008: 103 against 154 us), while
// with more tiles the pipelined kernel is faster (M=512, K=4096: 100 against 118 us;
// M=2048: 262 against 320-355 us). Whenever M fits one 128-row tile as well: the
// pipelined kernel's 256-row tiles then compute mostly padding (7B gate, K=3584,
// N=18944: M = 17 / 64 / 128 39.0 / 44.0 / 52.1 us against 66.9 / 67.2 / 67.8 us, while
// from M = 192 the pipelined kernel leads there, 68.6 against 86.0 us).
bool use_rb(const Weights& w, const Knobs& kn, int M)
{
    if (!rb_eligible(w, kn, M)) return false;
    if (kn.rb() == 2 || !pipe_eligible(w, kn, M) || M <= kRbBM) return true;
    const PipeSplit sp = pipe_split(w, kn, M);
    const int64_t items = sp.full + 2 * (sp.tiles - sp.full);
    return 2 * items < device_cus();
}

// Workspace of an mfma_w4_rb launch: fp16 A and row exponents, then ksw slices of Y
// (one when K is not split: the reduce applies the row exponents).
struct RbWs {
    size_t data, part_off;
    int64_t slice;
};
RbWs rb_ws(const Weights& w, int M, int ksw)
{
    RbWs r;
    r.slice = ((int64_t)M * w.N + 3) / 4 * 4;   // floats per K-split slice, 16-byte multiple
    r.part_off = a16_bytes(M, w.K);
    r.data = r.part_off + (size_t)ksw * r.slice * sizeof(float);
    return r;
}

int launch_rb(Weights& w, const Knobs& kn, const Ws& ws, const float* dA, float* dY, int M, hipStream_t stream,
              AConv* conv)
{
    const RbShape sh = rb_shape(w, kn, M);
    const int tiles_m = sh.tiles_m, tiles_n = sh.tiles_n, ksw = sh.ksw;
    const RbWs L = rb_ws(w, M, ksw);
    const AConvView av = a_conv_for(conv, ws, dA, M, w.K, stream);
    const uint32_t* a16 = av.a16;
    const int* rexp = av.rexp;
    float* part = reinterpret_cast<float*>(ws.data + L.part_off);
    RbParams p;
    p.b = w.d_b;
    p.sz4 = w.d_sz4;
    p.a16 = reinterpret_cast<const _Float16*>(a16);
    p.out = part;
    p.slice = L.slice;
    p.row_bytes = (int)w.row_bytes;
    p.M = M;
    p.N = w.N;
    p.K = w.K;
    p.tiles_m = tiles_m;
    p.tiles_n = tiles_n;
    p.ksw = ksw;
    const int items = tiles_m * tiles_n * ksw;
    const dim3 grid(((items + kXcds - 1) / kXcds) * kXcds);
    if (w.bits == 8) {
        if (sh.nf == 1)
            hipLaunchKernelGGL((mfma_w4_rb_kernel<1, true>), grid, dim3(256), 0, stream, p);
        else
            hipLaunchKernelGGL((mfma_w4_rb_kernel<2, true>), grid, dim3(256), 0, stream, p);
    } else if (sh.nf == 1) {
        hipLaunchKernelGGL((mfma_w4_rb_kernel<1, false>), grid, dim3(256), 0, stream, p);
    } else if (sh.nf == 2) {
        hipLaunchKernelGGL((mfma_w4_rb_kernel<2, false>), grid, dim3(256), 0, stream, p);
    } else {
        hipLaunchKernelGGL((mfma_w4_rb_kernel<4, false>), grid, dim3(256), 0, stream, p);
    }
    const int slice4 = (int)(L.slice / 4);
    hipLaunchKernelGGL(rb_reduce_kernel, dim3((unsigned)std::min((slice4 + 255) / 256, 8192)), dim3(256), 0, stream,
                       reinterpret_cast<const float4*>(part), dY, rexp, M * w.N, w.N, slice4, ksw,
                       (w.N % 4 == 0 && (reinterpret_cast<uintptr_t>(dY) & 15) == 0) ? 1 : 0);
    MS_HIP_CHECK(hipGetLastError());
    return MS_HIP_OK;
}

// mfma_w4_rb's chunk-major scales and zero points: built once, on the call's stream, by
// the first call that takes the kernel outside stream capture (then the stream is
// synchronised once, so calls on other streams find the copy complete). Returns 1 when
// the copy is there, 0 when it cannot be built now (capture), -1 on a HIP failure.
int ensure_rb_layout(Weights& w, hipStream_t stream)
{
    if (w.rb_ready.load(std::memory_order_acquire)) return 1;
    std::lock_guard<std::mutex> lock(w.ws_mu);
    if (w.rb_ready.load(std::memory_order_relaxed)) return 1;
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) {
        (void)hipGetLastError();
        return 0;
    }
    const int G = w.K / 128;
    const int64_t entries = (int64_t)G * w.N * 4;
    if (!w.d_sz4 && hipMalloc(&w.d_sz4, (size_t)entries * sizeof(uint32_t)) != hipSuccess) return -1;
    const int grid = (int)std::min<int64_t>((entries + 255) / 256, 8192);
    hipLaunchKernelGGL(rb_chunk_layout_kernel, dim3(grid), dim3(256), 0, stream, w.d_scales,
                       w.has_zp ? w.d_zp : nullptr, w.d_sz4, w.N, G, w.nb, w.zrb, log2_exact(w.bs), w.bits);
    if (hipGetLastError() != hipSuccess || hipStreamSynchronize(stream) != hipSuccess) return -1;
    w.rb_ready.store(1, std::memory_order_release);
    return 1;
}

// ---- dispatch ------------------------------------------------------------------------------
// Which kernel a call with M rows takes (ids of ms_hip_nbits_launch_info).
enum KernelId {
    kGeneric = 0, kGemv = 1, kMfma = 2, kPanel = 3, kPipe = 4, kSkinny = 5, kRb = 6, kGemvGeneral = 7,
    kMfmaGeneral = 8, kGemvW8 = 12
};

KernelId choose_kernel(const Weights& w, const Knobs& kn, int M)
{
    if (!w.fast) {
        if (M <= kPanelMaxM && skinny_eligible(w, kn, M)) return kSkinny;   // 8-bit small M
        if (pick_gemv8_config(w, kn, M) >= 0) return kGemvW8;
        // 8-bit prefill: the pipelined kernel (block size 32) by the same rule as 4-bit codes
        if (M > kPanelMaxM && pipe_eligible(w, kn, M) && !use_rb(w, kn, M)) return kPipe;
        if (rb_eligible(w, kn, M)) return kRb;
        if (!general_eligible(w)) return kGeneric;
        return M <= kPanelMaxM ? kGemvGeneral : kMfmaGeneral;
    }
    if (M <= kPanelMaxM) {
        if (skinny_eligible(w, kn, M)) return kSkinny;
        return pick_gemv_config(w, kn, M, w.N) >= 0 ? kGemv : kPanel;
    }
    if (use_rb(w, kn, M)) return kRb;
    if (pipe_eligible(w, kn, M)) return kPipe;
    return kMfma;
}

// Workspace (data bytes, counters) that kernel `k` needs for a call with M rows.
void workspace_need(const Weights& w, const Knobs& kn, KernelId k, int M, size_t* data, size_t* cnt)
{
    *data = 0;
    *cnt = 0;
    if (k == kSkinny) {
        skinny_ws(w, skinny_ksw(w, kn), M, data, cnt);
    } else if (k == kRb) {
        *data = rb_ws(w, M, rb_shape(w, kn, M).ksw).data;
    } else if (k == kPipe) {
        const PipeWs L = pipe_ws(w, M, pipe_split(w, kn, M));
        *data = L.data;
        *cnt = L.cnt;
    }
}

// The kernel a call takes when its workspace cannot be had (growth under capture).
KernelId workspace_free_kernel(const Weights& w, const Knobs& kn, int M)
{
    if (!w.fast) {
        if (pick_gemv8_config(w, kn, M) >= 0) return kGemvW8;
        if (!general_eligible(w)) return kGeneric;
        return M <= kPanelMaxM ? kGemvGeneral : kMfmaGeneral;
    }
    if (M <= kPanelMaxM) return pick_gemv_config(w, kn, M, w.N) >= 0 ? kGemv : kPanel;
    return kMfma;
}

int launch_kernel(Weights& w, const Knobs& kn, KernelId k, const Ws& ws, const float* dA, float* dY, int M,
                  hipStream_t stream, AConv* conv = nullptr)
{
    switch (k) {
        case kGeneric: return launch_generic(w, dA, dY, M, stream);
        case kGemvGeneral: return launch_gemv_general(w, dA, dY, M, stream);
        case kMfmaGeneral: return launch_mfma_general(w, dA, dY, M, stream);
        case kGemvW8: return launch_gemv_w8(w, kn, dA, dY, M, stream);
        case kGemv:
        case kPanel: return launch_gemv(w, kn, dA, dY, M, stream);
        case kSkinny: return launch_skinny(w, kn, ws, dA, dY, M, stream);
        case kRb: return launch_rb(w, kn, ws, dA, dY, M, stream, conv);
        case kPipe: return launch_pipe(w, kn, ws, dA, dY, M, stream, conv);
        case kMfma:
            return launch_mfma(w.d_b, w.d_scales, w.has_zp ? w.d_zp : nullptr, w.row_bytes, w.N, w.K, w.nb, w.zrb,
                               w.log2cpb, dA, dY, M, stream)
                       ? fail(MS_HIP_ERR_HIP, "[ms_hip] MFMA launch failed: %s", hipGetErrorString(hipGetLastError()))
                       : MS_HIP_OK;
    }
    return fail(MS_HIP_ERR_HIP, "[ms_hip] no kernel");
}

int check_call(const float* dA, float* dY, int M)
{
    if (M < 0) return fail(MS_HIP_ERR_INVALID, "MatMulNBits M must be non-negative; got %d.", M);
    if (M > 0 && (!dA || !dY)) return fail(MS_HIP_ERR_INVALID, "[ms_hip] null activation or output pointer");
    if (M > 0 && ((reinterpret_cast<uintptr_t>(dA) & 15) || (reinterpret_cast<uintptr_t>(dY) & 3)))
        return fail(MS_HIP_ERR_INVALID, "[ms_hip] A must be 16-byte and Y 4-byte aligned");
    return MS_HIP_OK;
}

// A call routed to mfma_w4_rb needs the handle's chunk-major scales: built here when
// `may_build` (and the stream is not capturing), else the call takes the exact
// workspace-free kernel instead.
int resolve_rb(Weights& w, const Knobs& kn, KernelId* k, int M, hipStream_t stream, bool may_build)
{
    if (*k != kRb || w.rb_ready.load(std::memory_order_acquire)) return MS_HIP_OK;
    const int r = may_build ? ensure_rb_layout(w, stream) : 0;
    if (r < 0) return fail(MS_HIP_ERR_HIP, "[ms_hip] scale re-layout failed: %s", hipGetErrorString(hipGetLastError()));
    if (r == 0) *k = workspace_free_kernel(w, kn, M);
    return MS_HIP_OK;
}

// One call with the handle's own (growable) workspace.
int enqueue_gemm(Weights& w, const float* dA, float* dY, int M, hipStream_t stream, AConv* conv = nullptr)
{
    int st = check_call(dA, dY, M);
    if (st || M == 0) return st;
    const Knobs kn = knobs_of(w);
    KernelId k = choose_kernel(w, kn, M);
    if ((st = resolve_rb(w, kn, &k, M, stream, true))) return st;
    size_t need_d = 0, need_c = 0;
    workspace_need(w, kn, k, M, &need_d, &need_c);
    Ws ws;
    if (need_d || need_c) {
        const int r = ensure_ws(w, need_d, need_c, stream, &ws);
        if (r < 0) return fail(MS_HIP_ERR_HIP, "[ms_hip] workspace allocation failed: %s", hipGetErrorString(hipGetLastError()));
        if (r == 0) k = workspace_free_kernel(w, kn, M);
    }
    return launch_kernel(w, kn, k, ws, dA, dY, M, stream, conv);
}

// ---- W4A8 (the opt-in approximate product) --------------------------------------------------
// Workspace of one call: activation codes [M][padK], their scales [M][nb] and the
// transposed scales [nb][Mp], each 256-byte aligned.
struct W4a8Layout {
    int padK = 0, Mp = 0;
    size_t sa_off = 0, sat_off = 0, total = 0;
};

W4a8Layout w4a8_layout(const Weights& w, int M)
{
    W4a8Layout L;
    L.padK = ((w.nb * w.bs + 31) / 32) * 32;
    L.Mp = ((M + 3) / 4) * 4;
    L.sa_off = align256((size_t)M * L.padK);
    L.sat_off = L.sa_off + align256((size_t)M * w.nb * sizeof(float));
    L.total = L.sat_off + align256((size_t)w.nb * L.Mp * sizeof(float));
    return L;
}

enum W4a8KernelId { kW8Gemv = 9, kW8Mfma = 10, kW8Generic = 11 };

W4a8KernelId w4a8_kernel(const Weights& w, int M)
{
    if (w.bits == 4 && w.bs % 32 == 0) return M <= 16 ? kW8Gemv : kW8Mfma;
    return kW8Generic;
}

int w4a8_grid(const Weights& w, int M, W4a8KernelId k)
{
    if (k == kW8Gemv) return (w.N + kW8RowsPerWg - 1) / kW8RowsPerWg;
    if (k == kW8Mfma) {
        const int tiles = ((M + kW8BM - 1) / kW8BM) * ((w.N + kW8BN - 1) / kW8BN);
        return ((tiles + kXcds - 1) / kXcds) * kXcds;
    }
    return (int)(((int64_t)M * w.N + 255) / 256);
}

typedef void (*W8GemvFn)(RawLayout, W4a8Args, float*);
template <size_t... I>
constexpr std::array<W8GemvFn, sizeof...(I)> w8_gemv_table(std::index_sequence<I...>)
{
    return {gemv_w4a8_kernel<(int)I + 1>...};
}
constexpr auto kW8GemvTable = w8_gemv_table(std::make_index_sequence<16>{});

int launch_w4a8(const Weights& w, const Ws& ws, const float* dA, float* dY, int M, hipStream_t stream)
{
    const W4a8Layout Lw = w4a8_layout(w, M);
    int8_t* aq = reinterpret_cast<int8_t*>(ws.data);
    float* sa = reinterpret_cast<float*>(ws.data + Lw.sa_off);
    float* sat = reinterpret_cast<float*>(ws.data + Lw.sat_off);
    const int64_t threads = (int64_t)Lw.Mp * w.nb * 8;
    hipLaunchKernelGGL(w4a8_quantize_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, stream, dA, aq,
                       sa, sat, M, Lw.Mp, w.K, w.bs, w.nb, Lw.padK);
    MS_HIP_CHECK(hipGetLastError());
    W4a8Args A;
    A.aq = aq;
    A.sa = sa;
    A.sat = sat;
    A.M = M;
    A.Mp = Lw.Mp;
    A.padK = Lw.padK;
    const RawLayout L = raw_layout(w);
    const W4a8KernelId k = w4a8_kernel(w, M);
    const int grid = w4a8_grid(w, M, k);
    if (k == kW8Gemv) {
        hipLaunchKernelGGL(kW8GemvTable[M - 1], dim3(grid), dim3(256), 0, stream, L, A, dY);
    } else if (k == kW8Mfma) {
        W4a8MfmaParams p;
        p.L = L;
        p.A = A;
        p.y = dY;
        p.tiles_m = (M + kW8BM - 1) / kW8BM;
        p.tiles_n = (w.N + kW8BN - 1) / kW8BN;
        hipLaunchKernelGGL(mfma_w4a8_kernel, dim3(grid), dim3(256), 0, stream, p);
    } else {
        hipLaunchKernelGGL(w4a8_generic_kernel, dim3(grid), dim3(256), 0, stream, L, A, dY);
    }
    MS_HIP_CHECK(hipGetLastError());
    return MS_HIP_OK;
}

int enqueue_w4a8(Weights& w, const float* dA, float* dY, int M, hipStream_t stream)
{
    if (w.zp_float)
        return fail(MS_HIP_ERR_UNSUPPORTED,
                    "[ms_hip] W4A8 takes packed or default zero points, as the native ms_qgemm_w4a8 does "
                    "(NativeQuant.cs:78-101); this handle has float zero points");
    int st = check_call(dA, dY, M);
    if (st || M == 0) return st;
    Ws ws;
    const int r = ensure_ws(w, w4a8_layout(w, M).total, 0, stream, &ws);
    if (r < 0) return fail(MS_HIP_ERR_HIP, "[ms_hip] workspace allocation failed: %s", hipGetErrorString(hipGetLastError()));
    if (r == 0)
        return fail(MS_HIP_ERR_UNSUPPORTED,
                    "[ms_hip] W4A8 needs the handle's workspace, which cannot grow under stream capture: "
                    "make one call of this size outside the capture first");
    return launch_w4a8(w, ws, dA, dY, M, stream);
}

int check_impl(int N, int K, int bits, int bs, int64_t b_len, int64_t scales_len, int zp_kind, int64_t zp_len,
               int64_t a_last_dim)
{
    // Messages of MatMulNBitsKernel.cs:87-161 (U+00D7 in UTF-8).
    if (N <= 0 || K <= 0)
        return fail(MS_HIP_ERR_INVALID, "MatMulNBits requires positive N and K attributes (got N=%d, K=%d).", N,
                    K);
    if (bits != 4 && bits != 8)
        return fail(MS_HIP_ERR_INVALID, "MatMulNBits supports bits=4 or bits=8; got %d.", bits);
    if (bs <= 0) return fail(MS_HIP_ERR_INVALID, "MatMulNBits requires a positive block_size; got %d.", bs);
    const int64_t nb = ((int64_t)K + bs - 1) / bs;
    const int64_t blob = ((int64_t)bs * bits + 7) / 8;
    const int64_t expected_b = (int64_t)N * nb * blob;
    if (b_len != expected_b)
        return fail(MS_HIP_ERR_INVALID,
                    "MatMulNBits B has %lld elements; expected %lld (N=%d \xC3\x97 n_blocks_per_row=%lld "
                    "\xC3\x97 blob_size=%lld).",
                    (long long)b_len, (long long)expected_b, N, (long long)nb, (long long)blob);
    const int64_t expected_scales = (int64_t)N * nb;
    if (scales_len != expected_scales)
        return fail(MS_HIP_ERR_INVALID,
                    "MatMulNBits scales has %lld elements; expected %lld (N=%d \xC3\x97 n_blocks_per_row=%lld).",
                    (long long)scales_len, (long long)expected_scales, N, (long long)nb);
    const int64_t zrb = (nb * bits + 7) / 8;
    if (zp_kind == 2 && zp_len != expected_scales)
        return fail(MS_HIP_ERR_INVALID, "MatMulNBits float zero_points has %lld elements; expected %lld.",
                    (long long)zp_len, (long long)expected_scales);
    if (zp_kind == 1 && zp_len != (int64_t)N * zrb)
        return fail(MS_HIP_ERR_INVALID,
                    "MatMulNBits packed zero_points has %lld bytes; expected %lld (N=%d \xC3\x97 %lld).",
                    (long long)zp_len, (long long)N * zrb, N, (long long)zrb);
    if (zp_kind != 0 && zp_kind != 1 && zp_kind != 2)
        return fail(MS_HIP_ERR_INVALID, "MatMulNBits zero_points must be Float32 or UInt8.");
    if (a_last_dim >= 0 && a_last_dim != K)
        return fail(MS_HIP_ERR_INVALID, "MatMulNBits A inner dimension must equal K=%d; got %lld.", K,
                    (long long)a_last_dim);
    return MS_HIP_OK;
}

// fp16 -> fp32, exact (the reference widens fp16 tensors the same way, GraphContext.cs:106).
__global__ __launch_bounds__(256) void f16_to_f32_kernel(const _Float16* __restrict__ in, float* __restrict__ out,
                                                         int64_t n)
{
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        out[i] = (float)in[i];
}

void launch_widen(const void* in, float* out, int64_t n, hipStream_t stream)
{
    hipLaunchKernelGGL(f16_to_f32_kernel, dim3((unsigned)std::min<int64_t>((n + 255) / 256, 4096)), dim3(256), 0,
                       stream, static_cast<const _Float16*>(in), out, n);
}

// Copies n elements of type `type` (MS_HIP_DTYPE_F32 or _F16) from host or device memory
// at src into the fp32 device buffer dst, widening fp16 exactly.
hipError_t upload_f32(float* dst, const void* src, int64_t n, int type, hipMemcpyKind kind)
{
    if (type == MS_HIP_DTYPE_F32) return hipMemcpy(dst, src, (size_t)n * 4, kind);
    void* tmp = nullptr;
    hipError_t e = hipMalloc(&tmp, (size_t)n * 2);
    if (e == hipSuccess) e = hipMemcpy(tmp, src, (size_t)n * 2, kind);
    if (e == hipSuccess) {
        launch_widen(tmp, dst, n, nullptr);
        e = hipGetLastError();
    }
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (tmp) (void)hipFree(tmp);
    return e;
}

// A new handle for the layout (N, K, bits, bs) with zero points of kind zp_kind (0 none,
// 1 packed uint8, 2 float): device buffers for the weights and the pinned error word. On
// failure everything is freed and *out stays null.
int new_weights(int N, int K, int bits, int bs, int zp_kind, Weights** out)
{
    *out = nullptr;
    Weights* w = new Weights();
    for (auto& k : w->knob) k.store(MS_HIP_TUNING_INHERIT);
    w->device = device_info().device;
    derive_layout(*w, N, K, bits, bs);
    w->has_zp = zp_kind == 1;
    w->zp_float = zp_kind == 2;
    if (w->zp_float) w->fast = 0;   // the 4-bit kernels take integer zero points only
    hipError_t e = hipMalloc(&w->d_b, (size_t)N * w->row_bytes);
    if (e == hipSuccess) e = hipMalloc(&w->d_scales, (size_t)N * w->nb * sizeof(float));
    if (e == hipSuccess && w->has_zp) e = hipMalloc(&w->d_zp, (size_t)N * w->zrb);
    if (e == hipSuccess && w->zp_float) e = hipMalloc(&w->d_zpf, (size_t)N * w->nb * sizeof(float));
    if (e == hipSuccess && !w->fast) e = hipMalloc(&w->d_wexp, (size_t)N * sizeof(int));
    if (e == hipSuccess) e = hipHostMalloc(reinterpret_cast<void**>(&w->h_err), 64, hipHostMallocMapped);
    if (e == hipSuccess) {
        *w->h_err = 0;
        e = hipHostGetDevicePointer(reinterpret_cast<void**>(&w->d_err), w->h_err, 0);
    }
    if (e != hipSuccess) {
        const int st = fail(MS_HIP_ERR_HIP, "[ms_hip] weight allocation failed: %s", hipGetErrorString(e));
        free_weights(*w);
        delete w;
        return st;
    }
    *out = w;
    return MS_HIP_OK;
}

int finish_create(Weights* w, int st, void** out_handle)
{
    if (!st) st = check_pipe_scales(*w);
    if (!st && w->d_wexp) {   // row exponents of the general GEMM
        hipLaunchKernelGGL(weight_row_exponent_kernel, dim3((w->N + 255) / 256), dim3(256), 0, nullptr, raw_layout(*w),
                           w->d_wexp);
        hipError_t e = hipGetLastError();
        if (e == hipSuccess) e = hipDeviceSynchronize();
        if (e != hipSuccess) st = fail(MS_HIP_ERR_HIP, "[ms_hip] weight exponents failed: %s", hipGetErrorString(e));
    }
    if (st) {
        free_weights(*w);
        delete w;
        return st;
    }
    {
        std::lock_guard<std::mutex> lock(g_live_mu);
        g_live.insert(w);
    }
    *out_handle = w;
    return MS_HIP_OK;
}

// ---- the allocation-free entry's scratch ---------------------------------------------------
// A file-scope device array: every GPU the library runs on holds its own copy from the
// moment the code object is loaded there until the process ends. Host code never uses
// the name `scratch` as an address (in host code it is only a stand-in for the symbol):
// the device address comes from hipGetSymbolAddress, once per device, and everything on
// the host (kernel arguments, fills) uses that pointer.
constexpr size_t kScratchDataBytes = (size_t)96 << 20;   // fp16 activations, exponents, partial sums
constexpr size_t kScratchCntInts = (size_t)64 << 10;      // split-K counters
__device__ __align__(256) uint8_t scratch[kScratchDataBytes + kScratchCntInts * sizeof(int)];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
uint8_t* g_scratch_ptr[kMaxDevices] = {};

// The device address of this device's scratch (device `dev` current), looked up once.
int scratch_for(int dev, uint8_t** out)
{
    if (dev < 0 || dev >= kMaxDevices) return fail(MS_HIP_ERR_INVALID, "[ms_hip] device %d out of range", dev);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return fail(MS_HIP_ERR_HIP, "[ms_hip] hipGetSymbolAddress(scratch) failed: %s", hipGetErrorString(e));
        g_scratch_ptr[dev] = static_cast<uint8_t*>(p);
    }
    *out = g_scratch_ptr[dev];
    return MS_HIP_OK;
}

}  // namespace

// =========================================================================================
extern "C" {

int ms_hip_available(void) { return disabled() ? 0 : device_info().ok; }

int ms_hip_debug_force_failure(int on)
{
    forced_failure().store(on ? 1 : 0, std::memory_order_relaxed);
    return MS_HIP_OK;
}

const char* ms_hip_device_name(void) { return device_info().name.c_str(); }

const char* ms_hip_build_info(void)
{
    return "ms_hip_nbits (hipcc " __VERSION__ ", --offload-arch=gfx950, -ffp-contract=off)";
}

const char* ms_hip_last_error(void) { return g_last_error.c_str(); }

int ms_hip_nbits_check(int N, int K, int bits, int block_size, int64_t b_len, int64_t scales_len, int zp_kind,
                       int64_t zp_len, int64_t a_last_dim)
{
    return check_impl(N, K, bits, block_size, b_len, scales_len, zp_kind, zp_len, a_last_dim);
}

int ms_hip_nbits_weights_create_ex(const uint8_t* bq, int64_t bq_len, const void* scales, int64_t scales_len,
                                   int scales_type, const void* zero_points, int64_t zp_len, int zp_type, int N, int K,
                                   int bits, int block_size, void** out_handle)
{
    if (!out_handle) return fail(MS_HIP_ERR_INVALID, "[ms_hip] out_handle is null");
    *out_handle = nullptr;
    if (scales_type != MS_HIP_DTYPE_F32 && scales_type != MS_HIP_DTYPE_F16)
        return fail(MS_HIP_ERR_INVALID, "[ms_hip] scales must be Float32 or Float16");
    if (!zero_points) zp_type = MS_HIP_DTYPE_NONE;
    const int zp_kind = zp_type == MS_HIP_DTYPE_NONE ? 0 : zp_type == MS_HIP_DTYPE_U8 ? 1
                      : (zp_type == MS_HIP_DTYPE_F32 || zp_type == MS_HIP_DTYPE_F16) ? 2 : 3;
    int st = check_impl(N, K, bits, block_size, bq_len, scales_len, zp_kind, zp_len, -1);
    if (st) return st;
    if (!bq || !scales) return fail(MS_HIP_ERR_INVALID, "[ms_hip] null B or scales pointer");
    if ((st = require_device())) return st;
    MS_HIP_CHECK(hipSetDevice(device_info().device));
    Weights* w = nullptr;
    if ((st = new_weights(N, K, bits, block_size, zp_kind, &w))) return st;
    hipError_t e = hipMemcpy(w->d_b, bq, (size_t)N * w->row_bytes, hipMemcpyHostToDevice);
    if (e == hipSuccess) e = upload_f32(w->d_scales, scales, (int64_t)N * w->nb, scales_type, hipMemcpyHostToDevice);
    if (e == hipSuccess && zp_kind == 1)
        e = hipMemcpy(w->d_zp, zero_points, (size_t)N * w->zrb, hipMemcpyHostToDevice);
    if (e == hipSuccess && zp_kind == 2)
        e = upload_f32(w->d_zpf, zero_points, (int64_t)N * w->nb, zp_type, hipMemcpyHostToDevice);
    if (e != hipSuccess) st = fail(MS_HIP_ERR_HIP, "[ms_hip] weight upload failed: %s", hipGetErrorString(e));
    return finish_create(w, st, out_handle);
}

}  // extern "C"

namespace {

// Streams bytes [offset, offset + length) of a file into device memory: pread into two
// pinned chunks alternately while the DMA engine copies the other one, so disk reads and
// PCIe transfers overlap and no host copy of the tensor is ever made.
int stream_file(const char* path, int64_t offset, int64_t length, void* dst)
{
    constexpr size_t kChunk = (size_t)8 << 20;
    if (length == 0) return MS_HIP_OK;
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return fail(MS_HIP_ERR_INVALID, "[ms_hip] cannot open '%s': %s", path, std::strerror(errno));
    uint8_t* pinned[2] = {nullptr, nullptr};
    hipEvent_t ev[2] = {nullptr, nullptr};
    hipStream_t s = nullptr;
    int st = MS_HIP_OK;
    hipError_t e = hipStreamCreateWithFlags(&s, hipStreamNonBlocking);
    for (int i = 0; i < 2 && e == hipSuccess; ++i) {
        e = hipHostMalloc(reinterpret_cast<void**>(&pinned[i]), kChunk, hipHostMallocDefault);
        if (e == hipSuccess) e = hipEventCreateWithFlags(&ev[i], hipEventDisableTiming);
    }
    if (e != hipSuccess) st = fail(MS_HIP_ERR_HIP, "[ms_hip] staging set-up failed: %s", hipGetErrorString(e));
    int64_t done = 0;
    for (int i = 0; st == MS_HIP_OK && done < length; ++i) {
        const int b = i & 1;
        if (i >= 2 && (e = hipEventSynchronize(ev[b])) != hipSuccess) {
            st = fail(MS_HIP_ERR_HIP, "[ms_hip] staging copy failed: %s", hipGetErrorString(e));
            break;
        }
        const size_t n = (size_t)std::min<int64_t>((int64_t)kChunk, length - done);
        size_t got = 0;
        while (got < n) {
            const ssize_t r = pread(fd, pinned[b] + got, n - got, (off_t)(offset + done + (int64_t)got));
            if (r < 0 && errno == EINTR) continue;
            if (r <= 0) {
                st = fail(MS_HIP_ERR_INVALID, "[ms_hip] '%s' ends before byte %lld", path,
                          (long long)(offset + length));
                break;
            }
            got += (size_t)r;
        }
        if (st) break;
        e = hipMemcpyAsync(static_cast<uint8_t*>(dst) + done, pinned[b], n, hipMemcpyHostToDevice, s);
        if (e == hipSuccess) e = hipEventRecord(ev[b], s);
        if (e != hipSuccess) st = fail(MS_HIP_ERR_HIP, "[ms_hip] staging copy failed: %s", hipGetErrorString(e));
        done += (int64_t)n;
    }
    if (s) (void)hipStreamSynchronize(s);
    for (int i = 0; i < 2; ++i) {
        if (ev[i]) (void)hipEventDestroy(ev[i]);
        if (pinned[i]) (void)hipHostFree(pinned[i]);
    }
    if (s) (void)hipStreamDestroy(s);
    close(fd);
    return st;
}

int elem_bytes(int dtype) { return dtype == MS_HIP_DTYPE_F32 ? 4 : dtype == MS_HIP_DTYPE_F16 ? 2 : 1; }

// A file slice of n fp32 values, or of n fp16 values widened on the device.
int stream_file_f32(const ms_hip_file_slice& sl, int64_t n, float* dst)
{
    if (sl.dtype == MS_HIP_DTYPE_F32) return stream_file(sl.path, sl.offset, n * 4, dst);
    void* tmp = nullptr;
    hipError_t e = hipMalloc(&tmp, (size_t)n * 2);
    if (e != hipSuccess) return fail(MS_HIP_ERR_HIP, "[ms_hip] allocation failed: %s", hipGetErrorString(e));
    int st = stream_file(sl.path, sl.offset, n * 2, tmp);
    if (!st) {
        launch_widen(tmp, dst, n, nullptr);
        e = hipGetLastError();
        if (e == hipSuccess) e = hipDeviceSynchronize();
        if (e != hipSuccess) st = fail(MS_HIP_ERR_HIP, "[ms_hip] widening failed: %s", hipGetErrorString(e));
    }
    (void)hipFree(tmp);
    return st;
}

}  // namespace

extern "C" {

int ms_hip_nbits_weights_create_from_files(const ms_hip_file_slice* b, const ms_hip_file_slice* scales,
                                           const ms_hip_file_slice* zero_points, int N, int K, int bits,
                                           int block_size, void** out_handle)
{
    if (!out_handle) return fail(MS_HIP_ERR_INVALID, "[ms_hip] out_handle is null");
    *out_handle = nullptr;
    if (!b || !scales || !b->path || !scales->path)
        return fail(MS_HIP_ERR_INVALID, "[ms_hip] B and scales need a file slice");
    if (b->dtype != MS_HIP_DTYPE_U8) return fail(MS_HIP_ERR_INVALID, "Tensor dtype is not UInt8; expected UInt8.");
    if (scales->dtype != MS_HIP_DTYPE_F32 && scales->dtype != MS_HIP_DTYPE_F16)
        return fail(MS_HIP_ERR_INVALID, "[ms_hip] scales must be Float32 or Float16");
    const bool has_zp = zero_points && zero_points->path;
    const int zp_type = has_zp ? zero_points->dtype : MS_HIP_DTYPE_NONE;
    const int zp_kind = zp_type == MS_HIP_DTYPE_NONE ? 0 : zp_type == MS_HIP_DTYPE_U8 ? 1
                      : (zp_type == MS_HIP_DTYPE_F32 || zp_type == MS_HIP_DTYPE_F16) ? 2 : 3;
    for (const ms_hip_file_slice* sl : {b, scales, has_zp ? zero_points : nullptr})
        if (sl && (sl->offset < 0 || sl->length < 0 || sl->length % elem_bytes(sl->dtype)))
            return fail(MS_HIP_ERR_INVALID, "[ms_hip] bad file slice of '%s'", sl->path);
    int st = check_impl(N, K, bits, block_size, b->length, scales->length / elem_bytes(scales->dtype), zp_kind,
                        has_zp ? zero_points->length / elem_bytes(zp_type) : 0, -1);
    if (st) return st;
    if ((st = require_device())) return st;
    MS_HIP_CHECK(hipSetDevice(device_info().device));
    Weights* w = nullptr;
    if ((st = new_weights(N, K, bits, block_size, zp_kind, &w))) return st;
    st = stream_file(b->path, b->offset, (int64_t)N * w->row_bytes, w->d_b);
    if (!st) st = stream_file_f32(*scales, (int64_t)N * w->nb, w->d_scales);
    if (!st && zp_kind == 1) st = stream_file(zero_points->path, zero_points->offset, (int64_t)N * w->zrb, w->d_zp);
    if (!st && zp_kind == 2) st = stream_file_f32(*zero_points, (int64_t)N * w->nb, w->d_zpf);
    return finish_create(w, st, out_handle);
}

int ms_hip_nbits_weights_create(const uint8_t* bq, int64_t bq_len, const float* scales, int64_t scales_len,
                                const uint8_t* zero_points, int64_t zp_len, int N, int K, int bits,
                                int block_size, void** out_handle)
{
    return ms_hip_nbits_weights_create_ex(bq, bq_len, scales, scales_len, MS_HIP_DTYPE_F32, zero_points, zp_len,
                                          zero_points ? MS_HIP_DTYPE_U8 : MS_HIP_DTYPE_NONE, N, K, bits, block_size,
                                          out_handle);
}

int ms_hip_nbits_weights_create_dev(const uint8_t* d_bq, const float* d_scales, const uint8_t* d_zero_points,
                                    int N, int K, int bits, int block_size, void** out_handle)
{
    if (!out_handle) return fail(MS_HIP_ERR_INVALID, "[ms_hip] out_handle is null");
    *out_handle = nullptr;
    int st = check_impl(N, K, bits, block_size, (int64_t)N * ((K + block_size - 1) / block_size) *
                                                    ((block_size * bits + 7) / 8),
                        (int64_t)N * ((K + block_size - 1) / block_size), 0, 0, -1);
    if (st) return st;
    if (!d_bq || !d_scales) return fail(MS_HIP_ERR_INVALID, "[ms_hip] null B or scales pointer");
    if ((st = require_device())) return st;
    MS_HIP_CHECK(hipSetDevice(device_info().device));
    Weights* w = nullptr;
    if ((st = new_weights(N, K, bits, block_size, d_zero_points ? 1 : 0, &w))) return st;
    hipError_t e = hipMemcpy(w->d_b, d_bq, (size_t)N * w->row_bytes, hipMemcpyDeviceToDevice);
    if (e == hipSuccess) e = hipMemcpy(w->d_scales, d_scales, (size_t)N * w->nb * sizeof(float), hipMemcpyDeviceToDevice);
    if (e == hipSuccess && d_zero_points)
        e = hipMemcpy(w->d_zp, d_zero_points, (size_t)N * w->zrb, hipMemcpyDeviceToDevice);
    if (e != hipSuccess) st = fail(MS_HIP_ERR_HIP, "[ms_hip] weight copy failed: %s", hipGetErrorString(e));
    return finish_create(w, st, out_handle);
}

int ms_hip_nbits_weights_destroy(void* handle)
{
    {
        std::lock_guard<std::mutex> lock(g_live_mu);
        if (!handle || !g_live.erase(handle)) return fail(MS_HIP_ERR_INVALID, "[ms_hip] invalid weights handle");
    }
    Weights* w = static_cast<Weights*>(handle);
    {
        std::lock_guard<std::mutex> lock(w->mu);
        if (w->stream) (void)hipStreamSynchronize(w->stream);
        // Device-pointer calls may still be in flight on other streams: their kernels use
        // the weights and the workspace until they finish.
        (void)hipDeviceSynchronize();
        free_weights(*w);
    }
    delete w;
    return MS_HIP_OK;
}

int ms_hip_nbits_weights_info(void* handle, int* N, int* K, int* bits, int* block_size, int* has_zp)
{
    Weights* w = from_handle(handle);
    if (!w) return fail(MS_HIP_ERR_INVALID, "[ms_hip] invalid weights handle");
    if (N) *N = w->N;
    if (K) *K = w->K;
    if (bits) *bits = w->bits;
    if (block_size) *block_size = w->bs;
    if (has_zp) *has_zp = w->has_zp;
    return MS_HIP_OK;
}

int ms_hip_nbits_gemm_dev(void* handle, const float* dA, float* dY, int M, void* stream)
{
    if (int st = gate()) return st;
    Weights* w = from_handle(handle);
    if (!w) return fail(MS_HIP_ERR_INVALID, "[ms_hip] invalid weights handle");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    const int st = take_device_error(*w, s);
    if (st) return st;
    return enqueue_gemm(*w, dA, dY, M, s);
}

int ms_hip_nbits_gemm_dev_f16(void* handle, const void* dA16, float* dY, int M, void* stream)
{
    if (int st = gate()) return st;
    Weights* w = from_handle(handle);
    if (!w) return fail(MS_HIP_ERR_INVALID, "[ms_hip] invalid weights handle");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    int st = take_device_error(*w, s);
    if (st) return st;
    if (M < 0) return fail(MS_HIP_ERR_INVALID, "MatMulNBits M must be non-negative; got %d.", M);
    if (M == 0) return MS_HIP_OK;
    if (!dA16 || !dY) return fail(MS_HIP_ERR_INVALID, "[ms_hip] null activation or output pointer");
    if ((reinterpret_cast<uintptr_t>(dA16) & 1) || (reinterpret_cast<uintptr_t>(dY) & 3))
        return fail(MS_HIP_ERR_INVALID, "[ms_hip] A must be 2-byte and Y 4-byte aligned");
    const Knobs kn = knobs_of(*w);
    KernelId k = choose_kernel(*w, kn, M);
    if ((st = resolve_rb(*w, kn, &k, M, s, true))) return st;
    size_t need_d = 0, need_c = 0;
    workspace_need(*w, kn, k, M, &need_d, &need_c);
    const size_t a_off = align256(need_d);
    Ws ws;
    const int r = ensure_ws(*w, a_off + (size_t)M * w->K * sizeof(float), need_c, s, &ws);
    if (r < 0) return fail(MS_HIP_ERR_HIP, "[ms_hip] workspace allocation failed: %s", hipGetErrorString(hipGetLastError()));
    if (r == 0)
        return fail(MS_HIP_ERR_UNSUPPORTED,
                    "[ms_hip] fp16 activations need the handle's workspace, which cannot grow under stream capture: "
                    "make one call of this size outside the capture first");
    float* a32 = reinterpret_cast<float*>(ws.data + a_off);
    launch_widen(dA16, a32, (int64_t)M * w->K, s);
    MS_HIP_CHECK(hipGetLastError());
    return launch_kernel(*w, kn, k, ws, a32, dY, M, s);
}

int ms_hip_nbits_gemm_dev_noalloc(void* handle, const float* dA, float* dY, int M, void* stream)
{
    if (int st = gate()) return st;
    Weights* w = from_handle(handle);
    if (!w) return fail(MS_HIP_ERR_INVALID, "[ms_hip] invalid weights handle");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    int st = take_device_error(*w, s);
    if (st) return st;
    if ((st = check_call(dA, dY, M)) || M == 0) return st;
    const Knobs kn = knobs_of(*w);
    KernelId k = choose_kernel(*w, kn, M);
    // the chunk-major scales are not built here (that allocates): without them, mfma_w4
    if ((st = resolve_rb(*w, kn, &k, M, s, false))) return st;
    size_t need_d = 0, need_c = 0;
    workspace_need(*w, kn, k, M, &need_d, &need_c);
    if (need_d > kScratchDataBytes || need_c > kScratchCntInts)
        return fail(MS_HIP_ERR_INVALID,
                    "[ms_hip] this call (M=%d, N=%d, K=%d) needs %zu bytes and %zu counters of workspace; the "
                    "allocation-free entry's fixed scratch holds %zu bytes and %zu counters (use "
                    "ms_hip_nbits_gemm_dev)",
                    M, w->N, w->K, need_d, need_c, kScratchDataBytes, kScratchCntInts);
    Ws ws;
    if (need_d || need_c) {
        int dev = -1;
        MS_HIP_CHECK(hipGetDevice(&dev));
        if (dev != w->device)
            return fail(MS_HIP_ERR_INVALID, "[ms_hip] the current device (%d) is not the handle's (%d)", dev,
                        w->device);
        uint8_t* base = nullptr;
        if ((st = scratch_for(dev, &base))) return st;
        ws.data = base;
        ws.data_bytes = kScratchDataBytes;
        ws.cnt = reinterpret_cast<int*>(base + kScratchDataBytes);
        ws.cnt_ints = kScratchCntInts;
        // The scratch keeps whatever the last call left: the counters this call uses start
        // at zero (a fill kernel, which a captured graph can hold).
        if ((st = zero_ints(ws.cnt, (int64_t)need_c, s))) return st;
    }
    return launch_kernel(*w, kn, k, ws, dA, dY, M, s);
}

int ms_hip_nbits_device_error(void* handle)
{
    Weights* w = from_handle(handle);
    if (!w) return fail(MS_HIP_ERR_INVALID, "[ms_hip] invalid weights handle");
    return take_device_error(*w, nullptr);
}

int ms_hip_nbits_gemm_dev_batch(void* const* handles, const float* const* dA, float* const* dY, int count, int M,
                                void* stream)
{
    if (int st = gate()) return st;
    if (count < 0 || (count > 0 && (!handles || !dA || !dY)))
        return fail(MS_HIP_ERR_INVALID, "[ms_hip] invalid batch arguments");
    std::vector<Weights*> ws((size_t)count);
    for (int i = 0; i < count; ++i)
        if (!(ws[i] = from_handle(handles[i])))
            return fail(MS_HIP_ERR_INVALID, "[ms_hip] invalid weights handle at batch index %d", i);
    const hipStream_t s = static_cast<hipStream_t>(stream);
    for (int i = 0; i < count; ++i) {
        const int st = take_device_error(*ws[i], s);
        if (st) return st;
    }
    // The prefill kernels' fp16 copy of an input, shared by the calls that read it (gate and
    // up at M > 16: one conversion instead of two). The copy sits in the workspace of the
    // handle that made it; a later call on that same handle could regrow the workspace, so
    // the copy is dropped before such a call.
    AConv conv;
    const Weights* conv_owner = nullptr;
    for (int i = 0; i < count;) {
        int ci = -1;
        const int n = batch_group(ws.data() + i, dA + i, count - i, M, &ci);
        if (n > 1) {
            GemvMember mem[kGemvMaxOps];
            for (int j = 0; j < n; ++j) {
                if (!dY[i + j] || (reinterpret_cast<uintptr_t>(dY[i + j]) & 3))
                    return fail(MS_HIP_ERR_INVALID, "[ms_hip] null or misaligned output at batch index %d", i + j);
                mem[j] = GemvMember{ws[i + j], dY[i + j]};
            }
            const int st = launch_gemv_group(mem, n, dA[i], M, ci, s);
            if (st) return st;
        } else {
            if (ws[i] == conv_owner) {
                conv = AConv{};
                conv_owner = nullptr;
            }
            const uint32_t* before = conv.a16;
            const int st = enqueue_gemm(*ws[i], dA[i], dY[i], M, s, &conv);
            if (st) return st;
            if (conv.a16 != before) conv_owner = ws[i];
        }
        i += n;
    }
    return MS_HIP_OK;
}

int ms_hip_nbits_gemm_dev_swiglu(void* gate_handle, void* up_handle, const float* dA, float* dH, int M,
                                 void* stream)
{
    if (int st = gate()) return st;
    Weights* wg = from_handle(gate_handle);
    Weights* wu = from_handle(up_handle);
    if (!wg || !wu) return fail(MS_HIP_ERR_INVALID, "[ms_hip] invalid weights handle");
    if (M < 0) return fail(MS_HIP_ERR_INVALID, "[ms_hip] M must be non-negative; got %d", M);
    if (wg->K != wu->K || wg->N != wu->N || wg->device != wu->device)
        return fail(MS_HIP_ERR_INVALID,
                    "[ms_hip] swiglu: the gate and up projections must share K, N and the device (got K=%d/%d, N=%d/%d)",
                    wg->K, wu->K, wg->N, wu->N);
    if (M == 0) return MS_HIP_OK;
    if (!dA || !dH || (reinterpret_cast<uintptr_t>(dH) & 3))
        return fail(MS_HIP_ERR_INVALID, "[ms_hip] swiglu: null or misaligned activations or output");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (int st = take_device_error(*wg, s)) return st;
    if (int st = take_device_error(*wu, s)) return st;
    int ci = -1;
    if (swiglu_fused_config(*wg, *wu, dA, M, &ci)) return launch_gemv_swiglu(*wg, *wu, dA, dH, ci, s);
    // Otherwise the three steps: gate into H, up into the gate handle's workspace, then the
    // SiLU-Mul in place (the same roundings as the fused form).
    if (int st = enqueue_gemm(*wg, dA, dH, M, s)) return st;
    Ws ws;
    const int got = ensure_ws(*wg, (size_t)M * wg->N * sizeof(float), 0, s, &ws);
    if (got < 0) return fail(MS_HIP_ERR_HIP, "[ms_hip] swiglu: workspace allocation failed");
    if (got == 0)
        return fail(MS_HIP_ERR_UNSUPPORTED,
                    "[ms_hip] swiglu: this call needs the gate handle's workspace to grow, which a captured stream "
                    "cannot do; make the call once outside capture first");
    float* dU = reinterpret_cast<float*>(ws.data);
    if (int st = enqueue_gemm(*wu, dA, dU, M, s)) return st;
    const int64_t n = (int64_t)M * wg->N;
    hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)std::min<int64_t>((n + 255) / 256, 8192)), dim3(256), 0, s,
                       dH, dU, dH, n);
    MS_HIP_CHECK(hipGetLastError());
    return MS_HIP_OK;
}

int ms_hip_nbits_swiglu_launch_info(void* gate_handle, void* up_handle, const float* dA, int M, int* fused,
                                    int* grid, int* block)
{
    Weights* wg = from_handle(gate_handle);
    Weights* wu = from_handle(up_handle);
    if (!wg || !wu) return fail(MS_HIP_ERR_INVALID, "[ms_hip] invalid weights handle");
    if (M <= 0) return fail(MS_HIP_ERR_INVALID, "[ms_hip] M must be positive; got %d", M);
    int ci = -1;
    const bool f = wg->K == wu->K && swiglu_fused_config(*wg, *wu, dA, M, &ci);
    const int rows = f ? gemv_rows(kGemvConfigs[ci]) / 2 : 1;
    if (fused) *fused = f ? 1 : 0;
    if (grid) *grid = f ? (wg->N + rows - 1) / rows : 0;
    if (block) *block = f ? kGemvConfigs[ci].waves * kWave : 0;
    return MS_HIP_OK;
}

// ---- SkipSimplifiedLayerNormalization fused into the projections that read its output ----
namespace {

bool ranges_overlap(const void* a, const void* b, size_t bytes)
{
    if (!a || !b) return false;
    const uintptr_t x = reinterpret_cast<uintptr_t>(a), y = reinterpret_cast<uintptr_t>(b);
    return x < y + bytes && y < x + bytes;
}

// Validation shared by the two entries: the norm's buffers (M rows of K) and their overlaps.
int skipnorm_check(const char* what, const float* dX, const float* dSkip, const float* dGamma, const float* dNorm,
                   const float* dSum, int M, int K)
{
    if (!dX || !dSkip || !dGamma || !dNorm)
        return fail(MS_HIP_ERR_INVALID, "[ms_hip] %s: null input, skip, gamma or normed output", what);
    for (const void* q : {(const void*)dX, (const void*)dSkip, (const void*)dGamma, (const void*)dNorm,
                          (const void*)dSum})
        if (reinterpret_cast<uintptr_t>(q) & 3)
            return fail(MS_HIP_ERR_INVALID, "[ms_hip] %s: buffers must be 4-byte aligned", what);
    const size_t bytes = (size_t)M * K * sizeof(float);
    for (const float* o : {dNorm, dSum})
        for (const float* i : {dX, dSkip})
            if (ranges_overlap(o, i, bytes))
                return fail(MS_HIP_ERR_INVALID,
                            "[ms_hip] %s: the normed output and the sum must not overlap the input or the skip", what);
    if (ranges_overlap(dNorm, dSum, bytes))
        return fail(MS_HIP_ERR_INVALID, "[ms_hip] %s: the normed output and the sum must not overlap", what);
    return MS_HIP_OK;
}

// A projection's output (M rows of N) may not overlap the norm's buffers (M rows of K):
// workgroups still reading X or Skip, or the normed rows, while others store Y.
int skipnorm_check_out(const char* what, const float* dY, int N, const float* dX, const float* dSkip,
                       const float* dNorm, const float* dSum, int M, int K)
{
    const uintptr_t y = reinterpret_cast<uintptr_t>(dY), ye = y + (size_t)M * N * sizeof(float);
    for (const float* q : {dX, dSkip, dNorm, dSum}) {
        if (!q) continue;
        const uintptr_t a = reinterpret_cast<uintptr_t>(q), ae = a + (size_t)M * K * sizeof(float);
        if (y < ae && a < ye)
            return fail(MS_HIP_ERR_INVALID, "[ms_hip] %s: an output must not overlap the input, skip, normed rows or sum",
                        what);
    }
    return MS_HIP_OK;
}

bool aligned16_all(std::initializer_list<const void*> ps)
{
    for (const void* q : ps)
        if (reinterpret_cast<uintptr_t>(q) & 15) return false;
    return true;
}

// The fused launch of the batch form: M = 1, every handle groupable with the first (at most
// kGemvMaxOps), a gemv_w4 config for their rows whose threads cover two per chunk, and
// 16-byte aligned norm buffers. *ci receives the config.
bool skipnorm_batch_fused(Weights* const* ws, int count, const float* dX, const float* dSkip, const float* dGamma,
                          const float* dNorm, const float* dSum, int M, int* ci)
{
    if (M != 1 || count < 1 || count > kGemvMaxOps) return false;
    if (!aligned16_all({dX, dSkip, dGamma, dNorm, dSum})) return false;
    const Weights& w0 = *ws[0];
    if (!gemv_groupable(w0, w0)) return false;
    int ntot = 0;
    for (int i = 0; i < count; ++i) {
        if (!gemv_groupable(w0, *ws[i])) return false;
        ntot += ws[i]->N;
    }
    const Knobs kn = knobs_of(w0);
    if (kn.skinny() == 2) return false;
    const int c = pick_gemv_config(w0, kn, 1, ntot);
    if (c < 0 || !norm_fits(kGemvConfigs[c], w0.K) || !kGemvNormTable[0][l_slot(w0)][c]) return false;
    *ci = c;
    return true;
}

bool skipnorm_swiglu_fused(const Weights& wg, const Weights& wu, const float* dX, const float* dSkip,
                           const float* dGamma, const float* dNorm, const float* dSum, int M, int* ci)
{
    int c = -1;
    if (!aligned16_all({dX, dSkip, dGamma, dNorm, dSum}) || !swiglu_fused_config(wg, wu, dNorm, M, &c)) return false;
    if (!norm_fits(kGemvConfigs[c], wg.K) || !kGemvNormTable[1][l_slot(wg)][c]) return false;
    *ci = c;
    return true;
}

}  // namespace

int ms_hip_nbits_gemm_dev_skipnorm(void* const* handles, int count, const float* dX, const float* dSkip,
                                   const float* dGamma, float eps, float* dNorm, float* dSum, float* const* dY, int M,
                                   void* stream)
{
    if (int st = gate()) return st;
    if (count <= 0 || !handles || !dY) return fail(MS_HIP_ERR_INVALID, "[ms_hip] skipnorm: invalid batch arguments");
    std::vector<Weights*> ws((size_t)count);
    for (int i = 0; i < count; ++i)
        if (!(ws[i] = from_handle(handles[i])))
            return fail(MS_HIP_ERR_INVALID, "[ms_hip] invalid weights handle at batch index %d", i);
    if (M < 0) return fail(MS_HIP_ERR_INVALID, "[ms_hip] M must be non-negative; got %d", M);
    const int K = ws[0]->K;
    for (int i = 1; i < count; ++i)
        if (ws[i]->K != K || ws[i]->device != ws[0]->device)
            return fail(MS_HIP_ERR_INVALID, "[ms_hip] skipnorm: every projection must share K and the device");
    if (M == 0) return MS_HIP_OK;
    if (int st = skipnorm_check("skipnorm", dX, dSkip, dGamma, dNorm, dSum, M, K)) return st;
    for (int i = 0; i < count; ++i) {
        if (!dY[i] || (reinterpret_cast<uintptr_t>(dY[i]) & 3))
            return fail(MS_HIP_ERR_INVALID, "[ms_hip] null or misaligned output at batch index %d", i);
        if (int st = skipnorm_check_out("skipnorm", dY[i], ws[i]->N, dX, dSkip, dNorm, dSum, M, K)) return st;
    }
    const hipStream_t s = static_cast<hipStream_t>(stream);
    for (int i = 0; i < count; ++i)
        if (int st = take_device_error(*ws[i], s)) return st;
    int ci = -1;
    if (skipnorm_batch_fused(ws.data(), count, dX, dSkip, dGamma, dNorm, dSum, M, &ci)) {
        GemvMember mem[kGemvMaxOps];
        for (int i = 0; i < count; ++i) mem[i] = GemvMember{ws[i], dY[i]};
        const NormArgs na{dX, dSkip, dGamma, dSum, dNorm, eps};
        return launch_gemv_group(mem, count, dX, 1, ci, s, &na);
    }
    // Otherwise the norm, then the batch on its output.
    if (int st = ms_hip_skip_rmsnorm(dX, dSkip, dGamma, nullptr, nullptr, dNorm, dSum, nullptr, M, K, eps, stream))
        return st;
    std::vector<const float*> dA((size_t)count, dNorm);
    return ms_hip_nbits_gemm_dev_batch(handles, dA.data(), dY, count, M, stream);
}

int ms_hip_nbits_gemm_dev_skipnorm_swiglu(void* gate_handle, void* up_handle, const float* dX, const float* dSkip,
                                          const float* dGamma, float eps, float* dNorm, float* dSum, float* dH, int M,
                                          void* stream)
{
    if (int st = gate()) return st;
    Weights* wg = from_handle(gate_handle);
    Weights* wu = from_handle(up_handle);
    if (!wg || !wu) return fail(MS_HIP_ERR_INVALID, "[ms_hip] invalid weights handle");
    if (M < 0) return fail(MS_HIP_ERR_INVALID, "[ms_hip] M must be non-negative; got %d", M);
    if (wg->K != wu->K || wg->N != wu->N || wg->device != wu->device)
        return fail(MS_HIP_ERR_INVALID,
                    "[ms_hip] swiglu: the gate and up projections must share K, N and the device (got K=%d/%d, N=%d/%d)",
                    wg->K, wu->K, wg->N, wu->N);
    if (M == 0) return MS_HIP_OK;
    if (int st = skipnorm_check("skipnorm_swiglu", dX, dSkip, dGamma, dNorm, dSum, M, wg->K)) return st;
    if (!dH || (reinterpret_cast<uintptr_t>(dH) & 3))
        return fail(MS_HIP_ERR_INVALID, "[ms_hip] swiglu: null or misaligned activations or output");
    if (int st = skipnorm_check_out("skipnorm_swiglu", dH, wg->N, dX, dSkip, dNorm, dSum, M, wg->K)) return st;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    if (int st = take_device_error(*wg, s)) return st;
    if (int st = take_device_error(*wu, s)) return st;
    int ci = -1;
    if (skipnorm_swiglu_fused(*wg, *wu, dX, dSkip, dGamma, dNorm, dSum, M, &ci)) {
        const NormArgs na{dX, dSkip, dGamma, dSum, dNorm, eps};
        return launch_gemv_swiglu(*wg, *wu, dX, dH, ci, s, &na);
    }
    if (int st = ms_hip_skip_rmsnorm(dX, dSkip, dGamma, nullptr, nullptr, dNorm, dSum, nullptr, M, wg->K, eps, stream))
        return st;
    return ms_hip_nbits_gemm_dev_swiglu(gate_handle, up_handle, dNorm, dH, M, stream);
}

int ms_hip_nbits_skipnorm_launch_info(void* const* handles, int count, int swiglu, const float* dX,
                                      const float* dSkip, const float* dGamma, const float* dNorm, const float* dSum,
                                      int M, int* fused, int* grid, int* block)
{
    if (count <= 0 || !handles || (swiglu && count != 2))
        return fail(MS_HIP_ERR_INVALID, "[ms_hip] skipnorm: invalid batch arguments");
    std::vector<Weights*> ws((size_t)count);
    for (int i = 0; i < count; ++i)
        if (!(ws[i] = from_handle(handles[i])))
            return fail(MS_HIP_ERR_INVALID, "[ms_hip] invalid weights handle at batch index %d", i);
    int ci = -1, gr = 0, rows = 1;
    bool f;
    if (swiglu) {
        f = ws[0]->K == ws[1]->K && ws[0]->N == ws[1]->N &&
            skipnorm_swiglu_fused(*ws[0], *ws[1], dX, dSkip, dGamma, dNorm, dSum, M, &ci);
        if (f) gr = (ws[0]->N + gemv_rows(kGemvConfigs[ci]) / 2 - 1) / (gemv_rows(kGemvConfigs[ci]) / 2);
    } else {
        f = skipnorm_batch_fused(ws.data(), count, dX, dSkip, dGamma, dNorm, dSum, M, &ci);
        if (f) {
            rows = gemv_rows(kGemvConfigs[ci]);
            for (int i = 0; i < count; ++i) gr += (ws[i]->N + rows - 1) / rows;
        }
    }
    if (fused) *fused = f ? 1 : 0;
    if (grid) *grid = f ? gr : 0;
    if (block) *block = f ? kGemvConfigs[ci].waves * kWave : 0;
    return MS_HIP_OK;
}

int ms_hip_nbits_batch_launch_info(void* const* handles, const float* const* dA, int count, int M, int* calls,
                                   int* kernel_id, int* lanes_per_row, int* grid, int* block)
{
    if (count <= 0 || !handles || !dA) return fail(MS_HIP_ERR_INVALID, "[ms_hip] invalid batch arguments");
    std::vector<Weights*> ws((size_t)count);
    for (int i = 0; i < count; ++i)
        if (!(ws[i] = from_handle(handles[i])))
            return fail(MS_HIP_ERR_INVALID, "[ms_hip] invalid weights handle at batch index %d", i);
    if (M <= 0) return fail(MS_HIP_ERR_INVALID, "[ms_hip] M must be positive; got %d", M);
    int ci = -1;
    const int n = batch_group(ws.data(), dA, count, M, &ci);
    if (calls) *calls = n;
    if (n == 1) return ms_hip_nbits_launch_info(handles[0], M, kernel_id, lanes_per_row, grid, block);
    const GemvConfig& c = kGemvConfigs[ci];
    int gr = 0;
    for (int j = 0; j < n; ++j) gr += (ws[j]->N + gemv_rows(c) - 1) / gemv_rows(c);
    if (kernel_id) *kernel_id = kGemv;
    if (lanes_per_row) *lanes_per_row = c.G;
    if (grid) *grid = gr;
    if (block) *block = c.waves * kWave;
    return MS_HIP_OK;
}

}  // extern "C"

namespace {

constexpr size_t kDirectStageBytes = (size_t)1 << 20;

// Device copy of n floats from pinned host memory (read across PCIe by the kernel).
__global__ __launch_bounds__(256) void stage_copy_kernel(const float* __restrict__ src, float* __restrict__ dst,
                                                         int64_t n)
{
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        dst[i] = src[i];
}

// The synchronous host-pointer call (exact or W4A8): pinned staging, one stream, one sync.
int host_gemm(void* handle, const float* a_host, float* y_host, int M, bool w4a8)
{
    if (int st = gate()) return st;
    Weights* w = from_handle(handle);
    if (!w) return fail(MS_HIP_ERR_INVALID, "[ms_hip] invalid weights handle");
    if (M < 0) return fail(MS_HIP_ERR_INVALID, "MatMulNBits M must be non-negative; got %d.", M);
    if (M == 0) return MS_HIP_OK;
    if (!a_host || !y_host) return fail(MS_HIP_ERR_INVALID, "[ms_hip] null activation or output pointer");
    std::lock_guard<std::mutex> lock(w->mu);
    MS_HIP_CHECK(hipSetDevice(w->device));
    if (!w->stream) MS_HIP_CHECK(hipStreamCreateWithFlags(&w->stream, hipStreamNonBlocking));
    const size_t a_bytes = (size_t)M * w->K * sizeof(float);
    const size_t a_span = align256(a_bytes);
    const size_t y_bytes = (size_t)M * w->N * sizeof(float);
    // Device staging, and pinned host staging: the copies then run as DMA at full PCIe
    // rate instead of going through the runtime's pageable bounce buffers.
    if (w->stage_bytes < a_span + y_bytes) {
        if (w->d_stage) MS_HIP_CHECK(hipFree(w->d_stage));
        w->d_stage = nullptr;
        w->stage_bytes = 0;
        MS_HIP_CHECK(hipMalloc(&w->d_stage, a_span + y_bytes));
        w->stage_bytes = a_span + y_bytes;
    }
    if (w->h_stage_bytes < a_span + y_bytes) {
        if (w->h_stage) MS_HIP_CHECK(hipHostFree(w->h_stage));
        w->h_stage = nullptr;
        w->h_stage_bytes = 0;
        MS_HIP_CHECK(hipHostMalloc(reinterpret_cast<void**>(&w->h_stage), a_span + y_bytes, hipHostMallocDefault));
        w->h_stage_bytes = a_span + y_bytes;
    }
    float* dA = w->d_stage;
    float* dY = reinterpret_cast<float*>(reinterpret_cast<char*>(w->d_stage) + a_span);
    float* hA = reinterpret_cast<float*>(w->h_stage);
    float* hY = reinterpret_cast<float*>(w->h_stage + a_span);
    std::memcpy(hA, a_host, a_bytes);
    // A crosses PCIe as a DMA copy through the pinned staging. For small calls (decode:
    // A and Y up to kDirectStageBytes each) the GEMM stores Y straight into the pinned
    // (device-mapped) host buffer, which saves the copy back and its set-up: every kernel
    // writes Y once and never reads it back. Measured on the 7B gate at M=1, eight handles
    // called in turn under a rotating weight stream, medians of per-call times: 32 us per
    // call with direct Y against 42 us with both copies; a kernel pulling A from the pinned
    // buffer instead of the DMA copy gained nothing. Large calls keep both DMA copies, which
    // stream at full PCIe rate without holding the GEMM's waves. Knob 10 selects the
    // staging for measurements.
    const bool small = a_bytes <= kDirectStageBytes && y_bytes <= kDirectStageBytes;
    const int mode = knobs_of(*w).host_staging() > 0 ? knobs_of(*w).host_staging() - 1 : (small ? 2 : 0);
    const bool direct_a = mode & 1, direct = mode & 2;
    if (direct_a) {
        const int64_t n = (int64_t)M * w->K;
        hipLaunchKernelGGL(stage_copy_kernel, dim3((unsigned)std::min<int64_t>((n + 255) / 256, 1024)), dim3(256), 0,
                           w->stream, hA, dA, n);
        MS_HIP_CHECK(hipGetLastError());
    } else {
        MS_HIP_CHECK(hipMemcpyAsync(dA, hA, a_bytes, hipMemcpyHostToDevice, w->stream));
    }
    float* yt = direct ? hY : dY;
    int st = take_device_error(*w, w->stream);
    if (!st) st = w4a8 ? enqueue_w4a8(*w, dA, yt, M, w->stream) : enqueue_gemm(*w, dA, yt, M, w->stream);
    if (st) {
        (void)hipStreamSynchronize(w->stream);
        return st;
    }
    if (!direct) MS_HIP_CHECK(hipMemcpyAsync(hY, dY, y_bytes, hipMemcpyDeviceToHost, w->stream));
    MS_HIP_CHECK(hipStreamSynchronize(w->stream));
    if ((st = take_device_error(*w, w->stream))) {
        (void)hipStreamSynchronize(w->stream);
        return st;
    }
    std::memcpy(y_host, hY, y_bytes);
    return MS_HIP_OK;
}

}  // namespace

extern "C" {

int ms_hip_nbits_gemm(void* handle, const float* a_host, float* y_host, int M)
{
    return host_gemm(handle, a_host, y_host, M, false);
}

int ms_hip_nbits_gemm_w4a8(void* handle, const float* a_host, float* y_host, int M)
{
    return host_gemm(handle, a_host, y_host, M, true);
}

int ms_hip_nbits_gemm_dev_w4a8(void* handle, const float* dA, float* dY, int M, void* stream)
{
    if (int st = gate()) return st;
    Weights* w = from_handle(handle);
    if (!w) return fail(MS_HIP_ERR_INVALID, "[ms_hip] invalid weights handle");
    const hipStream_t s = static_cast<hipStream_t>(stream);
    int st = take_device_error(*w, s);
    if (st) return st;
    return enqueue_w4a8(*w, dA, dY, M, s);
}

int ms_hip_nbits_launch_info_w4a8(void* handle, int M, int* kernel_id, int* grid)
{
    Weights* w = from_handle(handle);
    if (!w) return fail(MS_HIP_ERR_INVALID, "[ms_hip] invalid weights handle");
    if (M <= 0) return fail(MS_HIP_ERR_INVALID, "[ms_hip] M must be positive; got %d", M);
    if (w->zp_float) return fail(MS_HIP_ERR_UNSUPPORTED, "[ms_hip] W4A8 takes packed or default zero points");
    const W4a8KernelId k = w4a8_kernel(*w, M);
    if (kernel_id) *kernel_id = (int)k;
    if (grid) *grid = w4a8_grid(*w, M, k);
    return MS_HIP_OK;
}

int ms_hip_qgemm_w4a8(const float* a, const uint8_t* bq, const float* scales, const uint8_t* zero_points, float* y,
                      int M, int N, int K, int bits, int block_size)
{
    if (int st = gate()) return st;
    if (N <= 0 || K <= 0 || (bits != 4 && bits != 8) || block_size <= 0)
        return check_impl(N, K, bits, block_size, 0, 0, 0, 0, -1);
    const int64_t nb = (K + block_size - 1) / block_size;
    const int64_t blob = (block_size * bits + 7) / 8;
    const int64_t zrb = (nb * bits + 7) / 8;
    void* h = nullptr;
    int st = ms_hip_nbits_weights_create(bq, (int64_t)N * nb * blob, scales, (int64_t)N * nb, zero_points,
                                         (int64_t)N * zrb, N, K, bits, block_size, &h);
    if (st) return st;
    st = ms_hip_nbits_gemm_w4a8(h, a, y, M);
    const std::string err = g_last_error;
    ms_hip_nbits_weights_destroy(h);
    if (st) g_last_error = err;
    return st;
}

int ms_hip_qgemm_nbits(const float* a, const uint8_t* bq, const float* scales, const uint8_t* zero_points,
                       float* y, int M, int N, int K, int bits, int block_size)
{
    if (int st = gate()) return st;
    // Buffer lengths are implied by the dimensions here, as in ms_qgemm_nbits.
    if (N <= 0 || K <= 0 || (bits != 4 && bits != 8) || block_size <= 0)
        return check_impl(N, K, bits, block_size, 0, 0, 0, 0, -1);
    const int64_t nb = (K + block_size - 1) / block_size;
    const int64_t blob = (block_size * bits + 7) / 8;
    const int64_t zrb = (nb * bits + 7) / 8;
    void* h = nullptr;
    int st = ms_hip_nbits_weights_create(bq, (int64_t)N * nb * blob, scales, (int64_t)N * nb, zero_points,
                                     (int64_t)N * zrb, N, K, bits, block_size, &h);
    if (st) return st;
    st = ms_hip_nbits_gemm(h, a, y, M);
    const std::string err = g_last_error;
    ms_hip_nbits_weights_destroy(h);
    if (st) g_last_error = err;
    return st;
}

int ms_hip_nbits_dequant_dev(void* handle, float* dW, void* stream)
{
    if (int st = gate()) return st;
    Weights* w = from_handle(handle);
    if (!w) return fail(MS_HIP_ERR_INVALID, "[ms_hip] invalid weights handle");
    if (!dW) return fail(MS_HIP_ERR_INVALID, "[ms_hip] null output pointer");
    const int64_t total = (int64_t)w->N * w->K;
    hipLaunchKernelGGL(nbits_dequant_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), raw_layout(*w), dW);
    MS_HIP_CHECK(hipGetLastError());
    return MS_HIP_OK;
}

int ms_hip_nbits_dequant(void* handle, float* w_host)
{
    if (int st = gate()) return st;
    Weights* w = from_handle(handle);
    if (!w) return fail(MS_HIP_ERR_INVALID, "[ms_hip] invalid weights handle");
    if (!w_host) return fail(MS_HIP_ERR_INVALID, "[ms_hip] null output pointer");
    MS_HIP_CHECK(hipSetDevice(w->device));
    const size_t bytes = (size_t)w->N * w->K * sizeof(float);
    float* dW = nullptr;
    MS_HIP_CHECK(hipMalloc(&dW, bytes));
    int st = ms_hip_nbits_dequant_dev(handle, dW, nullptr);
    if (!st) {
        hipError_t e = hipMemcpy(w_host, dW, bytes, hipMemcpyDeviceToHost);
        if (e != hipSuccess) st = fail(MS_HIP_ERR_HIP, "[ms_hip] dequant download failed: %s", hipGetErrorString(e));
    }
    (void)hipFree(dW);
    return st;
}

int ms_hip_alloc(void** dptr, int64_t bytes)
{
    if (!dptr || bytes < 0) return fail(MS_HIP_ERR_INVALID, "[ms_hip] invalid alloc arguments");
    int st = require_device();
    if (st) return st;
    MS_HIP_CHECK(hipMalloc(dptr, (size_t)(bytes ? bytes : 1)));
    return MS_HIP_OK;
}

int ms_hip_free(void* dptr)
{
    if (dptr) MS_HIP_CHECK(hipFree(dptr));
    return MS_HIP_OK;
}

int ms_hip_upload(void* dptr, const void* host, int64_t bytes)
{
    if (bytes < 0 || (bytes && (!dptr || !host))) return fail(MS_HIP_ERR_INVALID, "[ms_hip] invalid upload");
    if (bytes) MS_HIP_CHECK(hipMemcpy(dptr, host, (size_t)bytes, hipMemcpyHostToDevice));
    return MS_HIP_OK;
}

int ms_hip_download(void* host, const void* dptr, int64_t bytes)
{
    if (bytes < 0 || (bytes && (!dptr || !host))) return fail(MS_HIP_ERR_INVALID, "[ms_hip] invalid download");
    if (bytes) MS_HIP_CHECK(hipMemcpy(host, dptr, (size_t)bytes, hipMemcpyDeviceToHost));
    return MS_HIP_OK;
}

int ms_hip_sync(void)
{
    int st = require_device();
    if (st) return st;
    MS_HIP_CHECK(hipDeviceSynchronize());
    return MS_HIP_OK;
}

int ms_hip_set_gemv_lanes(int lanes_per_row) { return ms_hip_set_tuning(0, lanes_per_row); }

int ms_hip_set_tuning(int knob, int value)
{
    const int st = validate_knob(knob, value);
    if (st) return st;
    g_knob[knob].store(value, std::memory_order_relaxed);
    return MS_HIP_OK;
}

int ms_hip_nbits_set_tuning(void* handle, int knob, int value)
{
    Weights* w = from_handle(handle);
    if (!w) return fail(MS_HIP_ERR_INVALID, "[ms_hip] invalid weights handle");
    if (value != MS_HIP_TUNING_INHERIT) {
        const int st = validate_knob(knob, value);
        if (st) return st;
    } else if (knob < 0 || knob >= kNumKnobs) {
        return fail(MS_HIP_ERR_INVALID, "[ms_hip] invalid tuning knob %d", knob);
    }
    w->knob[knob].store(value, std::memory_order_relaxed);
    return MS_HIP_OK;
}

int ms_hip_nbits_debug_set_counters(void* handle, int value, int next_epoch_tag)
{
    Weights* w = from_handle(handle);
    if (!w) return fail(MS_HIP_ERR_INVALID, "[ms_hip] invalid weights handle");
    std::lock_guard<std::mutex> lock(w->mu);
    std::lock_guard<std::mutex> wlock(w->ws_mu);
    if (!w->ws.cnt) return fail(MS_HIP_ERR_INVALID, "[ms_hip] the handle has no split-K counters yet");
    MS_HIP_CHECK(hipDeviceSynchronize());
    int v = value;
    if (next_epoch_tag) {   // the tag the next split-K launch will carry
        const uint32_t e = g_epoch.load(std::memory_order_relaxed);
        v = (int)(e % 0x7FFFFFFEu) + 1;
    }
    // Pairs of (arrival tag, ready flag): tags set, flags cleared.
    std::vector<int> fill(w->ws.cnt_ints, 0);
    for (size_t i = 0; i < fill.size(); i += 2) fill[i] = v;
    MS_HIP_CHECK(hipMemcpy(w->ws.cnt, fill.data(), fill.size() * sizeof(int), hipMemcpyHostToDevice));
    return MS_HIP_OK;
}

int ms_hip_nbits_launch_info(void* handle, int M, int* kernel_id, int* lanes_per_row, int* grid, int* block)
{
    Weights* w = from_handle(handle);
    if (!w) return fail(MS_HIP_ERR_INVALID, "[ms_hip] invalid weights handle");
    if (M <= 0) return fail(MS_HIP_ERR_INVALID, "[ms_hip] M must be positive; got %d", M);
    const Knobs kn = knobs_of(*w);
    const KernelId kid = choose_kernel(*w, kn, M);
    int G = 0, gr = 0, bl = 256;
    switch (kid) {
        case kGeneric: gr = (int)(((int64_t)M * w->N + 255) / 256); break;
        case kGemvGeneral: gr = (w->N + kGenRowsPerWg - 1) / kGenRowsPerWg; G = 16; break;
        case kGemvW8: {
            const int ci = pick_gemv8_config(*w, kn, M);
            G = kGemv8Configs[ci].G;
            gr = gemv8_grid(*w, ci);
            bl = kGemv8Configs[ci].waves * kWave;
            break;
        }
        case kMfmaGeneral:
            gr = ((M + kGenBM - 1) / kGenBM) * ((w->N + kGenBN - 1) / kGenBN);
            gr = ((gr + kXcds - 1) / kXcds) * kXcds;
            break;
        case kSkinny: gr = ((w->N + kSkinnyRows - 1) / kSkinnyRows) * skinny_ksw(*w, kn); break;
        case kGemv: {
            const GemvConfig& c = kGemvConfigs[pick_gemv_config(*w, kn, M, w->N)];
            G = c.G;
            gr = (w->N + gemv_rows(c) - 1) / gemv_rows(c);
            bl = c.waves * kWave;
            break;
        }
        case kPanel: {
            const PanelShape s = panel_shape(*w, kn, M);
            G = s.G;
            gr = s.grid;
            bl = kPanelThreads;
            break;
        }
        case kRb:
        {
            const RbShape sh = rb_shape(*w, kn, M);
            gr = sh.tiles_m * sh.tiles_n * sh.ksw;
            gr = ((gr + kXcds - 1) / kXcds) * kXcds;
            G = 64 * sh.nf;   // reported as the tile width
        }
            break;
        case kPipe: {
            const PipeSplit sp = pipe_split(*w, kn, M);
            gr = kXcds * (sp.xu + sp.xv);
            break;
        }
        case kMfma: mfma_launch_shape(w->N, M, &gr, &bl); break;
    }
    if (kernel_id) *kernel_id = kid;
    if (lanes_per_row) *lanes_per_row = G;
    if (grid) *grid = gr;
    if (block) *block = bl;
    return MS_HIP_OK;
}

}  // extern "C"

// =========================================================================================
// Decoder-layer neighbours of MatMulNBits (device pointers, stream-ordered, no allocation).
namespace {

int elementwise_grid(int64_t n) { return (int)std::min<int64_t>((n + 255) / 256, 8192); }

bool misaligned4(const void* p) { return p && (reinterpret_cast<uintptr_t>(p) & 3); }
bool misaligned16(const void* p) { return p && (reinterpret_cast<uintptr_t>(p) & 15); }

}  // namespace

extern "C" {

int ms_hip_rmsnorm(const float* dX, const float* dScale, float* dY, float* dInvStd, int64_t rows, int norm, float eps,
                   void* stream)
{
    if (int st = gate()) return st;
    if (rows < 0 || norm <= 0 || rows > INT_MAX)
        return fail(MS_HIP_ERR_INVALID, "[ms_hip] rmsnorm needs 0 <= rows <= 2^31-1 and norm > 0 (rows=%lld, norm=%d)",
                    (long long)rows, norm);
    if (rows == 0) return MS_HIP_OK;
    if (!dX || !dScale || !dY) return fail(MS_HIP_ERR_INVALID, "[ms_hip] rmsnorm: null input, scale or output");
    if (misaligned4(dX) || misaligned4(dScale) || misaligned4(dY) || misaligned4(dInvStd))
        return fail(MS_HIP_ERR_INVALID, "[ms_hip] rmsnorm: buffers must be 4-byte aligned");
    const int vec = !misaligned16(dX) && !misaligned16(dScale) && !misaligned16(dY);
    hipLaunchKernelGGL(rmsnorm_kernel, dim3((unsigned)rows), dim3(kNormThreads), 0, static_cast<hipStream_t>(stream),
                       dX, dScale, dY, dInvStd, norm, eps, vec);
    MS_HIP_CHECK(hipGetLastError());
    return MS_HIP_OK;
}

int ms_hip_skip_rmsnorm(const float* dInput, const float* dSkip, const float* dGamma, const float* dBeta,
                        const float* dBias, float* dOut, float* dSum, float* dInvStd, int64_t rows, int norm,
                        float eps, void* stream)
{
    if (int st = gate()) return st;
    if (rows < 0 || norm <= 0 || rows > INT_MAX)
        return fail(MS_HIP_ERR_INVALID,
                    "[ms_hip] skip_rmsnorm needs 0 <= rows <= 2^31-1 and norm > 0 (rows=%lld, norm=%d)",
                    (long long)rows, norm);
    if (rows == 0) return MS_HIP_OK;
    if (!dInput || !dSkip || !dGamma || !dOut)
        return fail(MS_HIP_ERR_INVALID, "[ms_hip] skip_rmsnorm: null input, skip, gamma or output");
    for (const void* q : {(const void*)dInput, (const void*)dSkip, (const void*)dGamma, (const void*)dBeta,
                          (const void*)dBias, (const void*)dOut, (const void*)dSum, (const void*)dInvStd})
        if (misaligned4(q)) return fail(MS_HIP_ERR_INVALID, "[ms_hip] skip_rmsnorm: buffers must be 4-byte aligned");
    int vec = 1;
    for (const void* q : {(const void*)dInput, (const void*)dSkip, (const void*)dGamma, (const void*)dBeta,
                          (const void*)dBias, (const void*)dOut, (const void*)dSum})
        if (misaligned16(q)) vec = 0;
    hipLaunchKernelGGL(skip_rmsnorm_kernel, dim3((unsigned)rows), dim3(kNormThreads), 0,
                       static_cast<hipStream_t>(stream), dInput, dSkip, dGamma, dBeta, dBias, dOut, dSum, dInvStd,
                       norm, eps, vec);
    MS_HIP_CHECK(hipGetLastError());
    return MS_HIP_OK;
}

int ms_hip_silu_mul(const float* dGate, const float* dUp, float* dY, int64_t n, void* stream)
{
    if (int st = gate()) return st;
    if (n < 0) return fail(MS_HIP_ERR_INVALID, "[ms_hip] silu_mul: negative length");
    if (n == 0) return MS_HIP_OK;
    if (!dGate || !dUp || !dY) return fail(MS_HIP_ERR_INVALID, "[ms_hip] silu_mul: null buffer");
    hipLaunchKernelGGL(silu_mul_kernel, dim3(elementwise_grid(n)), dim3(256), 0, static_cast<hipStream_t>(stream),
                       dGate, dUp, dY, n);
    MS_HIP_CHECK(hipGetLastError());
    return MS_HIP_OK;
}

int ms_hip_add(const float* dA, const float* dB, float* dY, int64_t n, void* stream)
{
    if (int st = gate()) return st;
    if (n < 0) return fail(MS_HIP_ERR_INVALID, "[ms_hip] add: negative length");
    if (n == 0) return MS_HIP_OK;
    if (!dA || !dB || !dY) return fail(MS_HIP_ERR_INVALID, "[ms_hip] add: null buffer");
    hipLaunchKernelGGL(add_kernel, dim3(elementwise_grid(n)), dim3(256), 0, static_cast<hipStream_t>(stream), dA, dB,
                       dY, n);
    MS_HIP_CHECK(hipGetLastError());
    return MS_HIP_OK;
}

int ms_hip_sigmoid(const float* dX, float* dY, int64_t n, void* stream)
{
    if (int st = gate()) return st;
    if (n < 0) return fail(MS_HIP_ERR_INVALID, "[ms_hip] sigmoid: negative length");
    if (n == 0) return MS_HIP_OK;
    if (!dX || !dY) return fail(MS_HIP_ERR_INVALID, "[ms_hip] sigmoid: null buffer");
    hipLaunchKernelGGL(sigmoid_kernel, dim3(elementwise_grid(n)), dim3(256), 0, static_cast<hipStream_t>(stream), dX,
                       dY, n);
    MS_HIP_CHECK(hipGetLastError());
    return MS_HIP_OK;
}

int ms_hip_mul(const float* dA, const float* dB, float* dY, int64_t n, void* stream)
{
    if (int st = gate()) return st;
    if (n < 0) return fail(MS_HIP_ERR_INVALID, "[ms_hip] mul: negative length");
    if (n == 0) return MS_HIP_OK;
    if (!dA || !dB || !dY) return fail(MS_HIP_ERR_INVALID, "[ms_hip] mul: null buffer");
    hipLaunchKernelGGL(mul_kernel, dim3(elementwise_grid(n)), dim3(256), 0, static_cast<hipStream_t>(stream), dA, dB,
                       dY, n);
    MS_HIP_CHECK(hipGetLastError());
    return MS_HIP_OK;
}

}  // extern "C"

namespace {

// How one GroupQueryAttention call runs: the lane-group kernel for head_dim 32/64/128/256
// (with key splits when few units meet a long history and a workspace is given), else the
// per-unit kernel; and the LDS each needs.
struct GqaPlan {
    int G = 0;          // lanes per row of gqa_rows_kernel<G>, 0: gqa_attention_kernel
    bool grouped = false;   // gqa_group_kernel<D> (every query head of a kv group per workgroup)
    bool flash = false;     // gqa_flash_kernel<D> (prefill on the fp32 matrix cores)
    int splits = 1;
    size_t lds = 0;
    int64_t ws_bytes = 0;
};

constexpr size_t kGqaMaxLds = 160 * 1024;

GqaPlan gqa_plan(const ms_hip_gqa_desc& d, int64_t ws_avail)
{
    GqaPlan pl;
    const int D = d.head_dim;
    const int64_t total = (int64_t)d.past_seq + d.kv_seq;
    const int64_t units = (int64_t)d.batch * d.num_heads * d.q_seq;
    const int grp = d.kv_num_heads > 0 ? d.num_heads / d.kv_num_heads : 0;
    if ((D == 64 || D == 128) && grp >= 1 && grp <= kGqaGroupMax && d.q_seq >= 1 && d.q_seq <= 8) {
        // Decode and short queries: one workgroup per (batch, kv head, query, key split),
        // enough splits for about 512 workgroups (at most 64, at least 16 keys each). The
        // keys stream through LDS, so any history length fits; without a workspace for the
        // splits' partials, one split per group.
        pl.grouped = true;
        const int64_t groups = (int64_t)d.batch * d.kv_num_heads * d.q_seq;
        int splits = (int)std::min<int64_t>({(int64_t)kGqaMaxSplits, std::max<int64_t>(1, (512 + groups - 1) / groups),
                                             std::max<int64_t>(1, (total + 15) / 16)});
        int64_t ws = splits > 1 ? units * splits * (D + 2) * (int64_t)sizeof(float) : 0;
        if (ws_avail >= 0 && ws > ws_avail) {
            splits = 1;
            ws = 0;
        }
        pl.splits = splits;
        pl.ws_bytes = ws;
        return pl;
    }
    if ((D == 64 || D == 128) && d.q_seq > 8) {
        // Prefill: flash attention, K and V streaming through LDS (any history length).
        pl.flash = true;
        pl.lds = (size_t)2 * kFlashK * (D + 4) * sizeof(float);
        return pl;
    }
    if (D == 32 || D == 64 || D == 128 || D == 256) {
        pl.G = D / 4;
        const int64_t fixed = D + (int64_t)(kGqaThreads / pl.G) * D + 1;
        // Few units: split the keys so that each workgroup reads its rows in one pass of
        // 4 * 256 / G rows (its loads in flight together), up to 4096 workgroups.
        const int64_t pass = 4 * (int64_t)(kGqaThreads / pl.G);
        int splits = 1;
        if (units > 0 && units < 1024 && total > pass)
            splits = (int)std::min<int64_t>({(int64_t)kGqaMaxSplits, (total + pass - 1) / pass,
                                             std::max<int64_t>(1, 4096 / units)});
        // a split's scores must fit in LDS
        while (splits < kGqaMaxSplits && (fixed + (total + splits - 1) / splits) * 4 > (int64_t)kGqaMaxLds) ++splits;
        const int64_t ws = splits > 1 ? units * splits * (D + 2) * (int64_t)sizeof(float) : 0;
        if (ws_avail >= 0 && ws > ws_avail) splits = 1;   // no room: one split per unit
        pl.splits = splits;
        pl.ws_bytes = splits > 1 ? units * splits * (D + 2) * (int64_t)sizeof(float) : 0;
        pl.lds = (size_t)(fixed + (total + splits - 1) / splits) * sizeof(float);
    } else {
        pl.lds = ((size_t)D + std::max(kGqaThreads, D) + (size_t)total) * sizeof(float);
    }
    return pl;
}

}  // namespace

extern "C" {

int64_t ms_hip_gqa_workspace_size(const ms_hip_gqa_desc* d)
{
    return d ? gqa_plan(*d, -1).ws_bytes : 0;
}

int ms_hip_gqa_check(const ms_hip_gqa_desc* d)
{
    // Messages of GroupQueryAttentionKernel.cs:69-76, :104-107, :136-145, :163-171.
    if (!d) return fail(MS_HIP_ERR_INVALID, "[ms_hip] null GroupQueryAttention descriptor");
    if (d->num_heads <= 0 || d->kv_num_heads <= 0)
        return fail(MS_HIP_ERR_INVALID, "GroupQueryAttention requires positive 'num_heads' and 'kv_num_heads'.");
    if (d->num_heads % d->kv_num_heads != 0)
        return fail(MS_HIP_ERR_INVALID, "GroupQueryAttention num_heads=%d must be a multiple of kv_num_heads=%d.",
                    d->num_heads, d->kv_num_heads);
    if (d->batch < 0 || d->q_seq < 0 || d->kv_seq < 0 || d->head_dim <= 0 || d->past_seq < 0)
        return fail(MS_HIP_ERR_INVALID, "[ms_hip] GroupQueryAttention: negative sizes or head_dim <= 0");
    if (d->packed_qkv && d->kv_seq != d->q_seq)
        return fail(MS_HIP_ERR_INVALID, "[ms_hip] packed QKV: kv_seq must equal q_seq");
    const int64_t total = (int64_t)d->past_seq + d->kv_seq;
    if (d->present_capacity < total)
        return fail(MS_HIP_ERR_INVALID, "[ms_hip] present capacity %d is below past + new rows (%lld)",
                    d->present_capacity, (long long)total);
    if (d->do_rotary && (d->cos_rows <= 0 || d->cos_cols <= 0))
        return fail(MS_HIP_ERR_INVALID,
                    "GroupQueryAttention do_rotary=1 requires cos_cache (input 7) and sin_cache (input 8).");
    const int64_t lds = (int64_t)gqa_plan(*d, -1).lds;
    if (lds > (int64_t)kGqaMaxLds)
        return fail(MS_HIP_ERR_UNSUPPORTED,
                    "[ms_hip] GroupQueryAttention keeps a unit's scores in LDS: total sequence %lld with head_dim %d "
                    "exceeds 160 KiB",
                    (long long)total, d->head_dim);
    return MS_HIP_OK;
}

int ms_hip_gqa(const ms_hip_gqa_desc* d, const float* dQ, const float* dK, const float* dV, const float* dPastK,
               const float* dPastV, const int32_t* dSeqlensK, const float* dCos, const float* dSin, float* dOut,
               float* dPresentK, float* dPresentV, void* dWorkspace, int64_t workspace_bytes, void* stream)
{
    if (int st = gate()) return st;
    if (int st = ms_hip_gqa_check(d)) return st;
    const hipStream_t s = static_cast<hipStream_t>(stream);
    GqaArgs p;
    p.B = d->batch;
    p.Sq = d->q_seq;
    p.Skv = d->kv_seq;
    p.H = d->num_heads;
    p.kvH = d->kv_num_heads;
    p.D = d->head_dim;
    p.past = d->past_seq;
    p.cap = d->present_capacity;
    p.total = d->past_seq + d->kv_seq;
    const int qh = p.H * p.D, kvh = p.kvH * p.D;
    if (!dQ || !dOut || !dPresentK || !dPresentV || (!d->packed_qkv && (!dK || !dV)))
        return fail(MS_HIP_ERR_INVALID, "[ms_hip] GroupQueryAttention: null query, key, value, output or present");
    if (p.past > 0 && !d->past_in_present && (!dPastK || !dPastV))
        return fail(MS_HIP_ERR_INVALID, "GroupQueryAttention past_key provided without past_value.");
    if (d->seqlens_len > 0 && !dSeqlensK) return fail(MS_HIP_ERR_INVALID, "[ms_hip] seqlens_len > 0 with null seqlens_k");
    for (const void* q : {(const void*)dQ, (const void*)dK, (const void*)dV, (const void*)dPastK, (const void*)dPastV,
                          (const void*)dCos, (const void*)dSin, (const void*)dOut, (const void*)dSeqlensK})
        if (misaligned4(q)) return fail(MS_HIP_ERR_INVALID, "[ms_hip] GroupQueryAttention: buffers must be 4-byte aligned");
    if ((p.D & 3) == 0 && ((reinterpret_cast<uintptr_t>(dPresentK) & 15) || (reinterpret_cast<uintptr_t>(dPresentV) & 15)))
        return fail(MS_HIP_ERR_INVALID, "[ms_hip] GroupQueryAttention: present buffers must be 16-byte aligned");
    if (misaligned4(dPresentK) || misaligned4(dPresentV))
        return fail(MS_HIP_ERR_INVALID, "[ms_hip] GroupQueryAttention: buffers must be 4-byte aligned");
    if (d->packed_qkv) {
        p.q_stride = qh + 2 * kvh;
        p.kv_stride = p.q_stride;
        p.k = dQ + qh;
        p.v = dQ + qh + kvh;
    } else {
        p.q_stride = qh;
        p.kv_stride = kvh;
        p.k = dK;
        p.v = dV;
    }
    p.q = dQ;
    p.past_k = dPastK;
    p.past_v = dPastV;
    p.seqlens = dSeqlensK;
    p.seqlens_len = d->seqlens_len;
    p.cos = dCos;
    p.sin = dSin;
    p.out = dOut;
    p.pk = dPresentK;
    p.pv = dPresentV;
    p.do_rotary = d->do_rotary ? 1 : 0;
    p.interleaved = d->rotary_interleaved ? 1 : 0;
    p.half = d->cos_cols;
    p.rot_half = d->do_rotary ? std::min(2 * d->cos_cols, p.D) / 2 : 0;   // :333-336
    p.cache_rows = d->cos_rows;
    p.window = d->local_window_size;
    p.scale = d->scale != 0.0f ? d->scale : 1.0f / std::sqrt((float)p.D);   // :214-215
    if (p.B == 0 || (p.Sq == 0 && p.Skv == 0)) return MS_HIP_OK;
    if (p.past > 0 && !d->past_in_present) {
        const int64_t n = (int64_t)p.B * p.kvH * p.past * p.D;
        hipLaunchKernelGGL(gqa_copy_past_kernel, dim3(elementwise_grid(n)), dim3(256), 0, s, p);
        MS_HIP_CHECK(hipGetLastError());
    }
    const GqaPlan plan = p.Sq > 0 ? gqa_plan(*d, dWorkspace && !misaligned4(dWorkspace) ? workspace_bytes : 0) : GqaPlan{};
    if (p.Skv > 0 && !plan.grouped) {   // the grouped kernel writes the new rows itself
        const int threads = std::min(256, ((p.D + 63) / 64) * 64);
        hipLaunchKernelGGL(gqa_append_kernel, dim3((unsigned)(p.B * p.Skv * p.kvH)), dim3(threads), 0, s, p);
        MS_HIP_CHECK(hipGetLastError());
    }
    if (p.Sq > 0) {
        const GqaPlan& pl = plan;
        if (pl.flash) {
            const void* fn = p.D == 128 ? reinterpret_cast<const void*>(gqa_flash_kernel<128>)
                                        : reinterpret_cast<const void*>(gqa_flash_kernel<64>);
            if (pl.lds > 64 * 1024)
                MS_HIP_CHECK(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)pl.lds));
            const unsigned grid = (unsigned)(p.B * p.H * ((p.Sq + kFlashQ - 1) / kFlashQ));
            if (p.D == 128)
                hipLaunchKernelGGL(gqa_flash_kernel<128>, dim3(grid), dim3(256), pl.lds, s, p);
            else
                hipLaunchKernelGGL(gqa_flash_kernel<64>, dim3(grid), dim3(256), pl.lds, s, p);
            MS_HIP_CHECK(hipGetLastError());
            return MS_HIP_OK;
        }
        if (pl.grouped) {
            const unsigned grid = (unsigned)(p.B * p.kvH * p.Sq * pl.splits);
            float* ws = static_cast<float*>(dWorkspace);
            if (p.D == 128)
                hipLaunchKernelGGL(gqa_group_kernel<128>, dim3(grid), dim3(kGqaThreads), 0, s, p, ws, pl.splits);
            else
                hipLaunchKernelGGL(gqa_group_kernel<64>, dim3(grid), dim3(kGqaThreads), 0, s, p, ws, pl.splits);
            MS_HIP_CHECK(hipGetLastError());
            if (pl.splits > 1) {
                hipLaunchKernelGGL(gqa_merge_kernel, dim3((unsigned)(p.B * p.H * p.Sq * ((p.D + 63) / 64))), dim3(64), 0,
                                   s, p, ws, pl.splits);
                MS_HIP_CHECK(hipGetLastError());
            }
            return MS_HIP_OK;
        }
        if (pl.lds > kGqaMaxLds)
            return fail(MS_HIP_ERR_UNSUPPORTED, "[ms_hip] GroupQueryAttention: history too long for one workgroup's "
                                                "scores without a workspace (ms_hip_gqa_workspace_size)");
        const void* fn = reinterpret_cast<const void*>(gqa_attention_kernel);
        switch (pl.G) {
            case 8: fn = reinterpret_cast<const void*>(gqa_rows_kernel<8>); break;
            case 16: fn = reinterpret_cast<const void*>(gqa_rows_kernel<16>); break;
            case 32: fn = reinterpret_cast<const void*>(gqa_rows_kernel<32>); break;
            case 64: fn = reinterpret_cast<const void*>(gqa_rows_kernel<64>); break;
            default: break;
        }
        if (pl.lds > 64 * 1024)
            MS_HIP_CHECK(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)pl.lds));
        const unsigned units = (unsigned)(p.B * p.H * p.Sq);
        float* ws = static_cast<float*>(dWorkspace);
        switch (pl.G) {
            case 8: hipLaunchKernelGGL(gqa_rows_kernel<8>, dim3(units * pl.splits), dim3(kGqaThreads), pl.lds, s, p, ws,
                                       pl.splits); break;
            case 16: hipLaunchKernelGGL(gqa_rows_kernel<16>, dim3(units * pl.splits), dim3(kGqaThreads), pl.lds, s, p,
                                        ws, pl.splits); break;
            case 32: hipLaunchKernelGGL(gqa_rows_kernel<32>, dim3(units * pl.splits), dim3(kGqaThreads), pl.lds, s, p,
                                        ws, pl.splits); break;
            case 64: hipLaunchKernelGGL(gqa_rows_kernel<64>, dim3(units * pl.splits), dim3(kGqaThreads), pl.lds, s, p,
                                        ws, pl.splits); break;
            default: hipLaunchKernelGGL(gqa_attention_kernel, dim3(units), dim3(kGqaThreads), pl.lds, s, p); break;
        }
        MS_HIP_CHECK(hipGetLastError());
        if (pl.splits > 1) {
            hipLaunchKernelGGL(gqa_combine_kernel, dim3(units), dim3(std::min(256, ((p.D + 63) / 64) * 64)), 0, s, p,
                               ws, pl.splits);
            MS_HIP_CHECK(hipGetLastError());
        }
    }
    return MS_HIP_OK;
}

}  // extern "C"
