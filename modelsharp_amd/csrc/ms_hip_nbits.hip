// ms_hip_nbits.hip — host runtime and C ABI of libms_hip_nbits.so (gfx950).
//
// Weights handles hold B, scales and packed zero points resident in HBM in the
// operator's own layout (uploaded once per initializer); each call dispatches
//   bits=4, block_size in {32,64,128,256}, K % 32 == 0 ("fast" layouts):
//     M <= 4, block_size 32 or 128, M*K/32 <= 1024              -> gemv_w4
//     M <= 16 otherwise                                         -> gemv_w4_panel
//     M >  16, block_size 32, K % 128 == 0, fp16-safe scales  -> a_to_f16 + mfma_w4_pipe
//     M >  16 otherwise                                         -> mfma_w4
//   anything else                                              -> generic
// Declarations and reference citations: include/ms_hip_kernels.h.
#include "../../include/ms_hip_kernels.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <array>
#include <atomic>
#include <cmath>
#include <utility>
#include <climits>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>

#include "gemv_w4.h"
#include "gemv_w4_panel.h"
#include "generic_nbits.h"
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

int require_device()
{
    const DeviceInfo& d = device_info();
    if (!d.ok) return fail(MS_HIP_ERR_NO_DEVICE, "[ms_hip] no gfx950 device is available");
    return MS_HIP_OK;
}

// ---- weights handle --------------------------------------------------------------------
struct Weights {
    int N = 0, K = 0, bits = 0, bs = 0, nb = 0, blob = 0, zrb = 0;
    int has_zp = 0;
    int64_t row_bytes = 0;
    int fast = 0;       // gemv_w4 / mfma_w4 eligible
    int log2cpb = 0;    // log2(bs / 32) when fast
    int device = 0;
    uint8_t* d_b = nullptr;
    float* d_scales = nullptr;
    uint8_t* d_zp = nullptr;
    // synchronous host-pointer path: staging buffers + stream, guarded by mu
    std::mutex mu;
    hipStream_t stream = nullptr;
    float* d_stage = nullptr;
    size_t stage_bytes = 0;
    // prefill pipeline: scales fp16-safe (checked at load), fp16 activation workspace
    int pipe_scales_ok = 0;
    std::mutex ws_mu;
    uint32_t* d_a16 = nullptr;
    size_t a16_bytes = 0;
    int* d_sync = nullptr;      // split-K arrival counters and flags, zero between launches
    float* d_part = nullptr;    // split-K partial sums, kPipeBM x kPipeBN floats per tile
    int sync_tiles = 0;         // tiles covered by d_sync and d_part
    float* d_rbpart = nullptr;  // mfma_w4_rb K-split partial sums [ksw][M][N]
    size_t rbpart_bytes = 0;
    // small-M matrix-core GEMV: K-split slots and counters
    uint8_t* d_sk = nullptr;    // skinny_w4 slots: [row tiles][workgroups per tile][16 x 128 floats]
    size_t sk_bytes = 0;
    int* d_sk_sync = nullptr;   // per row tile, zero between launches
    int sk_blocks = 0;
};

constexpr uint32_t kHandleMagic = 0x4D534E42u;   // "MSNB"
struct HandleBox {
    uint32_t magic = kHandleMagic;
    Weights w;
};

Weights* from_handle(void* h)
{
    HandleBox* box = static_cast<HandleBox*>(h);
    if (!box || box->magic != kHandleMagic) return nullptr;
    return &box->w;
}

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
    if (w.d_zp) (void)hipFree(w.d_zp);
    if (w.d_stage) (void)hipFree(w.d_stage);
    if (w.d_a16) (void)hipFree(w.d_a16);
    if (w.d_sync) (void)hipFree(w.d_sync);
    if (w.d_part) (void)hipFree(w.d_part);
    if (w.d_rbpart) (void)hipFree(w.d_rbpart);
    if (w.d_sk) (void)hipFree(w.d_sk);
    if (w.d_sk_sync) (void)hipFree(w.d_sk_sync);
    if (w.stream) (void)hipStreamDestroy(w.stream);
    w.d_b = nullptr;
    w.d_scales = nullptr;
    w.d_zp = nullptr;
    w.d_stage = nullptr;
    w.d_a16 = nullptr;
    w.a16_bytes = 0;
    w.d_sync = nullptr;
    w.d_part = nullptr;
    w.sync_tiles = 0;
    w.d_rbpart = nullptr;
    w.rbpart_bytes = 0;
    w.d_sk = nullptr;
    w.sk_bytes = 0;
    w.d_sk_sync = nullptr;
    w.sk_blocks = 0;
    w.stream = nullptr;
}

// Smallest nonzero and largest |scale| bit patterns (positive floats order as integers).
__global__ __launch_bounds__(256) void scale_range_kernel(const float* __restrict__ s, int64_t n, unsigned* out)
{
    unsigned lo = 0xFFFFFFFFu, hi = 0u;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
        const unsigned b = __builtin_bit_cast(unsigned, s[i]) & 0x7FFFFFFFu;
        if (b) {
            lo = min(lo, b);
            hi = max(hi, b);
        }
    }
    atomicMin(&out[0], lo);
    atomicMax(&out[1], hi);
}

// The pipelined prefill rounds scales to fp16 and forms (q - zp) * s in fp16: every
// nonzero |s| must be an fp16 normal (>= 2^-14) and 15 |s| must stay below 65504.
int check_pipe_scales(Weights& w)
{
    w.pipe_scales_ok = 0;
    if (!w.fast) return MS_HIP_OK;
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
    const unsigned kMaxScale = 0x45886000u;      // 4364.0: 15 * s < 65504
    w.pipe_scales_ok = (r[0] == 0xFFFFFFFFu) || (r[0] >= kMinNormal16 && r[1] <= kMaxScale);
    return MS_HIP_OK;
}

// ---- GEMV launch shape --------------------------------------------------------------------
// Tuning knobs (ms_hip_set_tuning); 0 = the shape heuristics below.
int g_panel_lanes_override = 0;  // knob 0: gemv_w4_panel lanes per row
int g_gemv_config = 0;           // knob 1: c+1 forces kGemvConfigs[c], -1 forces gemv_w4_panel
int g_pipe_off = 0;              // knob 2: 1 routes every prefill call to mfma_w4
int g_pipe_ksplit = 0;           // knob 3: 1 no prefill K split, 2 all tiles split, 3 the second half (where K allows)
int g_skinny = 0;                // knob 4: 1 keeps M <= 16 off skinny_w4, 2 sends every eligible M to it
int g_skinny_ksw = 0;            // knob 5: workgroups per skinny_w4 row block (0: heuristic)
int g_rb = 0;                    // knob 6: 1 keeps M > 16 off mfma_w4_rb, 2 sends every eligible M to it
int g_rb_ksw = 0;                // knob 7: mfma_w4_rb K split (0: heuristic)

// gemv_w4 instantiations: [M-1][L slot][config], L slot 0 = block size 32, 1 = block size 128.
typedef void (*GemvFn)(GemvParams);
template <int M, int L, size_t I>
constexpr GemvFn gemv_fn_at()
{
    constexpr GemvConfig c = kGemvConfigs[I];
    return gemv_w4_kernel<M, c.G, c.KW, c.U, L, c.waves, c.RL>;
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
// 8-wave configs. N is the launch's total
// rows (summed over a group). Indices are into kGemvConfigs; the streaming-read ceiling
// of the 7B gate+up launch's bytes (a plain row-pattern read, same rotation) is
// 14.5-15.1 us, against which its pick runs at about 20 us.
int pick_gemv_config(const Weights& w, int M, int N)
{
    if (g_gemv_config < 0) return -1;
    if (g_gemv_config > 0) {
        const int ci = g_gemv_config - 1;
        return gemv_config_fits(w, M, kGemvConfigs[ci]) ? ci : -1;
    }
    static constexpr int kLargeM2[] = {16, 11, 0, 6};   // M <= 2, N >= 16384
    static constexpr int kMidM2[] = {14, 11, 2};        // M <= 2, N >= 4096
    static constexpr int kSmallM2[] = {14, 13, 6, 8};   // M <= 2, N >= 2048
    static constexpr int kTinyM2[] = {3, 14, 8};        // M <= 2
    static constexpr int kLargeM4[] = {7, 6, 0};        // M <= 4, N >= 16384
    static constexpr int kMidM4[] = {15, 7, 8};         // M <= 4, N >= 4096
    static constexpr int kSmallM4[] = {6, 8, 0};        // M <= 4
    static constexpr int kWide[] = {9, 10};             // panels that need 16 waves to stage
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
        ci = N >= 16384 ? first_of(kLargeM2, 4) : N >= 4096 ? first_of(kMidM2, 3)
           : N >= 2048  ? first_of(kSmallM2, 4) : first_of(kTinyM2, 3);
    else
        ci = N >= 16384 ? first_of(kLargeM4, 3) : N >= 4096 ? first_of(kMidM4, 3) : first_of(kSmallM4, 3);
    if (ci < 0) ci = first_of(kWide, 2);
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

int launch_gemv_group(const GemvMember* mem, int n, const float* dA, int M, int ci, hipStream_t stream)
{
    const Weights& w0 = *mem[0].w;
    const GemvConfig& c = kGemvConfigs[ci];
    const int ls = l_slot(w0);
    GemvFn fn = kGemvTable[M - 1][ls][ci];
    const int rows = gemv_rows(c);
    const size_t lds = (size_t)M * (w0.K / 32) * kChunkStride4 * 16;
    if (lds > 64 * 1024 && !g_gemv_lds_raised[M - 1][ls][ci].load()) {
        MS_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds));
        g_gemv_lds_raised[M - 1][ls][ci].store(true);
    }
    GemvParams p;
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

// Members that one gemv_w4 launch can serve together: same device, 4-bit fast layout,
// K and block size (hence row_bytes, nb and zrb).
bool gemv_groupable(const Weights& a, const Weights& b)
{
    return a.device == b.device && a.fast && b.fast && a.bits == 4 && b.bits == 4 && a.K == b.K &&
           a.log2cpb == b.log2cpb && l_slot(a) >= 0;
}

// How many of the calls starting at handles[0] one launch serves: consecutive calls on
// the same activations (the projections of one input) that gemv_w4 can group, up to
// kGemvMaxOps; 1 when the first call launches alone. *ci receives the group's config.
bool skinny_eligible(const Weights& w, int M);
int skinny_ksw(const Weights& w);

int batch_group(void* const* handles, const float* const* dA, int count, int M, int* ci)
{
    const Weights* w = from_handle(handles[0]);
    if (M <= 0 || M > kGemvMaxM || !dA[0] || (reinterpret_cast<uintptr_t>(dA[0]) & 15)) return 1;
    if (skinny_eligible(*w, M)) return 1;   // the matrix-core small-M path launches per matrix
    int n = 1, ntot = w->N;
    while (n < count && n < kGemvMaxOps && dA[n] == dA[0] && gemv_groupable(*w, *from_handle(handles[n]))) {
        ntot += from_handle(handles[n])->N;
        ++n;
    }
    if (n == 1) return 1;
    *ci = pick_gemv_config(*w, M, ntot);
    return *ci >= 0 ? n : 1;
}

// ---- gemv_w4_panel: M <= 16, any fast block size, A staged in LDS panels ---------------
constexpr int kPanelMaxM = 16;
constexpr int kPanelLanes[3] = {16, 32, 64};

// Lanes per row G: lane efficiency on the row's C chunks x wave fill (>= 1024
// waves) x a penalty when a lane owns fewer than 3 chunks; ties go to the larger G.
int pick_panel_lanes(int N, int C)
{
    if (g_panel_lanes_override) return g_panel_lanes_override;
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

PanelFn panel_kernel(int M, int G)
{
    switch (M) {
        case 1: return panel_for_lanes<1>(G);
        case 2: return panel_for_lanes<2>(G);
        case 3: return panel_for_lanes<3>(G);
        case 4: return panel_for_lanes<4>(G);
        case 5: return panel_for_lanes<5>(G);
        case 6: return panel_for_lanes<6>(G);
        case 7: return panel_for_lanes<7>(G);
        case 8: return panel_for_lanes<8>(G);
        case 9: return panel_for_lanes<9>(G);
        case 10: return panel_for_lanes<10>(G);
        case 11: return panel_for_lanes<11>(G);
        case 12: return panel_for_lanes<12>(G);
        case 13: return panel_for_lanes<13>(G);
        case 14: return panel_for_lanes<14>(G);
        case 15: return panel_for_lanes<15>(G);
        default: return panel_for_lanes<16>(G);
    }
}

struct PanelShape {
    int G, grid, panel_chunks;
    size_t lds_bytes;
};

PanelShape panel_shape(const Weights& w, int M)
{
    PanelShape s;
    const int C = w.K / 32;
    s.G = pick_panel_lanes(w.N, C);
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

int launch_panel(const Weights& w, const float* dA, float* dY, int M, hipStream_t stream)
{
    const PanelShape s = panel_shape(w, M);
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
    hipLaunchKernelGGL(panel_kernel(M, s.G), dim3(s.grid), dim3(kPanelThreads), s.lds_bytes, stream, p);
    MS_HIP_CHECK(hipGetLastError());
    return MS_HIP_OK;
}

int launch_gemv(const Weights& w, const float* dA, float* dY, int M, hipStream_t stream)
{
    const int ci = pick_gemv_config(w, M, w.N);
    if (ci >= 0) {
        const GemvMember m{&w, dY};
        return launch_gemv_group(&m, 1, dA, M, ci, stream);
    }
    return launch_panel(w, dA, dY, M, stream);
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

// The pipelined prefill takes M > 16, block size 32, K a multiple of 128, fp16-safe
// scales, and buffers (Y included) below kPipeFar (its out-of-range offset).
bool pipe_eligible(const Weights& w, int M)
{
    return !g_pipe_off && w.fast && M > kPanelMaxM && w.log2cpb == 0 && (w.K % 128) == 0 && w.pipe_scales_ok &&
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
    int full, xu, xv;   // whole tiles [0, full); per-XCD whole and split work items
};
PipeSplit pipe_split(const Weights& w, int M)
{
    const int tiles = ((M + kPipeBM - 1) / kPipeBM) * ((w.N + kPipeBN - 1) / kPipeBN);
    int full = tiles;
    if (w.K / 128 >= 2) {
        if (g_pipe_ksplit == 2) {
            full = 0;
        } else if (g_pipe_ksplit == 3) {
            full = tiles / 2;
        } else if (g_pipe_ksplit == 0) {
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
    sp.full = full;
    sp.xu = (full + kXcds - 1) / kXcds;
    sp.xv = 2 * ((tiles - full + kXcds - 1) / kXcds);
    return sp;
}

// Returns 1 when the pipelined prefill was launched, 0 when the caller should use
// mfma_w4 (the workspace would have to grow while the stream is being captured),
// or a negative value on a launch error (last error set).
int launch_pipe(Weights& w, const float* dA, float* dY, int M, hipStream_t stream)
{
    const size_t need = (size_t)M * w.K * 2;
    const int tiles_m = (M + kPipeBM - 1) / kPipeBM, tiles_n = (w.N + kPipeBN - 1) / kPipeBN;
    const int tiles = tiles_m * tiles_n;
    const PipeSplit sp = pipe_split(w, M);
    uint32_t* ws = nullptr;
    int* sync = nullptr;
    float* part = nullptr;
    {
        std::lock_guard<std::mutex> lock(w.ws_mu);
        const bool grow_ws = w.a16_bytes < need, grow_sync = sp.full < tiles && w.sync_tiles < tiles;
        if (grow_ws || grow_sync) {
            hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
            if (hipStreamIsCapturing(stream, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) {
                (void)hipGetLastError();
                return 0;
            }
            if (hipStreamSynchronize(stream) != hipSuccess) return -1;
        }
        if (grow_ws) {
            if (w.d_a16 && hipFree(w.d_a16) != hipSuccess) return -1;
            w.d_a16 = nullptr;
            w.a16_bytes = 0;
            if (hipMalloc(&w.d_a16, need) != hipSuccess) return -1;
            w.a16_bytes = need;
        }
        if (grow_sync) {
            // The pairs are zeroed once here; every split launch leaves its pairs zero again.
            if (w.d_sync && hipFree(w.d_sync) != hipSuccess) return -1;
            if (w.d_part && hipFree(w.d_part) != hipSuccess) return -1;
            w.d_sync = nullptr;
            w.d_part = nullptr;
            w.sync_tiles = 0;
            if (hipMalloc(&w.d_sync, (size_t)tiles * 2 * sizeof(int)) != hipSuccess) return -1;
            // On the launch stream: a null-stream memset is not ordered before work on a
            // non-blocking stream. (Never reached under capture: checked above.)
            if (hipMemsetAsync(w.d_sync, 0, (size_t)tiles * 2 * sizeof(int), stream) != hipSuccess) return -1;
            if (hipMalloc(&w.d_part, (size_t)tiles * kPipeBM * kPipeBN * sizeof(float)) != hipSuccess) return -1;
            w.sync_tiles = tiles;
        }
        ws = w.d_a16;
        sync = w.d_sync;
        part = w.d_part;
    }
    static std::atomic<bool> lds_raised{false};
    if (!lds_raised.load()) {
        if (hipFuncSetAttribute(reinterpret_cast<const void*>(mfma_w4_pipe_kernel),
                                hipFuncAttributeMaxDynamicSharedMemorySize, kPipeLdsBytes) != hipSuccess)
            return -1;
        lds_raised.store(true);
    }
    const int64_t n8 = (int64_t)M * w.K / 8;
    hipLaunchKernelGGL(a_to_f16_kernel,
                       dim3((unsigned)std::min<int64_t>((n8 + 256 * kA16Groups - 1) / (256 * kA16Groups), 2048)),
                       dim3(256), 0, stream, dA, ws, n8);
    PipeParams p;
    p.b = w.d_b;
    p.scales = w.d_scales;
    p.zp = w.has_zp ? w.d_zp : nullptr;
    p.a16 = reinterpret_cast<const _Float16*>(ws);
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
    p.sync = sync;
    p.part = part;
    hipLaunchKernelGGL(mfma_w4_pipe_kernel, dim3(kXcds * (sp.xu + sp.xv)), dim3(256), kPipeLdsBytes, stream, p);
    return hipGetLastError() == hipSuccess ? 1 : -1;
}

// ---- skinny_w4: M <= 16 on the matrix cores at fp32-level accuracy (block size 128) ----

// The small-M matrix-core path takes block size 128 (a block is one group of four MFMA
// steps), K a multiple of 128, and 3 <= M <= 16: at M <= 2 gemv_w4 is faster (measured
// on the 7B MLP shapes: M=2 13.2 / 12.5 us against 15.4 / 16.7 us; M=3 20.4 / 24.2 us
// against 15.8 / 17.3 us), unless knob 4 says otherwise.
constexpr int kSkinnyMinM = 3;
bool skinny_eligible(const Weights& w, int M)
{
    if (g_skinny == 1 || !w.fast || w.log2cpb != 2 || (w.K % 128) != 0 || M < 1 || M > kSkinnyMT) return false;
    if ((int64_t)kSkinnyMT * w.K * 4 >= INT32_MAX) return false;
    return g_skinny == 2 || M >= kSkinnyMinM;
}

// Workgroups per row tile: each takes at most kSkinnyNB blocks and at least one; beyond
// that minimum, more only while the grid has fewer than two workgroups per CU (every
// extra split adds a slot to write and to sum).
int skinny_ksw(const Weights& w)
{
    const int tiles = (w.N + kSkinnyRows - 1) / kSkinnyRows;
    const int G = w.K / 128;
    const int kmin = (G + kSkinnyNB - 1) / kSkinnyNB;
    int ksw = kmin;
    if (g_skinny_ksw > 0) {
        ksw = g_skinny_ksw;
    } else {
        while (ksw < G && (int64_t)tiles * ksw < 2 * device_cus()) ++ksw;
    }
    return std::max(kmin, std::min(ksw, G));
}

// Returns 1 when launched, 0 when the caller should take gemv_w4 / gemv_w4_panel (the
// workspace would have to grow under capture), negative on a launch error.
int launch_skinny(Weights& w, const float* dA, float* dY, int M, hipStream_t stream)
{
    const int tiles = (w.N + kSkinnyRows - 1) / kSkinnyRows;
    const int ksw = skinny_ksw(w);
    const size_t need = ksw > 1 ? (size_t)tiles * ksw * kSkinnySlot * sizeof(float) : 0;
    uint8_t* ws = nullptr;
    int* sync = nullptr;
    if (ksw > 1) {
        std::lock_guard<std::mutex> lock(w.ws_mu);
        const bool grow = w.sk_bytes < need, grow_sync = w.sk_blocks < tiles;
        if (grow || grow_sync) {
            hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
            if (hipStreamIsCapturing(stream, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) {
                (void)hipGetLastError();
                return 0;
            }
            if (hipStreamSynchronize(stream) != hipSuccess) return -1;
        }
        if (grow) {
            if (w.d_sk && hipFree(w.d_sk) != hipSuccess) return -1;
            w.d_sk = nullptr;
            w.sk_bytes = 0;
            if (hipMalloc(&w.d_sk, need) != hipSuccess) return -1;
            w.sk_bytes = need;
        }
        if (grow_sync) {
            if (w.d_sk_sync && hipFree(w.d_sk_sync) != hipSuccess) return -1;
            w.d_sk_sync = nullptr;
            w.sk_blocks = 0;
            if (hipMalloc(&w.d_sk_sync, (size_t)tiles * sizeof(int)) != hipSuccess) return -1;
            // On the launch stream (never reached under capture: checked above).
            if (hipMemsetAsync(w.d_sk_sync, 0, (size_t)tiles * sizeof(int), stream) != hipSuccess) return -1;
            w.sk_blocks = tiles;
        }
        ws = w.d_sk;
        sync = w.d_sk_sync;
    }
    SkinnyParams p;
    p.b = w.d_b;
    p.scales = w.d_scales;
    p.zp = w.has_zp ? w.d_zp : nullptr;
    p.a = dA;
    p.y = dY;
    p.slots = reinterpret_cast<float*>(ws);
    p.sync = sync;
    p.row_bytes = (int)w.row_bytes;
    p.M = M;
    p.N = w.N;
    p.K = w.K;
    p.nb = w.nb;
    p.zrb = w.zrb;
    p.ksw = ksw;
    hipLaunchKernelGGL(skinny_w4_kernel, dim3(tiles * ksw), dim3(256), 0, stream, p);
    return hipGetLastError() == hipSuccess ? 1 : -1;
}

// ---- mfma_w4_rb: prefill with the weights dequantized into MFMA operand registers ----
// Any power-of-two block size >= 32, K a multiple of 128, fp16-safe scales (as the
// pipelined kernel: W = fl16((q - zp) * fl16(s))), every buffer below the out-of-range
// offset the kernel uses for padding rows.
bool rb_eligible(const Weights& w, int M)
{
    return g_rb != 1 && w.fast && M > kPanelMaxM && (w.K % 128) == 0 && w.pipe_scales_ok &&
           (int64_t)w.N * w.row_bytes < kOOB && (int64_t)M * w.K * 2 < kOOB && (int64_t)w.N * w.nb * 4 < kOOB &&
           (int64_t)M * w.N * 4 < kOOB;
}

// K split: the number of workgroups per 128 x 256 tile. A split runs in rounds of one
// workgroup per CU and pays a reduce pass over ksw + 1 copies of Y (written and read),
// so the pick minimises rounds x (blocks per workgroup) x t_block + reduce bytes / HBM
// rate, with t_block the measured time of one 128-k block of a workgroup (about 3.5 us:
// K=11008 unsplit at M=2048 takes 301 us for 86 blocks). On the 7B MLP shapes this
// picks the fastest measured split (M=128: 4 and 16; M=512, K=11008: 4).
int rb_ksw(const Weights& w, int M)
{
    const int G = w.K / 128;
    const int64_t tiles = (int64_t)((M + kRbBM - 1) / kRbBM) * ((w.N + kRbBN - 1) / kRbBN);
    if (g_rb_ksw > 0) return std::max(1, std::min(g_rb_ksw, G));
    const int cus = device_cus();
    const double t_block = 3.5e-6, hbm = 4.0e12, t_launch = 2e-6;
    const double ybytes = (double)M * w.N * 4;
    int pick = 1;
    double best = 1e30;
    for (int k = 1; k <= std::min(G, 32); ++k) {
        const double rounds = (double)((tiles * k + cus - 1) / cus);
        const double t = rounds * std::ceil((double)G / k) * t_block + (k > 1 ? (2.0 * k + 1) * ybytes / hbm + t_launch : 0.0);
        if (t < best * 0.97) {
            best = t;
            pick = k;
        }
    }
    return pick;
}

// Which prefill kernel: mfma_w4_rb where the pipelined kernel does not apply (block
// sizes other than 32), and where the pipelined launch would fill less than half of the
// CUs: measured on the 7B MLP shapes, 128 x 256 tiles with a wide K split beat it there
// (M=128: 49 / 45 us against 78 / 143 us; M=512, K=11008: 103 against 154 us), while
// with more tiles the pipelined kernel is faster (M=512, K=4096: 100 against 118 us;
// M=2048: 262 against 320-355 us).
bool use_rb(const Weights& w, int M)
{
    if (!rb_eligible(w, M)) return false;
    if (g_rb == 2 || !pipe_eligible(w, M)) return true;
    const int64_t tiles = (int64_t)((M + kPipeBM - 1) / kPipeBM) * ((w.N + kPipeBN - 1) / kPipeBN);
    const PipeSplit sp = pipe_split(w, M);
    const int64_t items = sp.full + 2 * (tiles - sp.full);
    return 2 * items < device_cus();
}

// Returns 1 when launched, 0 when the caller should take another kernel (the workspace
// would have to grow under capture), negative on a launch error.
int launch_rb(Weights& w, const float* dA, float* dY, int M, hipStream_t stream)
{
    const int tiles_m = (M + kRbBM - 1) / kRbBM, tiles_n = (w.N + kRbBN - 1) / kRbBN;
    const int ksw = rb_ksw(w, M);
    const size_t need_a = (size_t)M * w.K * 2;
    const int64_t slice = ((int64_t)M * w.N + 3) / 4 * 4;   // floats per K-split slice, 16-byte multiple
    const size_t need_p = ksw > 1 ? (size_t)ksw * slice * sizeof(float) : 0;
    uint32_t* ws = nullptr;
    float* part = nullptr;
    {
        std::lock_guard<std::mutex> lock(w.ws_mu);
        const bool grow_a = w.a16_bytes < need_a, grow_p = w.rbpart_bytes < need_p;
        if (grow_a || grow_p) {
            hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
            if (hipStreamIsCapturing(stream, &cs) != hipSuccess || cs != hipStreamCaptureStatusNone) {
                (void)hipGetLastError();
                return 0;
            }
            if (hipStreamSynchronize(stream) != hipSuccess) return -1;
        }
        if (grow_a) {
            if (w.d_a16 && hipFree(w.d_a16) != hipSuccess) return -1;
            w.d_a16 = nullptr;
            w.a16_bytes = 0;
            if (hipMalloc(&w.d_a16, need_a) != hipSuccess) return -1;
            w.a16_bytes = need_a;
        }
        if (grow_p) {
            if (w.d_rbpart && hipFree(w.d_rbpart) != hipSuccess) return -1;
            w.d_rbpart = nullptr;
            w.rbpart_bytes = 0;
            if (hipMalloc(&w.d_rbpart, need_p) != hipSuccess) return -1;
            w.rbpart_bytes = need_p;
        }
        ws = w.d_a16;
        part = w.d_rbpart;
    }
    const int64_t n8 = (int64_t)M * w.K / 8;
    hipLaunchKernelGGL(a_to_f16_kernel,
                       dim3((unsigned)std::min<int64_t>((n8 + 256 * kA16Groups - 1) / (256 * kA16Groups), 2048)),
                       dim3(256), 0, stream, dA, ws, n8);
    RbParams p;
    p.b = w.d_b;
    p.scales = w.d_scales;
    p.zp = w.has_zp ? w.d_zp : nullptr;
    p.a16 = reinterpret_cast<const _Float16*>(ws);
    p.out = ksw > 1 ? part : dY;
    p.slice = slice;
    p.row_bytes = (int)w.row_bytes;
    p.M = M;
    p.N = w.N;
    p.K = w.K;
    p.nb = w.nb;
    p.zrb = w.zrb;
    p.log2bs = w.log2cpb + 5;
    p.tiles_m = tiles_m;
    p.tiles_n = tiles_n;
    p.ksw = ksw;
    const int items = tiles_m * tiles_n * ksw;
    hipLaunchKernelGGL(mfma_w4_rb_kernel, dim3(((items + kXcds - 1) / kXcds) * kXcds), dim3(256), 0, stream, p);
    if (ksw > 1) {
        const int64_t slice4 = slice / 4;
        hipLaunchKernelGGL(rb_reduce_kernel, dim3((unsigned)std::min<int64_t>((slice4 + 255) / 256, 8192)), dim3(256),
                           0, stream, reinterpret_cast<const float4*>(part), dY, (int64_t)M * w.N, slice4, ksw);
    }
    return hipGetLastError() == hipSuccess ? 1 : -1;
}

int enqueue_gemm(Weights& w, const float* dA, float* dY, int M, hipStream_t stream)
{
    if (M < 0) return fail(MS_HIP_ERR_INVALID, "MatMulNBits M must be non-negative; got %d.", M);
    if (M == 0) return MS_HIP_OK;
    if (!dA || !dY) return fail(MS_HIP_ERR_INVALID, "[ms_hip] null activation or output pointer");
    if ((reinterpret_cast<uintptr_t>(dA) & 15) || (reinterpret_cast<uintptr_t>(dY) & 3))
        return fail(MS_HIP_ERR_INVALID, "[ms_hip] A must be 16-byte and Y 4-byte aligned");
    if (!w.fast) return launch_generic(w, dA, dY, M, stream);
    if (M <= kPanelMaxM) {
        if (skinny_eligible(w, M)) {
            const int r = launch_skinny(w, dA, dY, M, stream);
            if (r < 0) return fail(MS_HIP_ERR_HIP, "[ms_hip] small-M launch failed: %s", hipGetErrorString(hipGetLastError()));
            if (r > 0) return MS_HIP_OK;
        }
        return launch_gemv(w, dA, dY, M, stream);
    }
    if (use_rb(w, M)) {
        const int r = launch_rb(w, dA, dY, M, stream);
        if (r < 0) return fail(MS_HIP_ERR_HIP, "[ms_hip] prefill launch failed: %s", hipGetErrorString(hipGetLastError()));
        if (r > 0) return MS_HIP_OK;
    }
    if (pipe_eligible(w, M)) {
        const int r = launch_pipe(w, dA, dY, M, stream);
        if (r < 0) return fail(MS_HIP_ERR_HIP, "[ms_hip] prefill launch failed: %s", hipGetErrorString(hipGetLastError()));
        if (r > 0) return MS_HIP_OK;
    }
    return launch_mfma(w.d_b, w.d_scales, w.has_zp ? w.d_zp : nullptr, w.row_bytes, w.N, w.K, w.nb,
                       w.zrb, w.log2cpb, dA, dY, M, stream)
               ? fail(MS_HIP_ERR_HIP, "[ms_hip] MFMA launch failed: %s", hipGetErrorString(hipGetLastError()))
               : MS_HIP_OK;
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

int alloc_weights(Weights& w, int has_zp)
{
    w.has_zp = has_zp;
    MS_HIP_CHECK(hipMalloc(&w.d_b, (size_t)w.N * w.row_bytes));
    MS_HIP_CHECK(hipMalloc(&w.d_scales, (size_t)w.N * w.nb * sizeof(float)));
    if (has_zp) MS_HIP_CHECK(hipMalloc(&w.d_zp, (size_t)w.N * w.zrb));
    return MS_HIP_OK;
}

}  // namespace

// =========================================================================================
extern "C" {

int ms_hip_available(void) { return device_info().ok; }

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

int ms_hip_nbits_weights_create(const uint8_t* bq, int64_t bq_len, const float* scales, int64_t scales_len,
                                const uint8_t* zero_points, int64_t zp_len, int N, int K, int bits,
                                int block_size, void** out_handle)
{
    if (!out_handle) return fail(MS_HIP_ERR_INVALID, "[ms_hip] out_handle is null");
    *out_handle = nullptr;
    int st = check_impl(N, K, bits, block_size, bq_len, scales_len, zero_points ? 1 : 0, zp_len, -1);
    if (st) return st;
    if (!bq || !scales) return fail(MS_HIP_ERR_INVALID, "[ms_hip] null B or scales pointer");
    if ((st = require_device())) return st;
    MS_HIP_CHECK(hipSetDevice(device_info().device));
    HandleBox* box = new HandleBox();
    Weights& w = box->w;
    w.device = device_info().device;
    derive_layout(w, N, K, bits, block_size);
    st = alloc_weights(w, zero_points != nullptr);
    if (!st) {
        hipError_t e = hipMemcpy(w.d_b, bq, (size_t)N * w.row_bytes, hipMemcpyHostToDevice);
        if (e == hipSuccess)
            e = hipMemcpy(w.d_scales, scales, (size_t)N * w.nb * sizeof(float), hipMemcpyHostToDevice);
        if (e == hipSuccess && zero_points)
            e = hipMemcpy(w.d_zp, zero_points, (size_t)N * w.zrb, hipMemcpyHostToDevice);
        if (e != hipSuccess) st = fail(MS_HIP_ERR_HIP, "[ms_hip] weight upload failed: %s", hipGetErrorString(e));
        if (!st) st = check_pipe_scales(w);
    }
    if (st) {
        free_weights(w);
        delete box;
        return st;
    }
    *out_handle = box;
    return MS_HIP_OK;
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
    HandleBox* box = new HandleBox();
    Weights& w = box->w;
    w.device = device_info().device;
    derive_layout(w, N, K, bits, block_size);
    st = alloc_weights(w, d_zero_points != nullptr);
    if (!st) {
        hipError_t e = hipMemcpy(w.d_b, d_bq, (size_t)N * w.row_bytes, hipMemcpyDeviceToDevice);
        if (e == hipSuccess)
            e = hipMemcpy(w.d_scales, d_scales, (size_t)N * w.nb * sizeof(float), hipMemcpyDeviceToDevice);
        if (e == hipSuccess && d_zero_points)
            e = hipMemcpy(w.d_zp, d_zero_points, (size_t)N * w.zrb, hipMemcpyDeviceToDevice);
        if (e != hipSuccess) st = fail(MS_HIP_ERR_HIP, "[ms_hip] weight copy failed: %s", hipGetErrorString(e));
        if (!st) st = check_pipe_scales(w);
    }
    if (st) {
        free_weights(w);
        delete box;
        return st;
    }
    *out_handle = box;
    return MS_HIP_OK;
}

int ms_hip_nbits_weights_destroy(void* handle)
{
    Weights* w = from_handle(handle);
    if (!w) return fail(MS_HIP_ERR_INVALID, "[ms_hip] invalid weights handle");
    {
        std::lock_guard<std::mutex> lock(w->mu);
        if (w->stream) (void)hipStreamSynchronize(w->stream);
        free_weights(*w);
    }
    HandleBox* box = static_cast<HandleBox*>(handle);
    box->magic = 0;
    delete box;
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
    Weights* w = from_handle(handle);
    if (!w) return fail(MS_HIP_ERR_INVALID, "[ms_hip] invalid weights handle");
    return enqueue_gemm(*w, dA, dY, M, static_cast<hipStream_t>(stream));
}

int ms_hip_nbits_gemm_dev_batch(void* const* handles, const float* const* dA, float* const* dY, int count, int M,
                                void* stream)
{
    if (count < 0 || (count > 0 && (!handles || !dA || !dY)))
        return fail(MS_HIP_ERR_INVALID, "[ms_hip] invalid batch arguments");
    for (int i = 0; i < count; ++i)
        if (!from_handle(handles[i])) return fail(MS_HIP_ERR_INVALID, "[ms_hip] invalid weights handle at batch index %d", i);
    const hipStream_t s = static_cast<hipStream_t>(stream);
    for (int i = 0; i < count;) {
        int ci = -1;
        const int n = batch_group(handles + i, dA + i, count - i, M, &ci);
        if (n > 1) {
            GemvMember mem[kGemvMaxOps];
            for (int j = 0; j < n; ++j) {
                if (!dY[i + j] || (reinterpret_cast<uintptr_t>(dY[i + j]) & 3))
                    return fail(MS_HIP_ERR_INVALID, "[ms_hip] null or misaligned output at batch index %d", i + j);
                mem[j] = GemvMember{from_handle(handles[i + j]), dY[i + j]};
            }
            const int st = launch_gemv_group(mem, n, dA[i], M, ci, s);
            if (st) return st;
        } else {
            const int st = enqueue_gemm(*from_handle(handles[i]), dA[i], dY[i], M, s);
            if (st) return st;
        }
        i += n;
    }
    return MS_HIP_OK;
}

int ms_hip_nbits_batch_launch_info(void* const* handles, const float* const* dA, int count, int M, int* calls,
                                   int* kernel_id, int* lanes_per_row, int* grid, int* block)
{
    if (count <= 0 || !handles || !dA) return fail(MS_HIP_ERR_INVALID, "[ms_hip] invalid batch arguments");
    for (int i = 0; i < count; ++i)
        if (!from_handle(handles[i])) return fail(MS_HIP_ERR_INVALID, "[ms_hip] invalid weights handle at batch index %d", i);
    if (M <= 0) return fail(MS_HIP_ERR_INVALID, "[ms_hip] M must be positive; got %d", M);
    int ci = -1;
    const int n = batch_group(handles, dA, count, M, &ci);
    if (calls) *calls = n;
    if (n == 1) return ms_hip_nbits_launch_info(handles[0], M, kernel_id, lanes_per_row, grid, block);
    const GemvConfig& c = kGemvConfigs[ci];
    const int rows = gemv_rows(c);
    int gr = 0;
    for (int j = 0; j < n; ++j) gr += (from_handle(handles[j])->N + rows - 1) / rows;
    if (kernel_id) *kernel_id = 1;
    if (lanes_per_row) *lanes_per_row = c.G;
    if (grid) *grid = gr;
    if (block) *block = c.waves * kWave;
    return MS_HIP_OK;
}

int ms_hip_nbits_gemm(void* handle, const float* a_host, float* y_host, int M)
{
    Weights* w = from_handle(handle);
    if (!w) return fail(MS_HIP_ERR_INVALID, "[ms_hip] invalid weights handle");
    if (M < 0) return fail(MS_HIP_ERR_INVALID, "MatMulNBits M must be non-negative; got %d.", M);
    if (M == 0) return MS_HIP_OK;
    if (!a_host || !y_host) return fail(MS_HIP_ERR_INVALID, "[ms_hip] null activation or output pointer");
    std::lock_guard<std::mutex> lock(w->mu);
    MS_HIP_CHECK(hipSetDevice(w->device));
    if (!w->stream) MS_HIP_CHECK(hipStreamCreateWithFlags(&w->stream, hipStreamNonBlocking));
    const size_t a_bytes = (size_t)M * w->K * sizeof(float);
    const size_t a_span = (a_bytes + 255) & ~(size_t)255;
    const size_t y_bytes = (size_t)M * w->N * sizeof(float);
    if (w->stage_bytes < a_span + y_bytes) {
        if (w->d_stage) MS_HIP_CHECK(hipFree(w->d_stage));
        w->d_stage = nullptr;
        w->stage_bytes = 0;
        MS_HIP_CHECK(hipMalloc(&w->d_stage, a_span + y_bytes));
        w->stage_bytes = a_span + y_bytes;
    }
    float* dA = w->d_stage;
    float* dY = reinterpret_cast<float*>(reinterpret_cast<char*>(w->d_stage) + a_span);
    MS_HIP_CHECK(hipMemcpyAsync(dA, a_host, a_bytes, hipMemcpyHostToDevice, w->stream));
    const int st = enqueue_gemm(*w, dA, dY, M, w->stream);
    if (st) {
        (void)hipStreamSynchronize(w->stream);
        return st;
    }
    MS_HIP_CHECK(hipMemcpyAsync(y_host, dY, y_bytes, hipMemcpyDeviceToHost, w->stream));
    MS_HIP_CHECK(hipStreamSynchronize(w->stream));
    return MS_HIP_OK;
}

int ms_hip_qgemm_nbits(const float* a, const uint8_t* bq, const float* scales, const uint8_t* zero_points,
                       float* y, int M, int N, int K, int bits, int block_size)
{
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

int ms_hip_set_gemv_lanes(int lanes_per_row)
{
    if (lanes_per_row != 0 && lanes_per_row != 16 && lanes_per_row != 32 && lanes_per_row != 64)
        return fail(MS_HIP_ERR_INVALID, "[ms_hip] lanes_per_row must be 0, 16, 32 or 64; got %d", lanes_per_row);
    g_panel_lanes_override = lanes_per_row;
    return MS_HIP_OK;
}

int ms_hip_set_tuning(int knob, int value)
{
    switch (knob) {
        case 0: return ms_hip_set_gemv_lanes(value);
        case 1:
            if (value < -1 || value > kNumGemvConfigs) break;
            g_gemv_config = value;
            return MS_HIP_OK;
        case 2:
            if (value != 0 && value != 1) break;
            g_pipe_off = value;
            return MS_HIP_OK;
        case 3:
            if (value < 0 || value > 3) break;
            g_pipe_ksplit = value;
            return MS_HIP_OK;
        case 4:
            if (value < 0 || value > 2) break;
            g_skinny = value;
            return MS_HIP_OK;
        case 5:
            if (value < 0 || value > 64) break;
            g_skinny_ksw = value;
            return MS_HIP_OK;
        case 6:
            if (value < 0 || value > 2) break;
            g_rb = value;
            return MS_HIP_OK;
        case 7:
            if (value < 0 || value > 64) break;
            g_rb_ksw = value;
            return MS_HIP_OK;
        default: break;
    }
    return fail(MS_HIP_ERR_INVALID, "[ms_hip] invalid tuning knob %d = %d", knob, value);
}

int ms_hip_nbits_launch_info(void* handle, int M, int* kernel_id, int* lanes_per_row, int* grid, int* block)
{
    Weights* w = from_handle(handle);
    if (!w) return fail(MS_HIP_ERR_INVALID, "[ms_hip] invalid weights handle");
    if (M <= 0) return fail(MS_HIP_ERR_INVALID, "[ms_hip] M must be positive; got %d", M);
    int kid = 0, G = 0, gr = 0, bl = 0;
    if (!w->fast) {
        kid = 0;
        gr = (int)(((int64_t)M * w->N + 255) / 256);
        bl = 256;
    } else if (M <= kPanelMaxM && skinny_eligible(*w, M)) {
        kid = 5;
        gr = ((w->N + kSkinnyRows - 1) / kSkinnyRows) * skinny_ksw(*w);
        bl = 256;
    } else if (M <= kPanelMaxM) {
        const int ci = pick_gemv_config(*w, M, w->N);
        if (ci >= 0) {
            const GemvConfig& c = kGemvConfigs[ci];
            const int rows = gemv_rows(c);
            kid = 1;
            G = c.G;
            gr = (w->N + rows - 1) / rows;
            bl = c.waves * kWave;
        } else {
            const PanelShape s = panel_shape(*w, M);
            kid = 3;
            G = s.G;
            gr = s.grid;
            bl = kPanelThreads;
        }
    } else if (use_rb(*w, M)) {
        kid = 6;
        gr = ((M + kRbBM - 1) / kRbBM) * ((w->N + kRbBN - 1) / kRbBN) * rb_ksw(*w, M);
        gr = ((gr + kXcds - 1) / kXcds) * kXcds;
        bl = 256;
    } else if (pipe_eligible(*w, M)) {
        kid = 4;
        const PipeSplit sp = pipe_split(*w, M);
        gr = kXcds * (sp.xu + sp.xv);
        bl = 256;
    } else {
        kid = 2;
        mfma_launch_shape(w->N, M, &gr, &bl);
    }
    if (kernel_id) *kernel_id = kid;
    if (lanes_per_row) *lanes_per_row = G;
    if (grid) *grid = gr;
    if (block) *block = bl;
    return MS_HIP_OK;
}

}  // extern "C"
