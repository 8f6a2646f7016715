// gdn_noalloc.hip -- gdn_recurrence_noalloc: the gated delta-rule steps of
// gdn_test_recurrence on caller-owned device buffers, with no allocation of
// any kind (for callers that cannot allocate: code under HIP graph capture,
// serving loops).
//
// The only memory beyond the caller's inputs and outputs is the per-(step,
// head) (beta, decay) pair the recurrence kernel reads.  It lives in the
// file-scope device array `scratch` below (kScratchPairs pairs, 128 KiB on
// every GPU the library runs on, held until the process ends).  Steps are
// processed in chunks that fit it: one kernel fills the chunk's pairs, then
// one recurrence launch per step reads them; stream order keeps the next
// chunk's fill behind the last step that reads the previous one.  Every call
// on a GPU shares that GPU's array, so calls that overlap on one GPU race.
//
// Host code never passes `scratch` itself to a kernel: its name is a
// host-side stand-in, not a device address.  The device address is looked up
// once per device with hipGetSymbolAddress and kept in g_scratch_ptr.
#include <hip/hip_runtime.h>

#include <cstdio>
#include <mutex>

#include "gdn_amd.h"
#include "gdn_device.h"
#include "gdn_internal.h"

namespace {

constexpr int kScratchPairs = 16384;  // (beta, decay) pairs
constexpr int kMaxDevices = 64;
constexpr int kCols = 16;              // state columns per recurrence workgroup

__device__ __align__(256) float2 scratch[kScratchPairs];

std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {};

// The device address of `scratch` on the current device, looked up on the
// first call there.
float2 *scratch_ptr() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        gdn_error("gdn_recurrence_noalloc: no current device");
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void *p = nullptr;
        const hipError_t rc = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (rc != hipSuccess || p == nullptr) {
            std::fprintf(stderr, "gdn_recurrence_noalloc: hipGetSymbolAddress failed: %s\n", hipGetErrorString(rc));
            return nullptr;
        }
        g_scratch_ptr[dev] = p;
    }
    return static_cast<float2 *>(g_scratch_ptr[dev]);
}

// (beta, decay) of n (step, head) pairs, from raw (a, b, a_log, dt_bias).
__global__ __launch_bounds__(gdn::kT) void k_scalars(const float *__restrict__ a, const float *__restrict__ b,
                                                     const float *__restrict__ a_log,
                                                     const float *__restrict__ dt_bias, int n,
                                                     float2 *__restrict__ out) {
    const int i = blockIdx.x * gdn::kT + threadIdx.x;
    if (i >= n) return;
    float beta, decay;
    gdn::head_scalars(a[i], b[i], a_log[i], dt_bias[i], beta, decay);
    out[i] = make_float2(beta, decay);
}

// One step of every head: grid (256 / kCols, heads).
template <int C>
__global__ __launch_bounds__(gdn::kT) void k_step(const float *__restrict__ q, const float *__restrict__ k,
                                                  const float *__restrict__ v, const float2 *__restrict__ bd,
                                                  void *__restrict__ S, float *__restrict__ o) {
    const gdn::ScalarsFromPairs scal{reinterpret_cast<const float *>(bd)};
    gdn::recur_block<C, kCols, false, false, false>(q, k, v, scal, nullptr, S, o, nullptr, blockIdx.y,
                                                     blockIdx.x * kCols);
}

}  // namespace

extern "C" int gdn_recurrence_noalloc(int contract, uint32_t n_heads, uint32_t n_steps, const float *q,
                                      const float *k, const float *v, const float *a, const float *b,
                                      const float *a_log, const float *dt_bias, void *S, float *o,
                                      void *stream) {
    if (contract < GDN_CONTRACT_REF || contract > GDN_CONTRACT_FP32) {
        std::fprintf(stderr, "gdn_recurrence_noalloc: unknown contract %d\n", contract);
        return -1;
    }
    if (n_heads == 0 || n_heads > (uint32_t)kScratchPairs) {
        std::fprintf(stderr, "gdn_recurrence_noalloc: %u heads; the scratch array holds one step of at most %d\n",
                     n_heads, kScratchPairs);
        return -1;
    }
    if (n_steps == 0) return 0;
    if (!q || !k || !v || !a || !b || !a_log || !dt_bias || !S || !o) {
        gdn_error("gdn_recurrence_noalloc: a buffer pointer is NULL");
        return -1;
    }
    float2 *bd = scratch_ptr();
    if (bd == nullptr) return -1;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const uint32_t chunk = (uint32_t)kScratchPairs / n_heads;  // steps per scratch fill
    const dim3 grid(gdn::kHD / kCols, n_heads), block(gdn::kT);
    for (uint32_t s0 = 0; s0 < n_steps; s0 += chunk) {
        const uint32_t ns = (n_steps - s0 < chunk) ? n_steps - s0 : chunk;
        const size_t first = (size_t)s0 * n_heads;
        const int n = (int)(ns * n_heads);
        hipLaunchKernelGGL(k_scalars, dim3((unsigned)((n + gdn::kT - 1) / gdn::kT)), dim3(gdn::kT), 0, s,
                           a + first, b + first, a_log + first, dt_bias + first, n, bd);
        for (uint32_t st = 0; st < ns; ++st) {
            const size_t ov = (size_t)(s0 + st) * n_heads * gdn::kHD;
            const float2 *bds = bd + (size_t)st * n_heads;
            if (contract == GDN_CONTRACT_REF)
                hipLaunchKernelGGL(k_step<gdn::kRef>, grid, block, 0, s, q + ov, k + ov, v + ov, bds, S, o + ov);
            else if (contract == GDN_CONTRACT_BF16W_FP32S)
                hipLaunchKernelGGL(k_step<gdn::kBf16w>, grid, block, 0, s, q + ov, k + ov, v + ov, bds, S, o + ov);
            else
                hipLaunchKernelGGL(k_step<gdn::kFp32>, grid, block, 0, s, q + ov, k + ov, v + ov, bds, S, o + ov);
        }
    }
    const hipError_t rc = hipGetLastError();
    if (rc != hipSuccess) {
        std::fprintf(stderr, "gdn_recurrence_noalloc: launch failed: %s\n", hipGetErrorString(rc));
        return -1;
    }
    return 0;
}
