// scmp_sc_gemm_noalloc: the SC GEMM for callers that cannot allocate device memory.
//
// The only device memory scmp_sc_gemm needs beyond its inputs and outputs is the FP4
// kernel's split-tile workspace: one int counter per output tile and two slots of exact
// fp32 partial sums per persistent workgroup (scmp_sc_gemm_workspace_bytes). This entry
// point takes that workspace from a file-scope device array instead of the caller, so it
// performs no allocation of any kind. Each device holds its own copy of the array (loaded
// with this translation unit's code object) until the process ends; its address on the
// current device is looked up once per device with hipGetSymbolAddress and cached. The
// array's name is never passed to a kernel: on the host it is only a handle for that
// lookup.
//
// The counters are cleared by a fill kernel on the caller's stream before every launch
// (no hipMemsetAsync, so the call may also be captured into a graph), and every partial-sum
// slot is written by its owner before any reader counts in, so nothing left in the array by
// an earlier call is ever read. Calls that overlap on one device (two streams, two host
// threads) share the array and race.
#include <mutex>

#include "common.h"

// the workspace of every call of scmp_sc_gemm_noalloc on this device
static __device__ __align__(256) uint8_t scratch[SCMP_SC_GEMM_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;

std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices] = {nullptr};

// Device address of `scratch` on the current device (hipGetSymbolAddress on first use).
int scratch_on_current_device(void **out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        scmp::set_error("scmp_sc_gemm_noalloc: no current device (%s)",
                        e != hipSuccess ? hipGetErrorString(e) : "device index out of range");
        return SCMP_E_LAUNCH;
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void *p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr) {
            scmp::set_error("scmp_sc_gemm_noalloc: hipGetSymbolAddress(scratch) on device %d "
                            "failed: %s", dev, hipGetErrorString(e));
            return SCMP_E_LAUNCH;
        }
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return SCMP_OK;
}

}  // namespace

extern "C" int scmp_sc_gemm_noalloc(const scmp_gemm_args *args, hipStream_t stream) {
    SCMP_REQUIRE(args != nullptr, "scmp_sc_gemm_noalloc: null args");
    SCMP_REQUIRE(args->workspace == nullptr && args->workspace_bytes == 0,
                 "scmp_sc_gemm_noalloc: workspace must be NULL with workspace_bytes 0 (the "
                 "library supplies it)");
    const int64_t need = scmp_sc_gemm_workspace_bytes(args);
    SCMP_REQUIRE(need <= SCMP_SC_GEMM_NOALLOC_SCRATCH_BYTES,
                 "scmp_sc_gemm_noalloc: this problem needs %lld bytes of workspace, more than "
                 "the %lld bytes of the library's static scratch; call scmp_sc_gemm with a "
                 "caller-allocated workspace instead",
                 (long long)need, (long long)SCMP_SC_GEMM_NOALLOC_SCRATCH_BYTES);
    scmp_gemm_args a = *args;
    if (need > 0) {
        void *p = nullptr;
        const int rc = scratch_on_current_device(&p);
        if (rc != SCMP_OK) return rc;
        a.workspace = p;
        a.workspace_bytes = SCMP_SC_GEMM_NOALLOC_SCRATCH_BYTES;
    }
    return scmp_sc_gemm(&a, stream);
}
