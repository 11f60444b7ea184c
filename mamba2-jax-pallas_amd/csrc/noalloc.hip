// m2_ssd_combined_noalloc: the combined forward for callers that cannot
// allocate device memory (code under HIP graph capture, tight serving loops,
// harnesses that forbid hipMalloc).  It runs exactly the kernels of
// m2_ssd_combined, with the workspace (dA cumsum, dt', chunk-state weights,
// carry decay, states entering each chunk) taken from a file-scope device
// array instead of the caller's buffer.
//
// The array is M2_NOALLOC_SCRATCH_BYTES long and lives in this file's code
// object: every GPU the library runs this entry point on holds one copy until
// the process ends.  Host code never passes the array's name to a kernel (on
// the host it is only a stand-in symbol); its device address comes from
// hipGetSymbolAddress, looked up once per device, with that device current, on
// the first call there (or in m2_ssd_combined_noalloc_prepare), and kept per
// device.  The lookup may load the code object onto the device, which a stream
// under graph capture must not see: a first call on a capturing stream is
// refused, and callers that capture call the prepare function beforehand.
//
// Calls on one GPU share its array: two calls that overlap in time on one GPU
// (different streams, or the same stream from different threads without
// ordering) race on it.  Nothing in the workspace needs to start at zero
// (every slot is written before it is read), so a call does not clear it.
#include <mutex>

#include "m2_internal.h"

namespace {

static __device__ __align__(256) char scratch[M2_NOALLOC_SCRATCH_BYTES];

constexpr int MAX_DEVICES = 64;
std::mutex g_mu;
void* g_ptr[MAX_DEVICES];          // device address of `scratch` per device, or NULL

// The device address of `scratch` on the current device (looked up once; not
// while `capturing`).
int scratch_of_current_device(void** out, bool capturing) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess)
        return m2::set_error(M2_ERR_LAUNCH, "m2_ssd_combined_noalloc: hipGetDevice failed");
    if (dev < 0 || dev >= MAX_DEVICES)
        return m2::set_error(M2_ERR_UNSUPPORTED, "m2_ssd_combined_noalloc: device %d >= %d", dev,
                             MAX_DEVICES);
    std::lock_guard<std::mutex> lock(g_mu);
    if (!g_ptr[dev]) {
        if (capturing)
            return m2::set_error(M2_ERR_INVALID,
                                 "m2_ssd_combined_noalloc: first call on device %d is under stream "
                                 "capture; call m2_ssd_combined_noalloc_prepare() before capturing",
                                 dev);
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return m2::set_error(M2_ERR_LAUNCH, "m2_ssd_combined_noalloc: hipGetSymbolAddress: %s",
                                 hipGetErrorString(e));
        g_ptr[dev] = p;
    }
    *out = g_ptr[dev];
    return M2_OK;
}

}  // namespace

extern "C" int m2_ssd_combined_noalloc(const m2_ssd_combined_args* a, void* stream) {
    if (!a) return m2::set_error(M2_ERR_INVALID, "m2_ssd_combined_noalloc: NULL args");
    const size_t need = m2_ssd_combined_workspace_size(a);
    M2_REQUIRE(need != 0, M2_ERR_INVALID, "m2_ssd_combined_noalloc: bad chunk_size or dtype");
    M2_REQUIRE(need <= (size_t)M2_NOALLOC_SCRATCH_BYTES, M2_ERR_WORKSPACE,
               "m2_ssd_combined_noalloc: this problem needs a %zu-byte workspace, more than the "
               "%zu-byte static scratch; call m2_ssd_combined with a workspace instead",
               need, (size_t)M2_NOALLOC_SCRATCH_BYTES);
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing((hipStream_t)stream, &cap) != hipSuccess)
        return m2::set_error(M2_ERR_LAUNCH, "m2_ssd_combined_noalloc: hipStreamIsCapturing failed");
    void* ws = nullptr;
    int rc = scratch_of_current_device(&ws, cap != hipStreamCaptureStatusNone);
    if (rc) return rc;
    return m2::ssd_combined_on(*a, ws, (size_t)M2_NOALLOC_SCRATCH_BYTES, (hipStream_t)stream);
}

extern "C" int m2_ssd_combined_noalloc_prepare(void) {
    void* ws = nullptr;
    return scratch_of_current_device(&ws, false);
}
