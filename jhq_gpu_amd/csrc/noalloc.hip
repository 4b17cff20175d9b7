// noalloc.hip — IVF assignment that allocates nothing (jhq_k_assign_noalloc).
//
// jhq_k_assign keeps one 64-bit key per row (ordered score << 32 | list) that
// the argmin GEMM lowers with atomicMin; it takes that buffer from
// hipMallocAsync.  Callers that cannot allocate (code under HIP graph capture,
// serving loops, harnesses that forbid hipMalloc) use this variant: the keys
// live in a file-scope device array of kAssignScratchRows entries, one copy
// per device, held until the process ends.  The array's device address is
// looked up once per device with hipGetSymbolAddress and only that address is
// handed to kernels.  Every call overwrites the keys it uses (a fill kernel
// sets them to ~0 first), so nothing carries over between calls.  Calls on
// one device share the array, so they are ordered on the device: each call's
// stream waits for the previous call's last kernel (an event per device,
// created on the first call; events hold no device memory).  Inside a HIP
// graph capture the call records no event wait (a capture may not wait on
// work outside it): replays of such graphs that overlap on one device, or
// with other calls, race on the array.
#include "../../include/jhq.h"
#include "kernels.h"

#include <hip/hip_runtime.h>

#include <mutex>
#include <string>

namespace {

constexpr int64_t kAssignScratchRows = int64_t(1) << 20;  // 8 MiB of keys
constexpr int kMaxDevices = 64;

}  // namespace

static __device__ __align__(256) unsigned long long scratch[kAssignScratchRows];

namespace {

// Per device: the address of its copy of `scratch`, and the event recorded
// after the last call's kernels.  The mutex also makes a call's wait and
// record one step, so two host threads cannot both wait on the same event.
struct DeviceScratch {
    unsigned long long* ptr = nullptr;
    hipEvent_t last = nullptr;
    bool recorded = false;
};
std::mutex g_scratch_mu;
DeviceScratch g_scratch[kMaxDevices];

// The current device's state, set up on the first call on that device
// (with that device current).  The caller holds g_scratch_mu.
hipError_t device_scratch(DeviceScratch** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    DeviceScratch& st = g_scratch[dev];
    if (!st.ptr) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        st.ptr = static_cast<unsigned long long*>(p);
    }
    if (!st.last) {
        e = hipEventCreateWithFlags(&st.last, hipEventDisableTiming);
        if (e != hipSuccess) {
            st.last = nullptr;
            return e;
        }
    }
    *out = &st;
    return hipSuccess;
}

}  // namespace

// Defined in jhq_capi.hip: sets the thread-local message jhq_last_error returns.
int jhq_set_error(int code, const char* msg);

extern "C" int jhq_k_assign_noalloc(const float* d_y, int64_t n, int d, const float* d_cent,
                                    const float* d_cent_norms, int nlist, int32_t* d_assign,
                                    void* stream) {
    if (!d_y || !d_cent || !d_cent_norms || !d_assign || n < 0 || d <= 0 || nlist <= 0)
        return jhq_set_error(JHQ_EINVAL, "bad argument");
    if (n > kAssignScratchRows)
        return jhq_set_error(JHQ_EINVAL, ("jhq_k_assign_noalloc takes at most " +
                                          std::to_string(kAssignScratchRows) +
                                          " rows per call (its key array's size)")
                                             .c_str());
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    DeviceScratch* st = nullptr;
    hipError_t e = device_scratch(&st);
    if (e != hipSuccess)
        return jhq_set_error(JHQ_EDEVICE, (std::string("scratch set-up (hipGetSymbolAddress, "
                                                       "hipEventCreate): ") +
                                           hipGetErrorString(e))
                                              .c_str());
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    e = hipStreamIsCapturing(s, &cap);
    if (e != hipSuccess)
        return jhq_set_error(JHQ_EDEVICE,
                             (std::string("hipStreamIsCapturing: ") + hipGetErrorString(e)).c_str());
    const bool order = cap == hipStreamCaptureStatusNone;
    unsigned long long* keys = st->ptr;
    // after the previous call's kernels on this device, whatever its stream
    if (order && st->recorded) e = hipStreamWaitEvent(s, st->last, 0);
    if (e == hipSuccess) e = jhq::fill_u64(keys, n, ~0ull, s);
    if (e == hipSuccess) e = jhq::gemm_nt_argmin(d_y, d, d_cent, d, n, nlist, d, d_cent_norms, keys, s);
    if (e == hipSuccess) e = jhq::keys_to_assign(keys, n, d_assign, s);
    if (e == hipSuccess && order) {
        e = hipEventRecord(st->last, s);
        if (e == hipSuccess) st->recorded = true;
    }
    if (e != hipSuccess)
        return jhq_set_error(JHQ_EDEVICE, (std::string("assign: ") + hipGetErrorString(e)).c_str());
    return JHQ_OK;
}
