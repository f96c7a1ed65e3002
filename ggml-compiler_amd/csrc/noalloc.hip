// noalloc.hip - gcq_mul_mat_noalloc: ggml_mul_mat(W, x) of f32 rows for callers that cannot
// allocate device memory (code under HIP graph capture, serving loops, harnesses that forbid
// hipMalloc). The quantized activation, which gcq_mul_mat keeps in a caller-provided workspace,
// lives in `scratch`, a file-scope device array of GCQ_NOALLOC_SCRATCH_BYTES that every GPU the
// library runs on holds until the process ends.
//
// Host code never passes `scratch` itself to a kernel: on the host that name is a stand-in, not a
// device address. The first call on a device (with that device current) looks up the array's
// address on that device with hipGetSymbolAddress (in the thread's relaxed capture mode, so that a
// first call made while capturing a graph works) and keeps it per device; every launch takes that
// pointer. The kernels fully overwrite the part of the array a call uses before reading it, so
// nothing needs clearing between calls. Calls that overlap on one GPU (two streams, two threads)
// share the array and race.
#include "gcq_common.h"

#include <mutex>

#include "../../include/gcq.h"

namespace gcq {
namespace {

static __device__ __align__(256) uint8_t scratch[GCQ_NOALLOC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void * g_scratch_ptr[kMaxDevices] = {};

// The current device's address of `scratch`, looked up once per device.
void * device_scratch() {
    int dev = -1;
    check_hip(hipGetDevice(&dev), "hipGetDevice");
    require(dev >= 0 && dev < kMaxDevices, "device index " + std::to_string(dev) + " out of range");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        RelaxedCapture relaxed;  // the first call on a device may come under graph capture
        void * ptr = nullptr;
        check_hip(hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)), "hipGetSymbolAddress(scratch)");
        require(ptr != nullptr, "hipGetSymbolAddress(scratch) returned NULL");
        g_scratch_ptr[dev] = ptr;
    }
    return g_scratch_ptr[dev];
}

}  // namespace
}  // namespace gcq

using namespace gcq;

extern "C" int gcq_mul_mat_noalloc(int wtype, const void * w, int64_t N, int64_t K, const float * x, int64_t ldx,
                                   int64_t M, float * y, int64_t ldy, void * stream) {
    return guarded([&] {
        const size_t need = mul_mat_workspace_bytes(wtype, M, K);
        require(need <= (size_t) GCQ_NOALLOC_SCRATCH_BYTES,
                "mul_mat_noalloc: M = " + std::to_string(M) + ", K = " + std::to_string(K) + " needs " +
                    std::to_string(need) + " bytes of scratch, more than its " +
                    std::to_string((size_t) GCQ_NOALLOC_SCRATCH_BYTES) + " (use gcq_mul_mat with a workspace)");
        mul_mat_with_workspace(wtype, w, N, K, x, ldx, M, y, ldy, device_scratch(), (size_t) GCQ_NOALLOC_SCRATCH_BYTES,
                               as_stream(stream));
    });
}
