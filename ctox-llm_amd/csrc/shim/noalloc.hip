// Static device scratch of the allocation-free entry point
// (ctox_hip_launch_fused_matvec_noalloc, include/ctox_hip.h).
//
// The tiled matvec's cross-chunk combine needs slots for the chunks'
// partial sums. ctox_hip_launch_fused_matvec takes them from a per-backend
// buffer it grows with hipMalloc; callers that cannot allocate (serving
// loops, harnesses that forbid it) use this file-scope
// array instead, one copy per GPU, held until the process ends. Its address
// on each device is taken once with hipGetSymbolAddress at backend creation
// (ctox_noalloc_setup, called with that device current) and only that
// address is used from the host afterwards. The slots are tagged with a
// per-device launch number (never 0); the array starts cleared, and is
// cleared again by a fill kernel when the number wraps. The launch number is
// a kernel argument, so a launch captured into a HIP graph would replay with
// the same tag and could read the previous replay's slots: the entry point
// is not meant for capture.
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>
#include <mutex>

#include "ctox_hip.h"

#define CTOX_NOALLOC_WORDS (CTOX_NOALLOC_SCRATCH_BYTES / 8)

static __device__ __align__(256) uint64_t scratch[CTOX_NOALLOC_WORDS];

namespace {

constexpr int kMaxDevices = 64;

struct DeviceScratch {
    std::once_flag once;
    hipError_t err = hipSuccess;
    uint64_t *ptr = nullptr;  // device address of `scratch` on this device
    uint32_t seq = 0;         // tag of the last launch
    std::mutex m;
};

DeviceScratch g_dev[kMaxDevices];

__global__ void ctox_noalloc_clear(uint64_t *p, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) p[i] = 0;
}

}  // namespace

// Called by ctox_hip_backend_create with `device` current: the array's
// address on this device, and a cleared array (once per device).
extern "C" ctox_status ctox_noalloc_setup(int device) {
    if (device < 0 || device >= kMaxDevices) return CTOX_ERR_UNSUPPORTED_OPERATION;
    DeviceScratch &d = g_dev[device];
    std::call_once(d.once, [&] {
        void *p = nullptr;
        d.err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (d.err != hipSuccess) return;
        d.ptr = (uint64_t *)p;
        ctox_noalloc_clear<<<256, 256, 0, nullptr>>>(d.ptr, CTOX_NOALLOC_WORDS);
        d.err = hipGetLastError();
        if (d.err == hipSuccess) d.err = hipDeviceSynchronize();
    });
    return d.err == hipSuccess && d.ptr ? CTOX_OK : CTOX_ERR_INVALID_STATE;
}

// The device's slots and the tag of the next launch, queued on `stream`
// (a wrap of the tag clears the array first, with a kernel).
// The last CTOX_NOALLOC_ARRIVE_BYTES of the array are the batch-1 kernel's
// per-tile arrival counts (zero between launches: each launch's last arrival
// resets its count, and a wrap clears the whole array); the rest are slots.
#define CTOX_NOALLOC_ARRIVE_BYTES (256u << 10)
extern "C" ctox_status ctox_noalloc_slots(int device, void *stream, uint64_t **ptr, size_t *bytes, uint32_t *seq,
                                          uint32_t **arrive, size_t *arrive_n) {
    if (device < 0 || device >= kMaxDevices) return CTOX_ERR_UNSUPPORTED_OPERATION;
    DeviceScratch &d = g_dev[device];
    std::lock_guard<std::mutex> lock(d.m);
    if (!d.ptr) return CTOX_ERR_INVALID_STATE;
    if (++d.seq == 0) {
        ctox_noalloc_clear<<<256, 256, 0, (hipStream_t)stream>>>(d.ptr, CTOX_NOALLOC_WORDS);
        if (hipGetLastError() != hipSuccess) return CTOX_ERR_INVALID_STATE;
        d.seq = 1;
    }
    *ptr = d.ptr;
    *bytes = CTOX_NOALLOC_SCRATCH_BYTES - CTOX_NOALLOC_ARRIVE_BYTES;
    *seq = d.seq;
    *arrive = (uint32_t *)((char *)d.ptr + *bytes);
    *arrive_n = CTOX_NOALLOC_ARRIVE_BYTES / 4;
    return CTOX_OK;
}
