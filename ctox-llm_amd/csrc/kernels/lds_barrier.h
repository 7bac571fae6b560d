// Workgroup barrier that orders LDS accesses only. __syncthreads() also
// releases and acquires global memory at workgroup scope, which on gfx950
// waits for every outstanding global store of the wave (a memory round
// trip); kernels that exchange data only through LDS use this instead.
#pragma once
#include <hip/hip_runtime.h>

__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}
