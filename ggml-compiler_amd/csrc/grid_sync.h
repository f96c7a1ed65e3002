// grid_sync.h - a bounded grid barrier for launches whose workgroups are all resident at once
// (one workgroup per CU, grid = CU count), and the device-coherent word operations it uses.
//
// The eight XCDs' L2 caches are not coherent with each other inside a launch. The barrier words
// are read and written with agent-scope atomics (they reach the device-coherent level); data that
// one workgroup writes and another reads after the barrier must be stored device-coherently too
// (st_co / st_co_f, or buffer stores with the sc1 policy) and read at an address that no workgroup
// of the reader's XCD read earlier in the same launch, so that its L2 holds no older copy.
//
// Barrier words (unsigned, 64 apart = one 256-byte line each): [64 (1 + g)] arrivals of group g
// (workgroups b with b % 8 == g), [64 * 9] groups complete, [64 (10 + g)] release flag of group
// g, [64 * 18] workgroups that left the launch. Barrier k (1, 2, ... within a launch): each
// workgroup's stores complete, then one thread adds to its group's counter; the last of a group
// adds to the group counter, and the last group raises the 8 flags to k. A waiting workgroup polls
// its group's flag. Every wait gives up after a bounded spin and raises the error word (the host
// checks it: the launch's results are then invalid), so a barrier that cannot complete ends the
// kernel instead of hanging it. The last workgroup to leave (bar_leave) clears the words for the
// next launch.
#pragma once

#include "gcq_common.h"

namespace gcq {

constexpr int kBarWords = 64 * 19;
constexpr unsigned kSpinLimit = 1u << 22;  // polls before a wait gives up (about a second)

__device__ __forceinline__ unsigned ld_co(const unsigned * p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_co(unsigned * p, unsigned v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void st_co_f(float * p, float v) {
    __hip_atomic_store(reinterpret_cast<unsigned *>(p), __float_as_uint(v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ unsigned add_co(unsigned * p, unsigned v) {
    return __hip_atomic_fetch_add(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The thread that arrives and polls for its workgroup: lane 0 of the last wavefront.
__device__ __forceinline__ bool bar_thread() { return threadIdx.x == blockDim.x - 64; }

// First half of barrier k: every thread calls it after its stores of the phase.
__device__ __forceinline__ void bar_arrive(unsigned * bar, unsigned k, unsigned long long * stamp_at = nullptr) {
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_waitcnt(0);  // this wavefront's stores are complete
    __builtin_amdgcn_s_barrier();   // ... and every wavefront's
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    if (bar_thread()) {
        if (stamp_at) *stamp_at = __builtin_amdgcn_s_memrealtime();
        const unsigned n = gridDim.x, grp = blockIdx.x & 7u;
        const unsigned in_grp = (n - grp + 7u) / 8u;
        if (add_co(&bar[64 * (1 + grp)], 1u) == k * in_grp - 1u) {
            const unsigned groups = n < 8u ? n : 8u;
            if (add_co(&bar[64 * 9], 1u) == k * groups - 1u)
                for (unsigned g = 0; g < groups; g++) st_co(&bar[64 * (10 + g)], k);
        }
    }
}

// Second half: returns once every workgroup arrived (or the wait gave up and raised *err).
__device__ __forceinline__ void bar_wait(unsigned * bar, unsigned * err, unsigned k) {
    if (bar_thread()) {
        const unsigned grp = blockIdx.x & 7u;
        unsigned spins = 0;
        while (ld_co(&bar[64 * (10 + grp)]) < k) {
            __builtin_amdgcn_s_sleep(1);
            if (++spins > kSpinLimit || ld_co(err) != 0u) {
                st_co(err, 1u);
                break;
            }
        }
    }
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
    __builtin_amdgcn_s_barrier();
    __atomic_signal_fence(__ATOMIC_SEQ_CST);
}

// Called once by every workgroup after its last wait: the last one clears the words.
__device__ __forceinline__ void bar_leave(unsigned * bar) {
    if (threadIdx.x == 0 && add_co(&bar[64 * 18], 1u) == gridDim.x - 1u)
        for (int i = 0; i < kBarWords; i += 64) st_co(&bar[i], 0u);
}

}  // namespace gcq
