// pk_tagged.h — hand-over of values between workgroups of one launch.
//
// A value travels as a 64-bit word (tag << 32 | bits) written and read with
// relaxed agent-scope atomics: a word is single-copy atomic, so a reader that
// sees this launch's tag in a word sees the value that goes with it, and no
// fence (an L2 write-back or invalidate) is needed. The tag is a counter that
// the launch before advances (never 0: the buffers start zeroed).
// Polls are bounded: past the bound a wave sets status[0] and goes on, so
// that every wave ends; the host turns the flag into an error, or redoes the
// call with launches that do not wait. The bound is status[1] (0: the
// default below; a test sets a small one to force the give-up path).
#pragma once
#include "pk_internal.h"

constexpr uint32_t PK_POLL_BOUND = 1u << 18;

// The bound on polls of a launch: status[1], or PK_POLL_BOUND where it is 0.
__device__ __forceinline__ uint32_t pk_poll_bound(const uint32_t *status) {
    const uint32_t b = status[1];
    return b ? b : PK_POLL_BOUND;
}

// Polls the tagged word at p (lanes with use) until its tag is `tag` on
// every such lane of the wave; returns the low halves.
__device__ __forceinline__ uint32_t pk_wait_tagged(const uint64_t *p, bool use, uint32_t tag, uint32_t *status) {
    uint64_t w = use ? __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : (uint64_t)tag << 32;
    const uint32_t bound = pk_poll_bound(status);
    uint32_t n = 0;
    while (__any((uint32_t)(w >> 32) != tag)) {
        __builtin_amdgcn_s_sleep(1);
        if ((uint32_t)(w >> 32) != tag) w = __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (++n >= bound) {
            if ((threadIdx.x & 63) == 0) __hip_atomic_store(status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            break;
        }
    }
    return (uint32_t)w;
}

__device__ __forceinline__ void pk_put_tagged(uint64_t *p, uint32_t tag, uint32_t bits) {
    __hip_atomic_store(p, (uint64_t)tag << 32 | bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
