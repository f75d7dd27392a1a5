// rk_sync.h — a hand-off between the workgroups of one launch, for gfx950:
// producer workgroups store their part, waiting workgroups read it once all
// producers of the launch are done (the values-and-Wo launch).
#pragma once

#include "rk_dev.h"
#include "rk_fused.h"

namespace rk {

// A hand-off inside one launch, from the workgroups that produce an input
// to those that wait for all of it, through the
// words of `sync` (kSync*; zero when the owner is made, never reset).
// Launches of one stream run one after another, so a count that every
// producer (na of them) or every waiting workgroup (nw) of a launch adds
// one to tells the launch's number:
//  * a producer stores its part with agent-scope stores (to the level where
//    every XCD's loads of that scope look), waits until they are complete,
//    then adds one to kSyncDone; the producer whose add completes a
//    launch's count writes the launch's number into the flag words, one
//    128-byte line per XCD, so that the waiting workgroups of each XCD poll
//    their own line (measured: a hand-off in about 0.5 us where polls of
//    one shared word took about 6);
//  * a waiting workgroup adds one to kSyncArrive: the count before its add,
//    over nw, plus one is this launch's number. It polls its flag
//    (agent-scope loads) until the flag holds that number, then reads the
//    part with agent-scope loads.
// No fence is needed: the wait for the stores' completion orders them
// before the count. The poll is bounded by the device's real-time clock
// (kSyncTimeout); a workgroup that gives up sets the error word `err`,
// which the owner reads after the step.
__device__ __forceinline__ void sync_signal_done(unsigned long long *sync, int na) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's stores are complete
    if ((threadIdx.x & 63) == 0) {
        const unsigned long long old =
            __hip_atomic_fetch_add(sync + kSyncDone, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if ((old + 1) % (unsigned long long)na == 0) {
            const unsigned long long n = (old + 1) / (unsigned long long)na;
#pragma unroll
            for (int xcd = 0; xcd < 8; xcd++)
                __hip_atomic_store(sync + kSyncFlag + kSyncFlagStride * xcd, n, __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// The waiting side, by the whole workgroup: thread 0 registers and polls,
// then every wave passes a barrier (without a fence, so loads in flight are
// not waited for).
__device__ __forceinline__ void sync_wait_ready(unsigned long long *sync, int nw, unsigned long long *err) {
    if (threadIdx.x == 0) {
        const unsigned long long want =
            __hip_atomic_fetch_add(sync + kSyncArrive, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) /
                (unsigned long long)nw +
            1;
        const unsigned long long *f = sync + kSyncFlag + kSyncFlagStride * (blockIdx.x & 7);
        const unsigned long long t0 = __builtin_amdgcn_s_memrealtime();
        bool ok = false;
        for (int i = 0; i < (1 << 24); i++) {
            const unsigned long long v = __hip_atomic_load(f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if ((long long)(v - want) >= 0) {
                ok = true;
                break;
            }
            if (__builtin_amdgcn_s_memrealtime() - t0 > kSyncTimeout) break;
            __builtin_amdgcn_s_sleep(2);
        }
        if (!ok) __hip_atomic_store(err, 1ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    asm volatile("s_barrier" ::: "memory");
}

}  // namespace rk
